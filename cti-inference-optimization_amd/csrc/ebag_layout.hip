// Device builders of the flat sparse-feature layout consumed by the pooling kernels.
//
//  * pack:  S per-slot (values, offsets) pairs -> flat_values, flat_row_offsets, val_offsets
//           (online_best/infer.py:960-974 on device; same result as the host builders at
//           online_best/infer.py:446-474 and :139-154), plus the global offsets form.
//  * merge: K flat-layout sub-batches -> one flat layout, concatenated field by field in
//           sub-batch order with offsets rebased (online_best/infer.py:581-631, :2977-3037).
// Both are integer copy kernels: coalesced int64 loads/stores, HBM-bound.
#include <stdint.h>
#include <string.h>

#include "ebag_device.h"
#include "ebag_internal.h"

namespace cti {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxSlots = 64;
constexpr int kMaxSub = 32;

struct PackParams {
  const int64_t* vals[kMaxSlots];
  const int64_t* offs[kMaxSlots];
  int64_t nnz[kMaxSlots];
  int64_t vbase[kMaxSlots];  // exclusive prefix of nnz over all slots
  int64_t* flat_values;
  int64_t* flat_row_offsets;
  int64_t* val_offsets;
  int64_t* global_offsets;
  int64_t batch;
  int64_t total;
  int32_t num_slots;  // slots in this launch
  int32_t slot0;      // index of vals[0] among all slots
  int32_t all_slots;  // S of the whole layout (for the closing global offset)
  int32_t pad;
};

__global__ void __launch_bounds__(kThreads) pack_kernel(const PackParams p) {
  const int si = static_cast<int>(blockIdx.y);
  const int s = p.slot0 + si;
  const int64_t n = p.nnz[si];
  const int64_t vb = p.vbase[si];
  const int64_t* __restrict__ src_v = p.vals[si];
  const int64_t* __restrict__ src_o = p.offs[si];
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  for (int64_t i = i0; i < n; i += stride) p.flat_values[vb + i] = src_v[i];
  const int64_t B = p.batch;
  for (int64_t i = i0; i <= B; i += stride) {
    const int64_t o = src_o[i];
    p.flat_row_offsets[static_cast<int64_t>(s) * (B + 1) + i] = o;
    if (p.global_offsets && i < B) p.global_offsets[static_cast<int64_t>(s) * B + i] = vb + o;
  }
  if (i0 == 0) {
    p.val_offsets[s] = vb;
    if (p.global_offsets && s == p.all_slots - 1) p.global_offsets[static_cast<int64_t>(p.all_slots) * B] = p.total;
  }
}

struct MergeParams {
  const int64_t* vals[kMaxSub];
  const int64_t* vo[kMaxSub];
  const int64_t* ro[kMaxSub];
  int64_t bsub[kMaxSub];
  int64_t bbase[kMaxSub];
  int64_t nnz[kMaxSub];
  int64_t* flat_values;
  int64_t* flat_row_offsets;
  int64_t* val_offsets;
  int64_t* global_offsets;
  int64_t batch;
  int32_t num_sub;
  int32_t num_slots;
};

__device__ __forceinline__ int64_t slot_nnz(const MergeParams& p, int s, int k) {
  const int64_t a = p.vo[k][s];
  const int64_t e = s + 1 < p.num_slots ? p.vo[k][s + 1] : p.nnz[k];
  return e - a;
}

// grid: (chunks, num_slots * num_sub); block (x, s*K + k) copies slot s of sub-batch k.
__global__ void __launch_bounds__(kThreads) merge_kernel(const MergeParams p) {
  __shared__ int64_t s_red[3][kThreads];
  const int K = p.num_sub;
  const int s = static_cast<int>(blockIdx.y) / K;
  const int k = static_cast<int>(blockIdx.y) % K;
  const int t = static_cast<int>(threadIdx.x);

  // before: values of slots < s (all sub-batches); vb: slot s of sub-batches < k; tot: slot s.
  int64_t before = 0, vb = 0, tot = 0;
  const int pairs = (s + 1) * K;
  for (int i = t; i < pairs; i += kThreads) {
    const int ss = i / K, kk = i % K;
    const int64_t c = slot_nnz(p, ss, kk);
    if (ss < s) before += c;
    else {
      tot += c;
      if (kk < k) vb += c;
    }
  }
  s_red[0][t] = before;
  s_red[1][t] = vb;
  s_red[2][t] = tot;
  __syncthreads();
  for (int w = kThreads / 2; w > 0; w >>= 1) {
    if (t < w) {
      s_red[0][t] += s_red[0][t + w];
      s_red[1][t] += s_red[1][t + w];
      s_red[2][t] += s_red[2][t + w];
    }
    __syncthreads();
  }
  before = s_red[0][0];
  vb = s_red[1][0];
  tot = s_red[2][0];

  const int64_t B = p.batch;
  const int64_t Bk = p.bsub[k];
  const int64_t n = slot_nnz(p, s, k);
  const int64_t src0 = p.vo[k][s];
  const int64_t dst0 = before + vb;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * kThreads + t;
  const int64_t* __restrict__ sv = p.vals[k];
  const int64_t* __restrict__ so = p.ro[k] + static_cast<int64_t>(s) * (Bk + 1);
  for (int64_t i = i0; i < n; i += stride) p.flat_values[dst0 + i] = sv[src0 + i];
  int64_t* ro_out = p.flat_row_offsets + static_cast<int64_t>(s) * (B + 1) + p.bbase[k];
  int64_t* g_out = p.global_offsets ? p.global_offsets + static_cast<int64_t>(s) * B + p.bbase[k] : nullptr;
  for (int64_t i = i0; i < Bk; i += stride) {
    const int64_t o = so[i] + vb;
    ro_out[i] = o;
    if (g_out) g_out[i] = before + o;
  }
  if (i0 == 0) {
    if (k == K - 1) p.flat_row_offsets[static_cast<int64_t>(s) * (B + 1) + B] = tot;
    if (k == 0) p.val_offsets[s] = before;
    if (g_out && k == 0 && s == p.num_slots - 1)
      p.global_offsets[static_cast<int64_t>(p.num_slots) * B] = before + tot;
  }
}

int64_t chunks_for(int64_t n, int64_t cap) {
  int64_t c = (n + kThreads * 4 - 1) / (kThreads * 4);
  if (c < 1) c = 1;
  return c > cap ? cap : c;
}

}  // namespace
}  // namespace cti

using namespace cti;

extern "C" int cti_ebag_pack_slots(const int64_t* const* slot_values, const int64_t* const* slot_offsets,
                                   const int64_t* slot_nnz, int32_t num_slots, int64_t batch_size,
                                   int64_t* flat_values, int64_t* flat_row_offsets, int64_t* val_offsets,
                                   int64_t* global_offsets, void* stream) {
  clear_error();
  if (num_slots < 0) return set_error(CTI_EBAG_EINVAL, "num_slots must be >= 0 (got %d)", num_slots);
  if (batch_size < 0) return set_error(CTI_EBAG_EINVAL, "batch_size must be >= 0 (got %lld)", (long long)batch_size);
  if (num_slots == 0) return CTI_EBAG_OK;
  if (!slot_values || !slot_offsets || !slot_nnz) return set_error(CTI_EBAG_EINVAL, "NULL host array argument");
  if (!flat_row_offsets || !val_offsets) return set_error(CTI_EBAG_EINVAL, "NULL output pointer");
  int64_t total = 0;
  for (int s = 0; s < num_slots; ++s) {
    if (slot_nnz[s] < 0) return set_error(CTI_EBAG_EINVAL, "slot %d: nnz must be >= 0", s);
    if (!slot_offsets[s]) return set_error(CTI_EBAG_EINVAL, "slot %d: offsets pointer is NULL", s);
    if (slot_nnz[s] > 0 && !slot_values[s]) return set_error(CTI_EBAG_EINVAL, "slot %d: values pointer is NULL", s);
    total += slot_nnz[s];
  }
  if (total > 0 && !flat_values) return set_error(CTI_EBAG_EINVAL, "flat_values is NULL");
  int64_t running = 0;
  for (int s0 = 0; s0 < num_slots; s0 += kMaxSlots) {
    const int ns = num_slots - s0 < kMaxSlots ? num_slots - s0 : kMaxSlots;
    PackParams p;
    memset(&p, 0, sizeof(p));
    int64_t longest = batch_size + 1;
    for (int i = 0; i < ns; ++i) {
      p.vals[i] = slot_values[s0 + i];
      p.offs[i] = slot_offsets[s0 + i];
      p.nnz[i] = slot_nnz[s0 + i];
      p.vbase[i] = running;
      running += slot_nnz[s0 + i];
      if (slot_nnz[s0 + i] > longest) longest = slot_nnz[s0 + i];
    }
    p.flat_values = flat_values;
    p.flat_row_offsets = flat_row_offsets;
    p.val_offsets = val_offsets;
    p.global_offsets = global_offsets;
    p.batch = batch_size;
    p.total = total;
    p.num_slots = ns;
    p.slot0 = s0;
    p.all_slots = num_slots;
    const dim3 grid(static_cast<unsigned>(chunks_for(longest, 1024)), static_cast<unsigned>(ns));
    hipLaunchKernelGGL(pack_kernel, grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream), p);
    const int rc = check_launch("cti_ebag_pack_slots");
    if (rc != CTI_EBAG_OK) return rc;
  }
  return CTI_EBAG_OK;
}

extern "C" int cti_ebag_merge_batches(const int64_t* const* sub_values, const int64_t* const* sub_val_offsets,
                                      const int64_t* const* sub_row_offsets, const int64_t* sub_batch,
                                      const int64_t* sub_nnz, int32_t num_sub, int32_t num_slots,
                                      int64_t* flat_values, int64_t* flat_row_offsets, int64_t* val_offsets,
                                      int64_t* global_offsets, void* stream) {
  clear_error();
  if (num_sub < 0 || num_slots < 0) return set_error(CTI_EBAG_EINVAL, "num_sub and num_slots must be >= 0");
  if (num_sub == 0 || num_slots == 0) return CTI_EBAG_OK;
  if (num_sub > kMaxSub) return set_error(CTI_EBAG_EUNSUPPORTED, "at most %d sub-batches per merge (got %d)", kMaxSub, num_sub);
  if (static_cast<int64_t>(num_slots) * num_sub > 65535)
    return set_error(CTI_EBAG_EUNSUPPORTED, "num_slots * num_sub must be <= 65535 (got %d * %d)", num_slots, num_sub);
  if (!sub_values || !sub_val_offsets || !sub_row_offsets || !sub_batch || !sub_nnz)
    return set_error(CTI_EBAG_EINVAL, "NULL host array argument");
  if (!flat_row_offsets || !val_offsets) return set_error(CTI_EBAG_EINVAL, "NULL output pointer");
  MergeParams p;
  memset(&p, 0, sizeof(p));
  int64_t B = 0, total = 0, longest = 1;
  for (int k = 0; k < num_sub; ++k) {
    if (sub_batch[k] < 0 || sub_nnz[k] < 0) return set_error(CTI_EBAG_EINVAL, "sub-batch %d: negative size", k);
    if (!sub_val_offsets[k] || !sub_row_offsets[k] || (sub_nnz[k] > 0 && !sub_values[k]))
      return set_error(CTI_EBAG_EINVAL, "sub-batch %d: NULL device pointer", k);
    p.vals[k] = sub_values[k];
    p.vo[k] = sub_val_offsets[k];
    p.ro[k] = sub_row_offsets[k];
    p.bsub[k] = sub_batch[k];
    p.bbase[k] = B;
    p.nnz[k] = sub_nnz[k];
    B += sub_batch[k];
    total += sub_nnz[k];
    if (sub_nnz[k] > longest) longest = sub_nnz[k];
    if (sub_batch[k] > longest) longest = sub_batch[k];
  }
  if (total > 0 && !flat_values) return set_error(CTI_EBAG_EINVAL, "flat_values is NULL");
  p.flat_values = flat_values;
  p.flat_row_offsets = flat_row_offsets;
  p.val_offsets = val_offsets;
  p.global_offsets = global_offsets;
  p.batch = B;
  p.num_sub = num_sub;
  p.num_slots = num_slots;
  const int64_t per_slot = (longest + num_slots - 1) / num_slots;
  const dim3 grid(static_cast<unsigned>(chunks_for(per_slot, 256)), static_cast<unsigned>(num_slots * num_sub));
  hipLaunchKernelGGL(merge_kernel, grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream), p);
  return check_launch("cti_ebag_merge_batches");
}
