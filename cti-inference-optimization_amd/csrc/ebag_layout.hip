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

// Two int64 moved as one 16-byte access (the arrays are 8-byte aligned; the hardware takes
// multi-dword accesses at dword alignment).
struct __attribute__((aligned(8))) I64Pair {
  int64_t a, b;
};

// x, or with `wrap` the int64 value of its low 32 bits read as int32 (torch's .int().long()).
__device__ __forceinline__ int64_t wrap32(int64_t x, bool wrap) {
  return wrap ? static_cast<int64_t>(static_cast<int32_t>(static_cast<uint32_t>(static_cast<uint64_t>(x)))) : x;
}

// Elements e and e + 1 of src[0, n) (e < n; the second is 0 past the end), and their store as
// dst[i] = post + wrap32(src[i] + add).
__device__ __forceinline__ I64Pair load_pair(const int64_t* __restrict__ src, int64_t e, int64_t n) {
  I64Pair v;
  if (e + 1 < n) {
    __builtin_memcpy(&v, src + e, sizeof(v));
  } else {
    v.a = src[e];
    v.b = 0;
  }
  return v;
}
__device__ __forceinline__ void store_pair(int64_t* __restrict__ dst, int64_t e, int64_t n, I64Pair v, int64_t add,
                                           bool wrap, int64_t post) {
  v.a = post + wrap32(v.a + add, wrap);
  v.b = post + wrap32(v.b + add, wrap);
  if (e + 1 < n) __builtin_memcpy(dst + e, &v, sizeof(v));
  else dst[e] = v.a;
}

// dst[i] = post + wrap32(src[i] + add) for i < n; grid-stride item j covers elements 2j and 2j+1.
__device__ __forceinline__ void copy_add_i64(const int64_t* __restrict__ src, int64_t* __restrict__ dst, int64_t n,
                                             int64_t add, int64_t j0, int64_t stride, bool wrap = false,
                                             int64_t post = 0) {
  for (int64_t j = j0; 2 * j < n; j += stride) {
    const int64_t e = 2 * j;
    if (e + 1 < n) {
      I64Pair v;
      __builtin_memcpy(&v, src + e, sizeof(v));
      v.a = post + wrap32(v.a + add, wrap);
      v.b = post + wrap32(v.b + add, wrap);
      __builtin_memcpy(dst + e, &v, sizeof(v));
    } else {
      dst[e] = post + wrap32(src[e] + add, wrap);
    }
  }
}

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
  copy_add_i64(src_v, p.flat_values + vb, n, 0, i0, stride);
  const int64_t B = p.batch;
  copy_add_i64(src_o, p.flat_row_offsets + static_cast<int64_t>(s) * (B + 1), B + 1, 0, i0, stride);
  if (p.global_offsets) copy_add_i64(src_o, p.global_offsets + static_cast<int64_t>(s) * B, B, vb, i0, stride);
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
  int32_t wrap32;  // the pair merge's int32 round trip of values and row offsets
};

// Slot s of sub-batch k: values [slot_start, slot_start + slot_nnz), its val_offsets entries
// clamped to [0, nnz] (a malformed entry yields an empty or shortened slot, never a read outside
// the sub-batch's values).
__device__ __forceinline__ int64_t slot_start(const MergeParams& p, int s, int k) {
  return clamp_i64(p.vo[k][s], 0, p.nnz[k]);
}
__device__ __forceinline__ int64_t slot_nnz(const MergeParams& p, int s, int k) {
  const int64_t a = slot_start(p, s, k);
  const int64_t e = s + 1 < p.num_slots ? clamp_i64(p.vo[k][s + 1], a, p.nnz[k]) : p.nnz[k];
  return e - a;
}

// grid: (chunks, num_slots * num_sub); block (x, s*K + k) copies slot s of sub-batch k.
__global__ void __launch_bounds__(kThreads) merge_kernel(const MergeParams p) {
  __shared__ int64_t s_red[3][kThreads / kWave];
  const int K = p.num_sub;
  const int s = static_cast<int>(blockIdx.y) / K;
  const int k = static_cast<int>(blockIdx.y) % K;
  const int t = static_cast<int>(threadIdx.x);
  // The grid is sized for the largest slot; a workgroup past this slot's values and offsets
  // (two per thread per grid-stride item) has nothing to copy. Workgroup 0 always stays: it
  // writes the slot's closing entries.
  const int64_t n_here = slot_nnz(p, s, k);
  const int64_t work = n_here > p.bsub[k] ? n_here : p.bsub[k];
  if (blockIdx.x > 0 && static_cast<int64_t>(blockIdx.x) * kThreads * 2 >= work) return;

  // This thread's first pair of values and of row offsets is read before the slot's destination
  // (which needs the sizes of all earlier slots) is summed, so the two latencies overlap.
  const int64_t Bk = p.bsub[k];
  const int64_t n = n_here;
  const int64_t src0 = slot_start(p, s, k);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * kThreads + t;
  const int64_t e0 = 2 * i0;
  const int64_t* __restrict__ so = p.ro[k] + static_cast<int64_t>(s) * (Bk + 1);
  I64Pair v0 = {0, 0}, o0 = {0, 0};
  if (e0 < n) v0 = load_pair(p.vals[k] + src0, e0, n);
  if (e0 < Bk) o0 = load_pair(so, e0, Bk);

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
  // wavefront sums (xor butterfly), then the wavefronts' sums through LDS (one barrier)
  const int lane = lane_id();
#pragma unroll
  for (int m = kWave / 2; m > 0; m >>= 1) {
    before += shfl_i64(before, lane ^ m);
    vb += shfl_i64(vb, lane ^ m);
    tot += shfl_i64(tot, lane ^ m);
  }
  constexpr int kWaves = kThreads / kWave;
  if (lane == 0) {
    s_red[0][t / kWave] = before;
    s_red[1][t / kWave] = vb;
    s_red[2][t / kWave] = tot;
  }
  __syncthreads();
  before = vb = tot = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    before += s_red[0][w];
    vb += s_red[1][w];
    tot += s_red[2][w];
  }

  const int64_t B = p.batch;
  const int64_t dst0 = before + vb;
  const bool w = p.wrap32 != 0;
  int64_t* const dst_ro = p.flat_row_offsets + static_cast<int64_t>(s) * (B + 1) + p.bbase[k];
  // global form: slot base + the (possibly wrapped) slot-local offset, as a reader of the merged
  // flat layout would add them
  int64_t* const dst_go = p.global_offsets ? p.global_offsets + static_cast<int64_t>(s) * B + p.bbase[k] : nullptr;
  if (e0 < n) store_pair(p.flat_values + dst0, e0, n, v0, 0, w, 0);
  if (e0 < Bk) {
    store_pair(dst_ro, e0, Bk, o0, vb, w, 0);
    if (dst_go) store_pair(dst_go, e0, Bk, o0, vb, w, before);
  }
  copy_add_i64(p.vals[k] + src0, p.flat_values + dst0, n, 0, i0 + stride, stride, w);
  copy_add_i64(so, dst_ro, Bk, vb, i0 + stride, stride, w);
  if (dst_go) copy_add_i64(so, dst_go, Bk, vb, i0 + stride, stride, w, before);
  if (i0 == 0) {
    if (k == K - 1) p.flat_row_offsets[static_cast<int64_t>(s) * (B + 1) + B] = wrap32(tot, w);
    if (k == 0) p.val_offsets[s] = before;
    if (p.global_offsets && k == 0 && s == p.num_slots - 1)
      p.global_offsets[static_cast<int64_t>(p.num_slots) * B] = before + wrap32(tot, w);
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

namespace cti {
namespace {

int merge(const int64_t* const* sub_values, const int64_t* const* sub_val_offsets,
          const int64_t* const* sub_row_offsets, const int64_t* sub_batch, const int64_t* sub_nnz, int32_t num_sub,
          int32_t num_slots, int64_t* flat_values, int64_t* flat_row_offsets, int64_t* val_offsets,
          int64_t* global_offsets, bool wrap32, void* stream) {
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
  p.wrap32 = wrap32 ? 1 : 0;
  const int64_t per_slot = (longest + num_slots - 1) / num_slots;
  const dim3 grid(static_cast<unsigned>(chunks_for(per_slot, 256)), static_cast<unsigned>(num_slots * num_sub));
  hipLaunchKernelGGL(merge_kernel, grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream), p);
  return check_launch("cti_ebag_merge_batches");
}

}  // namespace
}  // namespace cti

extern "C" int cti_ebag_merge_batches(const int64_t* const* sub_values, const int64_t* const* sub_val_offsets,
                                      const int64_t* const* sub_row_offsets, const int64_t* sub_batch,
                                      const int64_t* sub_nnz, int32_t num_sub, int32_t num_slots,
                                      int64_t* flat_values, int64_t* flat_row_offsets, int64_t* val_offsets,
                                      int64_t* global_offsets, void* stream) {
  clear_error();
  return merge(sub_values, sub_val_offsets, sub_row_offsets, sub_batch, sub_nnz, num_sub, num_slots, flat_values,
               flat_row_offsets, val_offsets, global_offsets, false, stream);
}

extern "C" int cti_ebag_merge_batches_int32(const int64_t* const* sub_values, const int64_t* const* sub_val_offsets,
                                            const int64_t* const* sub_row_offsets, const int64_t* sub_batch,
                                            const int64_t* sub_nnz, int32_t num_sub, int32_t num_slots,
                                            int64_t* flat_values, int64_t* flat_row_offsets, int64_t* val_offsets,
                                            int64_t* global_offsets, void* stream) {
  clear_error();
  return merge(sub_values, sub_val_offsets, sub_row_offsets, sub_batch, sub_nnz, num_sub, num_slots, flat_values,
               flat_row_offsets, val_offsets, global_offsets, true, stream);
}
