// Fused multi-field embedding-bag pooling for MI355X (gfx950).
//
// Semantics follow the reference kernel online_best/infer.py:805-827 and the per-field oracle
// loop baseline/infer.py:256-263:
//   out[b, col_f + d] = pool_{i in bag(f, b)} table_f[clamp(values[i], 0, rows_f - 1), d]
// with fp32 accumulation in element order, empty bag -> 0, and one rounding to the output type.
//
// Work decomposition (memory-bound gather; no matrix cores):
//   * A workgroup is 4 wavefronts and owns one tile of consecutive bags of one field.
//   * A row of D elements is read as 16-byte vectors by LANES = row_bytes/16 lanes; a wavefront
//     therefore holds R = 64/LANES "subgroups", each pooling one bag. Each lane of a subgroup
//     accumulates its columns over the bag's rows in order, so a bag pooled this way matches a
//     sequential fp32 sum bit for bit. For D = 128 bf16: 16 lanes x 16 B per row, 4 bags per
//     wavefront, 16 bags per workgroup, up to 8 rows in flight per subgroup.
//   * Bags longer than the split threshold are pooled after the short ones by the whole
//     workgroup: each wavefront takes a contiguous quarter of the bag, its subgroups take
//     interleaved rows, partials are combined across subgroups with xor shuffles and across
//     wavefronts through LDS, always in the same order (results are deterministic).
//   * Indices are loaded once per subgroup chunk (one lane per index, coalesced) and broadcast
//     to the subgroup with ds_bpermute; rows are clamped before the address is formed.
//   * Blocks are renumbered so that each of the 8 XCDs (each with its own L2) works on a
//     contiguous range of tiles, i.e. on a few fields, which keeps repeated (Zipf-hot) rows of a
//     field in one L2.
//   * Shapes whose rows are not whole 16-byte vectors (or misaligned buffers) use an element-wise
//     kernel with one wavefront per bag.
#include <stdint.h>
#include <string.h>

#include <vector>

#include "ebag_device.h"
#include "ebag_internal.h"

namespace cti {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWave * kWaves;
constexpr int kMaxFields = 64;

enum Variant : int {
  kVarL1 = 0,  // LANES = 1 << v, one 16-byte vector per lane, for v = 0..6
  kVarL64V2 = 7,
  kVarL64V4 = 8,
  kVarGeneric = 9,
  kNumVariants = 10,
};

struct FieldDesc {
  const char* table;   // row 0 of the field's table
  int64_t max_row;     // rows - 1 (clamp bound)
  int64_t row_bytes;   // byte distance between consecutive rows
  int32_t dim;         // columns pooled
  int32_t out_col;     // first output column
  int32_t gidx;        // field index used for offsets / val_base
  int32_t tile_begin;  // first tile of the field inside this launch
};

struct PoolParams {
  const void* values;
  const int64_t* offsets;   // bag offsets, field f starts at offsets + gidx * offsets_stride
  const int64_t* val_base;  // optional per-field base added to offsets (reference layout)
  char* out;
  const int32_t* tile_order;  // optional logical->physical tile map (length-binning pass)
  int64_t nnz;
  int64_t offsets_stride;
  int64_t out_row_stride;  // elements
  int64_t batch;
  int32_t num_fields;
  int32_t num_tiles;
  int32_t pooling;  // CTI_EBAG_SUM / CTI_EBAG_MEAN
  int32_t long_threshold;
  int32_t idx32;
  int32_t pad;
  FieldDesc f[kMaxFields];
};

// The hardware deals workgroups to the 8 XCDs round-robin by id. Renumber so XCD x receives
// one contiguous range of tiles (a bijection on [0, n)).
__device__ __forceinline__ int xcd_contiguous(int bid, int n) {
  const int x = bid & 7, s = bid >> 3;
  const int q = n >> 3, r = n & 7;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + s;
}

__device__ __forceinline__ int block_tile(const PoolParams& p) {
  const int bid = static_cast<int>(blockIdx.x);
  // With a binned order the list is already ranked heavy-first; deal it round-robin.
  if (p.tile_order) return p.tile_order[bid];
  return xcd_contiguous(bid, static_cast<int>(gridDim.x));
}

__device__ __forceinline__ int find_field(const PoolParams& p, int tile) {
  int lo = 0, hi = p.num_fields - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (p.f[mid].tile_begin <= tile) lo = mid; else hi = mid - 1;
  }
  return lo;
}

__device__ __forceinline__ int64_t load_index(const PoolParams& p, int64_t e) {
  return p.idx32 ? static_cast<int64_t>(static_cast<const int32_t*>(p.values)[e])
                 : static_cast<const int64_t*>(p.values)[e];
}

__device__ __forceinline__ void bag_range(const PoolParams& p, int gidx, int64_t b,
                                          int64_t& start, int64_t& end) {
  const int64_t* o = p.offsets + static_cast<int64_t>(gidx) * p.offsets_stride + b;
  const int64_t base = p.val_base ? p.val_base[gidx] : 0;
  start = clamp_i64(base + o[0], 0, p.nnz);
  end = clamp_i64(base + o[1], start, p.nnz);
}

// Vector kernel: LANES lanes x VPL 16-byte vectors per row.
template <typename TT, typename OT, int LANES, int VPL>
__global__ void __launch_bounds__(kThreads) pool_kernel(const PoolParams p) {
  constexpr int R = kWave / LANES;               // bags per wavefront
  constexpr int TB = kWaves * R;                 // bags per tile
  constexpr int VEC = 16 / Elem<TT>::kBytes;     // elements per 16-byte vector
  constexpr int NACC = VPL * VEC;                // fp32 accumulators per lane
  constexpr int D = LANES * NACC;                // row width handled by this instance
  constexpr int U0 = 8 / VPL;                    // rows in flight per subgroup per step
  constexpr int U = U0 < LANES ? U0 : LANES;

  __shared__ float s_red[kWaves * D];
  __shared__ int64_t s_start[TB], s_end[TB], s_bag[TB];
  __shared__ int s_cnt[kWaves];

  const int tile = block_tile(p);
  const int fi = find_field(p, tile);
  const char* const table = p.f[fi].table;
  const int64_t max_row = p.f[fi].max_row;
  const int64_t row_bytes = p.f[fi].row_bytes;
  const int gidx = p.f[fi].gidx;
  const int out_col = p.f[fi].out_col;

  const int lane = lane_id();
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int g = lane / LANES;   // subgroup inside the wavefront
  const int sl = lane % LANES;  // lane inside the subgroup

  const int64_t b = static_cast<int64_t>(tile - p.f[fi].tile_begin) * TB + wave * R + g;
  const bool valid = b < p.batch;
  int64_t start = 0, end = 0;
  if (valid) bag_range(p, gidx, b, start, end);
  const int64_t L = end - start;
  const bool split = valid && L > 0 && L > p.long_threshold;
  const int64_t Ls = split ? 0 : L;

  // ---- short bags: one subgroup per bag, rows accumulated in order -------------------------
  float acc[NACC];
#pragma unroll
  for (int i = 0; i < NACC; ++i) acc[i] = 0.f;

  const int64_t maxL = wave_max_i64(Ls);
  for (int64_t c = 0; c < maxL; c += LANES) {
    int64_t roff = 0;
    if (c + sl < Ls) roff = clamp_i64(load_index(p, start + c + sl), 0, max_row) * row_bytes;
    const int n = static_cast<int>(maxL - c < LANES ? maxL - c : LANES);
    for (int k = 0; k < n; k += U) {
      uint4 v[U][VPL];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t ro = shfl_i64(roff, g * LANES + k + u);
        const bool act = c + k + u < Ls;
#pragma unroll
        for (int q = 0; q < VPL; ++q) {
          v[u][q] = act ? load16(table + ro + (q * LANES + sl) * 16) : make_uint4(0u, 0u, 0u, 0u);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int q = 0; q < VPL; ++q) acc16(acc + q * VEC, v[u][q], TT{});
      }
    }
  }

  if (valid && !split) {
    if (p.pooling == CTI_EBAG_MEAN && L > 0) {
      const float fl = static_cast<float>(L);
#pragma unroll
      for (int i = 0; i < NACC; ++i) acc[i] = acc[i] / fl;
    }
    OT* o = reinterpret_cast<OT*>(p.out) + b * p.out_row_stride + out_col;
#pragma unroll
    for (int q = 0; q < VPL; ++q) store_out<VEC>(o + (q * LANES + sl) * VEC, acc + q * VEC);
  }

  // ---- long bags of this tile: split over the 4 wavefronts ---------------------------------
  const uint64_t m = __ballot(split && sl == 0);
  if (lane == 0) s_cnt[wave] = __popcll(m);
  __syncthreads();
  int before = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int cw = s_cnt[w];
    before += w < wave ? cw : 0;
    total += cw;
  }
  if (total == 0) return;  // uniform over the workgroup
  if (split && sl == 0) {
    const int pos = before + __popcll(m & ((1ull << lane) - 1ull));
    s_start[pos] = start;
    s_end[pos] = end;
    s_bag[pos] = b;
  }
  __syncthreads();

  for (int j = 0; j < total; ++j) {
    const int64_t bs = s_start[j], be = s_end[j], bb = s_bag[j];
    const int64_t per = (be - bs + kWaves - 1) / kWaves;
    const int64_t s0 = bs + wave * per < be ? bs + wave * per : be;
    const int64_t s1 = s0 + per < be ? s0 + per : be;

    float pa[NACC];
#pragma unroll
    for (int i = 0; i < NACC; ++i) pa[i] = 0.f;
    for (int64_t c = s0; c < s1; c += kWave) {
      int64_t roff = 0;
      if (c + lane < s1) roff = clamp_i64(load_index(p, c + lane), 0, max_row) * row_bytes;
      const int n = static_cast<int>(s1 - c < kWave ? s1 - c : kWave);
      for (int k = 0; k < n; k += U * R) {
        uint4 v[U][VPL];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int e = k + u * R + g;  // < 64 because U * R <= 64
          const int64_t ro = shfl_i64(roff, e);
          const bool act = e < n;
#pragma unroll
          for (int q = 0; q < VPL; ++q) {
            v[u][q] = act ? load16(table + ro + (q * LANES + sl) * 16) : make_uint4(0u, 0u, 0u, 0u);
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
          for (int q = 0; q < VPL; ++q) acc16(pa + q * VEC, v[u][q], TT{});
        }
      }
    }
    // subgroups -> wavefront: butterfly over the lane bits above the subgroup width
#pragma unroll
    for (int mk = LANES; mk < kWave; mk <<= 1) {
#pragma unroll
      for (int i = 0; i < NACC; ++i) pa[i] += shfl_xor_f32(pa[i], mk);
    }
    if (g == 0) {
#pragma unroll
      for (int q = 0; q < VPL; ++q) {
#pragma unroll
        for (int i = 0; i < VEC; ++i) s_red[wave * D + (q * LANES + sl) * VEC + i] = pa[q * VEC + i];
      }
    }
    __syncthreads();
    if (wave == 0 && g == 0) {
      float r[NACC];
#pragma unroll
      for (int q = 0; q < VPL; ++q) {
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          const int col = (q * LANES + sl) * VEC + i;
          float x = s_red[col];
#pragma unroll
          for (int w = 1; w < kWaves; ++w) x += s_red[w * D + col];
          r[q * VEC + i] = x;
        }
      }
      if (p.pooling == CTI_EBAG_MEAN) {
        const float fl = static_cast<float>(be - bs);
#pragma unroll
        for (int i = 0; i < NACC; ++i) r[i] = r[i] / fl;
      }
      OT* o = reinterpret_cast<OT*>(p.out) + bb * p.out_row_stride + out_col;
#pragma unroll
      for (int q = 0; q < VPL; ++q) store_out<VEC>(o + (q * LANES + sl) * VEC, r + q * VEC);
    }
    __syncthreads();
  }
}

// Element-wise kernel for any row width / alignment: one wavefront per bag, rows accumulated in
// order, 4 columns per lane per pass.
template <typename TT, typename OT>
__global__ void __launch_bounds__(kThreads) pool_generic_kernel(const PoolParams p) {
  constexpr int NC = 4;
  const int tile = block_tile(p);
  const int fi = find_field(p, tile);
  const char* const table = p.f[fi].table;
  const int64_t max_row = p.f[fi].max_row;
  const int64_t row_bytes = p.f[fi].row_bytes;
  const int dim = p.f[fi].dim;
  const int out_col = p.f[fi].out_col;
  const int lane = lane_id();
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int64_t b = static_cast<int64_t>(tile - p.f[fi].tile_begin) * kWaves + wave;
  if (b >= p.batch) return;  // uniform over the wavefront; this kernel has no block barriers
  int64_t start, end;
  bag_range(p, p.f[fi].gidx, b, start, end);
  const int64_t L = end - start;
  OT* o = reinterpret_cast<OT*>(p.out) + b * p.out_row_stride + out_col;
  for (int c0 = 0; c0 < dim; c0 += kWave * NC) {
    float acc[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i) acc[i] = 0.f;
    for (int64_t c = start; c < end; c += kWave) {
      int64_t roff = 0;
      if (c + lane < end) roff = clamp_i64(load_index(p, c + lane), 0, max_row) * row_bytes;
      const int n = static_cast<int>(end - c < kWave ? end - c : kWave);
      for (int k = 0; k < n; ++k) {
        const int64_t ro = shfl_i64(roff, k);
#pragma unroll
        for (int i = 0; i < NC; ++i) {
          const int col = c0 + i * kWave + lane;
          if (col < dim) acc[i] += Elem<TT>::load(table + ro + static_cast<int64_t>(col) * Elem<TT>::kBytes);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int col = c0 + i * kWave + lane;
      if (col < dim) {
        float r = acc[i];
        if (p.pooling == CTI_EBAG_MEAN && L > 0) r = r / static_cast<float>(L);
        store_one(o + col, r);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------------------
int lanes_of(int variant) { return variant <= 6 ? (1 << variant) : 64; }
int bags_per_tile(int variant) { return variant == kVarGeneric ? kWaves : kWaves * (kWave / lanes_of(variant)); }

int default_long_threshold(int variant) {
  if (variant == kVarGeneric) return INT32_MAX;  // the element-wise kernel never splits
  const int lanes = lanes_of(variant);
  int t = 4 * lanes;
  if (t < 16) t = 16;
  if (t > 256) t = 256;
  return t;
}

int pick_variant(const cti_ebag_table& t, int tb, int ob, const void* out, int64_t out_row_stride) {
  const int64_t row_bytes = static_cast<int64_t>(t.dim) * tb;
  const bool table_ok = (reinterpret_cast<uintptr_t>(t.data) % 16 == 0) && ((t.row_stride * tb) % 16 == 0);
  const int vec = 16 / tb;
  const int align = vec * ob < 16 ? vec * ob : 16;
  const bool out_ok = (reinterpret_cast<uintptr_t>(out) % align == 0) &&
                      ((out_row_stride * ob) % align == 0) &&
                      ((static_cast<int64_t>(t.out_col) * ob) % align == 0);
  if (!table_ok || !out_ok || row_bytes % 16 != 0) return kVarGeneric;
  const int64_t nvec = row_bytes / 16;
  for (int v = 0; v <= 6; ++v) {
    if (nvec == (int64_t{1} << v)) return v;
  }
  if (nvec == 128) return kVarL64V2;
  if (nvec == 256) return kVarL64V4;
  return kVarGeneric;
}

template <typename TT, typename OT>
hipError_t launch_variant(int variant, const PoolParams& p, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(p.num_tiles)), block(kThreads);
  switch (variant) {
    case 0: hipLaunchKernelGGL((pool_kernel<TT, OT, 1, 1>), grid, block, 0, s, p); break;
    case 1: hipLaunchKernelGGL((pool_kernel<TT, OT, 2, 1>), grid, block, 0, s, p); break;
    case 2: hipLaunchKernelGGL((pool_kernel<TT, OT, 4, 1>), grid, block, 0, s, p); break;
    case 3: hipLaunchKernelGGL((pool_kernel<TT, OT, 8, 1>), grid, block, 0, s, p); break;
    case 4: hipLaunchKernelGGL((pool_kernel<TT, OT, 16, 1>), grid, block, 0, s, p); break;
    case 5: hipLaunchKernelGGL((pool_kernel<TT, OT, 32, 1>), grid, block, 0, s, p); break;
    case 6: hipLaunchKernelGGL((pool_kernel<TT, OT, 64, 1>), grid, block, 0, s, p); break;
    case kVarL64V2: hipLaunchKernelGGL((pool_kernel<TT, OT, 64, 2>), grid, block, 0, s, p); break;
    case kVarL64V4: hipLaunchKernelGGL((pool_kernel<TT, OT, 64, 4>), grid, block, 0, s, p); break;
    default: hipLaunchKernelGGL((pool_generic_kernel<TT, OT>), grid, block, 0, s, p); break;
  }
  return hipGetLastError();
}

hipError_t launch_typed(int tdt, int odt, int variant, const PoolParams& p, hipStream_t s) {
  switch (tdt * 3 + odt) {
    case CTI_EBAG_F32 * 3 + CTI_EBAG_F32: return launch_variant<float, float>(variant, p, s);
    case CTI_EBAG_F32 * 3 + CTI_EBAG_BF16: return launch_variant<float, bf16_t>(variant, p, s);
    case CTI_EBAG_F32 * 3 + CTI_EBAG_F16: return launch_variant<float, f16_t>(variant, p, s);
    case CTI_EBAG_BF16 * 3 + CTI_EBAG_F32: return launch_variant<bf16_t, float>(variant, p, s);
    case CTI_EBAG_BF16 * 3 + CTI_EBAG_BF16: return launch_variant<bf16_t, bf16_t>(variant, p, s);
    case CTI_EBAG_BF16 * 3 + CTI_EBAG_F16: return launch_variant<bf16_t, f16_t>(variant, p, s);
    case CTI_EBAG_F16 * 3 + CTI_EBAG_F32: return launch_variant<f16_t, float>(variant, p, s);
    case CTI_EBAG_F16 * 3 + CTI_EBAG_BF16: return launch_variant<f16_t, bf16_t>(variant, p, s);
    default: return launch_variant<f16_t, f16_t>(variant, p, s);
  }
}

struct Job {
  const void* values;
  int32_t idx32;
  int64_t nnz;
  const int64_t* offsets;
  const int64_t* val_base;
  int64_t offsets_stride;
  int64_t batch;
  int32_t num_fields;
  const cti_ebag_table* tables;
  int32_t tdt;
  int32_t pooling;
  void* out;
  int32_t odt;
  int64_t out_row_stride;
  int32_t long_threshold;  // 0 = per-variant default
};

int validate_tables(const Job& j) {
  for (int f = 0; f < j.num_fields; ++f) {
    const cti_ebag_table& t = j.tables[f];
    if (!t.data) return set_error(CTI_EBAG_EINVAL, "table %d: data is NULL", f);
    if (t.rows < 1) return set_error(CTI_EBAG_EINVAL, "table %d: rows must be >= 1 (got %lld)", f, (long long)t.rows);
    if (t.dim < 1) return set_error(CTI_EBAG_EINVAL, "table %d: dim must be >= 1 (got %d)", f, t.dim);
    if (t.row_stride < t.dim) return set_error(CTI_EBAG_EINVAL, "table %d: row_stride %lld < dim %d", f, (long long)t.row_stride, t.dim);
    if (t.out_col < 0 || static_cast<int64_t>(t.out_col) + t.dim > j.out_row_stride)
      return set_error(CTI_EBAG_EINVAL, "table %d: columns [%d, %lld) fall outside the output row of %lld", f, t.out_col,
                       (long long)t.out_col + t.dim, (long long)j.out_row_stride);
  }
  return CTI_EBAG_OK;
}

int run_job(const Job& j, hipStream_t stream) {
  if (j.batch == 0 || j.num_fields == 0) return CTI_EBAG_OK;
  const int tb = dtype_bytes(j.tdt), ob = dtype_bytes(j.odt);
  // Group fields by kernel variant; each group is one launch (per 64 fields).
  std::vector<int> var(j.num_fields);
  for (int f = 0; f < j.num_fields; ++f) var[f] = pick_variant(j.tables[f], tb, ob, j.out, j.out_row_stride);
  for (int v = 0; v < kNumVariants; ++v) {
    std::vector<int> fields;
    for (int f = 0; f < j.num_fields; ++f) if (var[f] == v) fields.push_back(f);
    for (size_t c0 = 0; c0 < fields.size(); c0 += kMaxFields) {
      PoolParams p;
      memset(&p, 0, sizeof(p));
      p.values = j.values;
      p.offsets = j.offsets;
      p.val_base = j.val_base;
      p.out = static_cast<char*>(j.out);
      p.tile_order = nullptr;
      p.nnz = j.nnz;
      p.offsets_stride = j.offsets_stride;
      p.out_row_stride = j.out_row_stride;
      p.batch = j.batch;
      p.pooling = j.pooling;
      p.idx32 = j.idx32;
      p.long_threshold = j.long_threshold == 0 ? default_long_threshold(v)
                                               : (j.long_threshold < 0 ? -1 : j.long_threshold);
      const int bpt = bags_per_tile(v);
      const int64_t tiles_per_field = (j.batch + bpt - 1) / bpt;
      const size_t nf = fields.size() - c0 < static_cast<size_t>(kMaxFields) ? fields.size() - c0 : kMaxFields;
      if (tiles_per_field * static_cast<int64_t>(nf) > INT32_MAX)
        return set_error(CTI_EBAG_EUNSUPPORTED, "batch of %lld samples needs more than 2^31 tiles", (long long)j.batch);
      p.num_fields = static_cast<int32_t>(nf);
      for (size_t i = 0; i < nf; ++i) {
        const int f = fields[c0 + i];
        const cti_ebag_table& t = j.tables[f];
        FieldDesc& d = p.f[i];
        d.table = static_cast<const char*>(t.data);
        d.max_row = t.rows - 1;
        d.row_bytes = t.row_stride * tb;
        d.dim = t.dim;
        d.out_col = t.out_col;
        d.gidx = f;
        d.tile_begin = static_cast<int32_t>(tiles_per_field * static_cast<int64_t>(i));
      }
      p.num_tiles = static_cast<int32_t>(tiles_per_field * static_cast<int64_t>(nf));
      const hipError_t e = launch_typed(j.tdt, j.odt, v, p, stream);
      if (e != hipSuccess) return set_error(CTI_EBAG_EHIP, "pooling kernel launch failed: %s", hipGetErrorString(e));
    }
  }
  return CTI_EBAG_OK;
}

bool dtype_ok(int32_t dt) { return dt == CTI_EBAG_F32 || dt == CTI_EBAG_BF16 || dt == CTI_EBAG_F16; }

}  // namespace
}  // namespace cti

using namespace cti;

extern "C" int cti_ebag_fused_all_slots(const int64_t* values, const int64_t* val_offsets,
                                        const int64_t* row_offsets, const void* weight, int32_t dtype,
                                        void* out, int64_t batch_size, int32_t num_slots, int32_t emb_dim,
                                        int64_t max_idx, int64_t nnz, void* stream) {
  clear_error();
  if (batch_size < 0) return set_error(CTI_EBAG_EINVAL, "batch_size must be >= 0 (got %lld)", (long long)batch_size);
  if (num_slots < 0) return set_error(CTI_EBAG_EINVAL, "num_slots must be >= 0 (got %d)", num_slots);
  if (emb_dim < 1) return set_error(CTI_EBAG_EINVAL, "emb_dim must be >= 1 (got %d)", emb_dim);
  if (max_idx < 0) return set_error(CTI_EBAG_EINVAL, "max_idx must be >= 0 (got %lld)", (long long)max_idx);
  if (nnz < 0) return set_error(CTI_EBAG_EINVAL, "nnz must be >= 0 (got %lld)", (long long)nnz);
  if (!dtype_ok(dtype)) return set_error(CTI_EBAG_EINVAL, "unknown dtype code %d", dtype);
  if (batch_size == 0 || num_slots == 0) return CTI_EBAG_OK;
  if (!val_offsets || !row_offsets || !weight || !out || (nnz > 0 && !values))
    return set_error(CTI_EBAG_EINVAL, "NULL device pointer among values/val_offsets/row_offsets/weight/out");
  std::vector<cti_ebag_table> tables(num_slots);
  for (int s = 0; s < num_slots; ++s) {
    tables[s].data = weight;
    tables[s].rows = max_idx + 1;
    tables[s].row_stride = emb_dim;
    tables[s].dim = emb_dim;
    tables[s].out_col = s * emb_dim;
  }
  Job j;
  j.values = values;
  j.idx32 = 0;
  j.nnz = nnz;
  j.offsets = row_offsets;
  j.val_base = val_offsets;
  j.offsets_stride = batch_size + 1;
  j.batch = batch_size;
  j.num_fields = num_slots;
  j.tables = tables.data();
  j.tdt = dtype;
  j.pooling = CTI_EBAG_SUM;
  j.out = out;
  j.odt = dtype;
  j.out_row_stride = static_cast<int64_t>(num_slots) * emb_dim;
  j.long_threshold = 0;
  return run_job(j, static_cast<hipStream_t>(stream));
}

extern "C" int64_t cti_ebag_workspace_bytes(int64_t batch_size, int32_t num_fields) {
  if (batch_size < 0 || num_fields < 0) return -1;
  return 0;
}

extern "C" int cti_ebag_forward(const void* values, int32_t index_type, int64_t nnz, const int64_t* offsets,
                                int64_t batch_size, int32_t num_fields, const cti_ebag_table* tables,
                                int32_t table_dtype, int32_t pooling, void* out, int32_t out_dtype,
                                int64_t out_row_stride, void* workspace, int64_t workspace_bytes,
                                const cti_ebag_options* opts, void* stream) {
  clear_error();
  (void)workspace;
  (void)workspace_bytes;
  if (index_type != CTI_EBAG_I64 && index_type != CTI_EBAG_I32)
    return set_error(CTI_EBAG_EINVAL, "unknown index type code %d", index_type);
  if (!dtype_ok(table_dtype)) return set_error(CTI_EBAG_EINVAL, "unknown table dtype code %d", table_dtype);
  if (!dtype_ok(out_dtype)) return set_error(CTI_EBAG_EINVAL, "unknown output dtype code %d", out_dtype);
  if (pooling != CTI_EBAG_SUM && pooling != CTI_EBAG_MEAN) return set_error(CTI_EBAG_EINVAL, "unknown pooling code %d", pooling);
  if (nnz < 0) return set_error(CTI_EBAG_EINVAL, "nnz must be >= 0 (got %lld)", (long long)nnz);
  if (batch_size < 0) return set_error(CTI_EBAG_EINVAL, "batch_size must be >= 0 (got %lld)", (long long)batch_size);
  if (num_fields < 0) return set_error(CTI_EBAG_EINVAL, "num_fields must be >= 0 (got %d)", num_fields);
  if (out_row_stride < 1) return set_error(CTI_EBAG_EINVAL, "out_row_stride must be >= 1 (got %lld)", (long long)out_row_stride);
  if (batch_size == 0 || num_fields == 0) return CTI_EBAG_OK;
  if (!tables) return set_error(CTI_EBAG_EINVAL, "tables (host array) is NULL");
  if (!offsets || !out || (nnz > 0 && !values)) return set_error(CTI_EBAG_EINVAL, "NULL device pointer among values/offsets/out");
  if (opts && opts->use_bins) return set_error(CTI_EBAG_EUNSUPPORTED, "length binning is not available in this build");
  Job j;
  j.values = values;
  j.idx32 = index_type == CTI_EBAG_I32;
  j.nnz = nnz;
  j.offsets = offsets;
  j.val_base = nullptr;
  j.offsets_stride = batch_size;
  j.batch = batch_size;
  j.num_fields = num_fields;
  j.tables = tables;
  j.tdt = table_dtype;
  j.pooling = pooling;
  j.out = out;
  j.odt = out_dtype;
  j.out_row_stride = out_row_stride;
  j.long_threshold = opts ? opts->long_threshold : 0;
  const int rc = validate_tables(j);
  if (rc != CTI_EBAG_OK) return rc;
  return run_job(j, static_cast<hipStream_t>(stream));
}
