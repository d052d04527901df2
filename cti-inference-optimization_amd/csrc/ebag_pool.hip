// Fused multi-field embedding-bag pooling for MI355X (gfx950).
//
// Semantics follow the reference kernel online_best/infer.py:805-827 and the per-field oracle
// loop baseline/infer.py:256-263:
//   out[b, col_f + d] = pool_{i in bag(f, b)} table_f[clamp(values[i], 0, rows_f - 1), d]
// with fp32 accumulation, empty bag -> 0, and one rounding to the output type. int8 tables
// (online_best/infer.py:904-942) accumulate acc = fma(q, row_scale[row], acc) in element order.
//
// This is a gather (no matrix cores); on MI355X it is bound by vector-ALU issue and memory latency
// more than by HBM bandwidth, so the design keeps VALU work per pooled row small. Decomposition:
//   * A row of D elements is read as lane vectors (16 bytes; 8 bytes for int8, so a lane holds
//     8 elements either way) by LANES = row_bytes / vector bytes lanes, so a 64-lane wavefront
//     holds R = 64/LANES lane groups ("subgroups"). For D = 128 bf16: 16 lanes x 16 B per row,
//     4 subgroups per wavefront; D = 128 int8: 16 lanes x 8 B.
//   * Main kernel: one wavefront per workgroup, one tile of ROUNDS * R consecutive bags of one
//     field. The tile's short bags are ranked by length and pooled R at a time, one bag per
//     subgroup, so the bags pooled side by side need about the same number of steps:
//       - short bag (L <= sub_threshold): each lane adds its columns of the bag's rows in element
//         order, so the result equals a sequential fp32 sum bit for bit;
//       - medium bag (sub_threshold < L <= block_threshold): split over the wavefront's subgroups
//         (interleaved rows), partials combined with an xor butterfly in a fixed order;
//       - long bag (L > block_threshold, only with the length-binning pass): left to the long kernel.
//     Single-wavefront workgroups need no workgroup barrier, so a wavefront retires as soon as its
//     own bags are done (measured: multi-wavefront workgroups are slower, also when they share a
//     length ranking). Row ids are clamped, narrowed to 32 bits (tables have < 2^31 rows) and
//     broadcast through LDS; a step reads kRowsInFlight ids, then issues that many row loads
//     before consuming any. A bag's ids are loaded one chunk ahead, so the next chunk's id load
//     completes under the current chunk's row loads. Tables under 4 GiB with power-of-two row sizes are read with buffer
//     loads: a row's offset is one shift-add, and rows past a bag's end use an out-of-range offset
//     that returns zeros without a memory request (no per-row branch).
//   * Streamed tiles (256-byte rows of fp32 / bf16 / fp16 tables and 128-byte rows of int8 tables,
//     without binning and with the default short-bag limit): the same tiles, but the wavefront
//     walks the tile's rows in order across bag boundaries (with well-formed offsets they are one
//     contiguous run of `values`), each lane holding 4 bytes (int8: 2 bytes and the row's scale)
//     of every row, one row per load instruction, 16 rows in flight;
//     a bag is stored when its last row has been added, so every bag, whatever its length, is a
//     sequential fp32 sum in element order. Row ids come one 64-row chunk at a time through
//     buffer loads over `values` (the next chunk in flight) and are broadcast with readlane.
//     No lane group waits for another's longer bag and no bag is split.
//   * Dispatch order (optional): a launch can follow a tile order made one batch ahead, in which
//     each XCD starts its tiles with the most rows per bag, and make the next batch's order in a
//     few extra workgroups at its first dispatch positions. It shortens the launch's drain; the
//     results do not depend on it.
//   * Mean: one fp64 reciprocal per bag, RN32(RN64(sum * 1/L)) per element, which equals the IEEE
//     fp32 division except for quotients below the normal range (those take the division).
//     Conversions to bf16 use the hardware round-to-nearest-even pack.
//   * Length-binning pass (optional): one thread per bag; bags longer than block_threshold are
//     appended, with their value ranges, to one of two lists in the caller's workspace (one
//     global atomic per workgroup and list): up to split_threshold rows on the one-wavefront
//     list, longer ones on the split list.
//   * Long kernel: 8 wavefronts (4 for 2 KB rows) per workgroup, looping over the lists; a bag on
//     the split list is cut into one contiguous slice per wavefront and the wavefront partials
//     are combined through LDS in wavefront order; a bag on the one-wavefront list is pooled by
//     one wavefront, which loads its next bag's entry meanwhile.
//   * Fields whose rows differ in width but are 4 to 64 lanes of one vector share one launch
//     sequence: the main kernel runs each tile's own row shape, the long kernel picks each bag's
//     shape at run time.
//   * List counter hand-off without contended atomics: the binning pass counts into `count`; the
//     main kernel, which runs between the two, has one thread move `count` to `total` and zero
//     `count`; the long kernel reads `total`. A call therefore leaves `count` at zero for the next.
//   * Tiles are renumbered so each of the 8 XCDs (own L2 each) works on a contiguous range of
//     tiles, i.e. on a few fields at a time.
//   * Rows that are not whole lane vectors, or misaligned buffers, use an element-wise kernel
//     (one wavefront per bag, element order, never split).
// All kernels write disjoint output rows and combine partial sums in a fixed order, so results
// are deterministic run to run.
#include <stdint.h>
#include <string.h>

#include <type_traits>
#include <vector>

#include "ebag_device.h"
#include "ebag_internal.h"

namespace cti {
namespace {

// Measured constants (MI355X, 28 x 4096 bags of bf16 rows of 128):
//   row loads in flight per lane before they are consumed: 1 / 2 / 4 / 8 / 16 ran 86.7 / 66.3 /
//   56.3 / 58.4 / 68.1 us on an early build (8 against 4 later: 44.8 against 44.3);
//   rounds of R length-ranked bags per tile: 2 / 3 / 4 ran 41.7 / 42.5 / 42.1 us.
constexpr int kRowsInFlight = 4;
constexpr int kRounds = 2;

constexpr int kMainThreads = kWave;  // main kernel: one wavefront per workgroup
constexpr int kBinThreads = 256;
constexpr int64_t kLongBlocksMax = 1024;  // workgroups of the long kernel (they loop over the list)
constexpr int kMaxFields = 64;
constexpr int64_t kNoLimit = INT64_MAX;

// One lane's row vector (Elem<TT>::kVecBytes bytes; an 8-byte vector fills .x and .y).
template <typename TT>
__device__ __forceinline__ uint4 load_row_vec(const char* p) {
  if constexpr (Elem<TT>::kVecBytes == 16) {
    return load16(p);
  } else {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    return make_uint4(v.x, v.y, 0u, 0u);
  }
}

enum Variant : int {
  kVarL1 = 0,  // LANES = 1 << v, one lane vector per lane, for v = 0..6
  kVarL64V2 = 7,
  kVarL64V4 = 8,
  kVarGeneric = 9,
  kNumVariants = 10,
  kVarMixed = 10,  // fields of several of the shapes kMixedLo..kMixedHi in one launch sequence
};
// Shapes a mixed-width launch covers: 4 to 64 lanes of one vector per row, i.e. rows of 64 B to
// 1 KB (bf16 D = 32..512, fp32 D = 16..256, int8 D = 32..512). Each shape the kernels switch
// over adds registers; rows of 16 or 32 B keep launches of their own.
constexpr int kMixedLo = 2, kMixedHi = 6;

struct FieldDesc {
  const char* table;   // row 0 of the field's table
  const float* row_scale;  // per-row scale of an int8 table (NULL otherwise)
  int64_t max_row;     // rows - 1 (clamp bound)
  int64_t row_bytes;   // byte distance between consecutive rows
  int32_t dim;         // columns pooled
  int32_t out_col;     // first output column
  int32_t gidx;        // field index used for offsets / val_base
  uint32_t span_bytes; // bytes from row 0 to the end of the last row, when below 4 GiB (else 0)
  int32_t lanes_log2;  // mixed-width launches: the field's rows are 1 << lanes_log2 lanes x one vector
  int32_t tile_begin;  // mixed-width launches: the field's first tile (fields in tile order)
};

struct PoolParams {
  const void* values;
  const void* offsets;      // bag offsets, field f starts at offsets + gidx * offsets_stride
  const void* val_base;     // optional per-field base added to offsets (reference layout)
  char* out;
  int64_t nnz;
  int64_t offsets_stride;
  int64_t out_row_stride;   // elements
  int64_t batch;
  int64_t sub_threshold;    // longer bags are split over a wavefront's subgroups
  int64_t block_threshold;  // longer bags go to the list kernel (kNoLimit without binning)
  int64_t split_threshold;  // listed bags longer than this are split over a workgroup
  unsigned int* bin_count;  // binning: list lengths being built (NULL without binning): [0] one-wave, [2] split
  unsigned int* bin_total;  // binning: list lengths handed to the list kernel: [0] one-wave, [2] split
  const int32_t* tile_order;  // optional dispatch order of this launch (layout at kOrderMagic), NULL = none
  int32_t* next_order;        // optional: the first kOrderBlocks workgroups write the next batch's order here
  const void* next_offsets;   // the next batch's bag offsets (type and layout of `offsets`)
  int32_t order_blocks;       // with next_order: workgroups that make it (8 x chunks per XCD range)
  int32_t num_fields;
  int32_t num_tiles;
  int32_t tiles_per_field;  // every field of a launch has the same number of tiles
  uint32_t tpf_inv;         // floor((2^32 - 1) / tiles_per_field): field_of_tile's multiplier
  int32_t pooling;          // CTI_EBAG_SUM / CTI_EBAG_MEAN
  int32_t idx32;
  int32_t off32;            // offsets and val_base are int32 (else int64)
  int32_t buffer_ok;        // every field's span_bytes is set: rows are read with buffer loads
  int32_t round_bf16;       // int8 tables: round each result to bf16 before the output type (the
                            // reference's int8 kernel stores acc.to(bfloat16), online_best/infer.py:941)
  int32_t stream_ok;        // rows of 16 lane vectors may take streamed tiles (no binning, default
                            // short-bag limit, walks and id offsets within 32 bits)
  int32_t stream_out;       // the output block is at least kStreamOutBytes: non-temporal stores
  FieldDesc f[kMaxFields];
};

// Workspace of the length-binning pass: counters, then the list of long bags.
// Two lists share the workspace's entry array: bags pooled by one wavefront each grow from the
// front, bags split over a workgroup's wavefronts grow from the back (together they never exceed
// the number of bags of a launch, which the array holds).
// Each entry also carries the bag's value range, so the list kernel needs no offset lookup.
struct LongList {
  unsigned int* count;   // one-wavefront list length, incremented by the binning pass
  unsigned int* total;   // its snapshot read by the list kernel
  unsigned int* count2;  // split list length
  unsigned int* total2;
  int64_t* bags;         // entries: (local field index << 40) | sample index
  int64_t* starts;       // entry i's bag is values[starts[i], ends[i])
  int64_t* ends;
  int64_t capacity;      // entries in each array; split entry j is at index capacity - 1 - j
};
constexpr int64_t kWorkspaceHeader = 256;
static_assert(sizeof(PoolParams) + sizeof(LongList) <= 4096, "kernel arguments must fit in 4 KB");

__device__ __forceinline__ int xcd_contiguous(int bid, int n) {
  // Hardware deals workgroups to the 8 XCDs round-robin; map XCD x to one contiguous range.
  const int x = bid & 7, s = bid >> 3;
  const int q = n >> 3, r = n & 7;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + s;
}

// Tile position of dispatch position `pos` in a launch of n tiles.
__device__ __forceinline__ int xcd_position(int pos, int n) { return xcd_contiguous(pos, n); }

__device__ __forceinline__ int block_tile() {
  return xcd_position(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
}

// int8 tables of the reference-layout entry points: the pooled value as the reference's int8
// kernel leaves it, rounded to bf16 (round to nearest even) whatever the output type.
template <typename TT, int N>
__device__ __forceinline__ void round_like_reference(const PoolParams& p, float* r) {
  if constexpr (Quantized<TT>::value) {
    if (p.round_bf16) {
#pragma unroll
      for (int i = 0; i < N; ++i) r[i] = __uint_as_float(pack_bf16x2(r[i], 0.f) << 16);
    }
  }
}

// Buffer resource over one table: 32-bit byte offsets, offsets at or past the span read as zeros.
typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc make_rsrc(const char* base, uint32_t span) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), static_cast<short>(0), static_cast<int>(span),
                                           0x00020000);  // raw buffer, 32-bit data format
}
__device__ __forceinline__ uint4 buffer_load16(Rsrc r, unsigned int off) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}
template <typename TT>
__device__ __forceinline__ uint4 buffer_load_vec(Rsrc r, unsigned int off) {
  if constexpr (Elem<TT>::kVecBytes == 16) {
    return buffer_load16(r, off);
  } else {
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    return make_uint4(v.x, v.y, 0u, 0u);
  }
}
__device__ __forceinline__ float buffer_load_f32(Rsrc r, unsigned int off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

__device__ __forceinline__ int64_t load_index(const PoolParams& p, int64_t e) {
  return p.idx32 ? static_cast<int64_t>(static_cast<const int32_t*>(p.values)[e])
                 : static_cast<const int64_t*>(p.values)[e];
}

__device__ __forceinline__ int64_t load_offset(const PoolParams& p, const void* a, int64_t i) {
  return p.off32 ? static_cast<int64_t>(static_cast<const int32_t*>(a)[i]) : static_cast<const int64_t*>(a)[i];
}

// Bag b of field gidx: values[start, end), clamped to [0, nnz]. The three loads are issued before
// any is used (a branch around the optional base, or a conversion right after each load, would
// make each wait for the one before): without val_base the base is read from the offsets array
// and masked off.
template <typename OFF>
__device__ __forceinline__ void bag_range_typed(const PoolParams& p, int gidx, int64_t b, int64_t& start,
                                                int64_t& end) {
  const int64_t i = static_cast<int64_t>(gidx) * p.offsets_stride + b;
  const OFF* const o = static_cast<const OFF*>(p.offsets);
  const OFF* const vb = p.val_base ? static_cast<const OFF*>(p.val_base) + gidx : o;
  const OFF x0 = o[i], x1 = o[i + 1], xb = *vb;
  const int64_t base = p.val_base ? static_cast<int64_t>(xb) : 0;
  start = clamp_i64(base + static_cast<int64_t>(x0), 0, p.nnz);
  end = clamp_i64(base + static_cast<int64_t>(x1), start, p.nnz);
}
__device__ __forceinline__ void bag_range(const PoolParams& p, int gidx, int64_t b,
                                          int64_t& start, int64_t& end) {
  if (p.off32) bag_range_typed<int32_t>(p, gidx, b, start, end);
  else bag_range_typed<int64_t>(p, gidx, b, start, end);
}

// Row shape of one kernel instance.
template <typename TT, int LANES, int VPL>
struct Shape {
  static constexpr int R = kWave / LANES;            // subgroups per wavefront
  static constexpr int VB = Elem<TT>::kVecBytes;     // bytes per lane vector
  static constexpr int VEC = VB / Elem<TT>::kBytes;  // elements per lane vector
  static constexpr int NACC = VPL * VEC;             // fp32 accumulators per lane
  static constexpr int D = LANES * NACC;             // row width
  static constexpr int U0 = kRowsInFlight / VPL > 0 ? kRowsInFlight / VPL : 1;
  static constexpr int U = U0 < LANES ? U0 : LANES;  // rows per subgroup per step
};

// Accumulate the rows of elements [s0, s1) into this lane's columns; subgroup g of the
// wavefront takes elements s0 + g, s0 + g + R, ... in order. Wave-uniform s0, s1. `ids` is this
// wavefront's private 64-entry LDS slice for row ids: its accesses are ordered by program order
// within the wavefront, so no workgroup barrier is involved.
template <typename TT, int LANES, int VPL>
__device__ __forceinline__ void wave_slice_partial(const PoolParams& p, const char* table, const float* row_scale,
                                                   int64_t max_row, int64_t row_bytes, int64_t s0, int64_t s1,
                                                   float* pa, unsigned int* ids) {
  using S = Shape<TT, LANES, VPL>;
  const int lane = lane_id();
  const int g = lane / LANES, sl = lane % LANES;
  int64_t next_id = s0 + lane < s1 ? load_index(p, s0 + lane) : 0;
  for (int64_t c = s0; c < s1; c += kWave) {
    // ids one chunk ahead: the next chunk's id load overlaps this chunk's row loads
    const int64_t id = next_id;
    if (c + kWave + lane < s1) next_id = load_index(p, c + kWave + lane);
    ids[lane] = c + lane < s1 ? static_cast<unsigned int>(clamp_i64(id, 0, max_row)) : 0u;
    const int n = static_cast<int>(s1 - c < kWave ? s1 - c : kWave);
    for (int k = 0; k < n; k += S::U * S::R) {
      uint4 v[S::U][VPL];
      float sc[S::U];
#pragma unroll
      for (int u = 0; u < S::U; ++u) {
        const int e = k + u * S::R + g;  // < 64 because U * R <= 64
        const char* row = table + static_cast<uint64_t>(ids[e]) * static_cast<uint64_t>(row_bytes);
        const bool act = e < n;
#pragma unroll
        for (int q = 0; q < VPL; ++q)
          v[u][q] = act ? load_row_vec<TT>(row + (q * LANES + sl) * S::VB) : make_uint4(0u, 0u, 0u, 0u);
        sc[u] = 1.f;
        if constexpr (Quantized<TT>::value) sc[u] = act ? row_scale[ids[e]] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < S::U; ++u) {
#pragma unroll
        for (int q = 0; q < VPL; ++q) acc_row<TT>(pa + q * S::VEC, v[u][q], sc[u]);
      }
    }
  }
  // subgroups -> wavefront: butterfly over the lane bits above the subgroup width
#pragma unroll
  for (int mk = LANES; mk < kWave; mk <<= 1) {
#pragma unroll
    for (int i = 0; i < S::NACC; ++i) pa[i] += shfl_xor_f32(pa[i], mk);
  }
}

template <typename TT, typename OT, int LANES, int VPL>
__device__ __forceinline__ void store_bag(const PoolParams& p, int64_t b, int out_col, int64_t L, float* a) {
  using S = Shape<TT, LANES, VPL>;
  const int sl = lane_id() % LANES;
  float r[S::NACC];
#pragma unroll
  for (int i = 0; i < S::NACC; ++i) r[i] = a[i];
  if (p.pooling == CTI_EBAG_MEAN && L > 0) div_by_count<S::NACC>(r, 1.0 / static_cast<double>(L), static_cast<float>(L));
  round_like_reference<TT, S::NACC>(p, r);
  OT* o = reinterpret_cast<OT*>(p.out) + b * p.out_row_stride + out_col;
#pragma unroll
  for (int q = 0; q < VPL; ++q) store_out<S::VEC>(o + (q * LANES + sl) * S::VEC, r + q * S::VEC, p.stream_out);
}

// U row loads of one step: elements k .. k+U-1 of this subgroup's current chunk, whose row ids
// are in `ids` (the subgroup's slice of the wavefront's LDS row-id buffer; immediate offsets).
template <typename TT, int LANES, int VPL>
__device__ __forceinline__ void load_step(const char* table, const float* row_scale, int64_t row_bytes,
                                          const unsigned int* ids, int sl, int k, int live,
                                          uint4 (&v)[Shape<TT, LANES, VPL>::U][VPL], float (&sc)[Shape<TT, LANES, VPL>::U]) {
  using S = Shape<TT, LANES, VPL>;
#pragma unroll
  for (int u = 0; u < S::U; ++u) {
    const unsigned int r = ids[k + u];
    const char* row = table + static_cast<uint64_t>(r) * static_cast<uint64_t>(row_bytes);
    const bool act = k + u < live;
#pragma unroll
    for (int q = 0; q < VPL; ++q)
      v[u][q] = act ? load_row_vec<TT>(row + (q * LANES + sl) * S::VB) : make_uint4(0u, 0u, 0u, 0u);
    sc[u] = 1.f;
    if constexpr (Quantized<TT>::value) sc[u] = act ? row_scale[r] : 0.f;
  }
}

template <typename TT, int LANES, int VPL>
__device__ __forceinline__ void add_step(float* acc, const uint4 (&v)[Shape<TT, LANES, VPL>::U][VPL],
                                         const float (&sc)[Shape<TT, LANES, VPL>::U]) {
  using S = Shape<TT, LANES, VPL>;
#pragma unroll
  for (int u = 0; u < S::U; ++u) {
#pragma unroll
    for (int q = 0; q < VPL; ++q) acc_row<TT>(acc + q * S::VEC, v[u][q], sc[u]);
  }
}

// Tile of the main kernel: ROUNDS rounds of R bags (R = lane groups per wavefront).
template <typename TT, int LANES, int VPL>
struct TileShape {
  static constexpr int R = kWave / LANES;
  static constexpr int ROUNDS = kRounds * R <= kWave ? kRounds : kWave / R;
  static constexpr int NB = R * ROUNDS;  // bags per tile
};

template <int NB>
struct TileLds {
  unsigned int ids[kWave];  // row ids of the current chunk, LANES per subgroup
  int order[NB];            // tile bags by rank: short bags, longest first
  int len[NB];
  int64_t start[NB];
};

template <typename TT, int LANES, int VPL>
using TileLdsOf = TileLds<TileShape<TT, LANES, VPL>::NB>;

// One tile of NB consecutive bags of one field, pooled by one wavefront:
//   short (L <= sub_threshold): one subgroup per bag, rows in element order. The short bags are
//     ranked by length and taken R at a time, longest first, so the R bags pooled side by side
//     need about the same number of steps;
//   medium (sub_threshold < L <= block_threshold): the whole wavefront, one bag at a time;
//   long (L > block_threshold): left to the long kernel.
// A chunk of LANES row ids per subgroup is loaded once (one lane per id, coalesced), clamped, and
// broadcast through the wavefront's LDS slice; each step then issues U row loads per lane.
template <typename TT, typename OT, int LANES, int VPL, bool BUF>
__device__ __forceinline__ void pool_tile(const PoolParams& p, int fi, int local_tile, TileLdsOf<TT, LANES, VPL>& s) {
  using S = Shape<TT, LANES, VPL>;
  constexpr int U = S::U;
  constexpr int R = S::R;
  constexpr int NB = TileShape<TT, LANES, VPL>::NB;
  const char* const table = p.f[fi].table;
  const int64_t max_row = p.f[fi].max_row;
  const int64_t row_bytes = p.f[fi].row_bytes;
  const int gidx = p.f[fi].gidx;
  const int out_col = p.f[fi].out_col;
  const float* const row_scale = p.f[fi].row_scale;
  const Rsrc rsrc = make_rsrc(table, BUF ? p.f[fi].span_bytes : 0u);
  // int8 tables: the row scales, read alongside the rows (out-of-range offsets read as 0)
  const Rsrc srsrc = make_rsrc(reinterpret_cast<const char*>(row_scale),
                               BUF && Quantized<TT>::value ? static_cast<uint32_t>((max_row + 1) * 4) : 0u);
  const unsigned int shift = static_cast<unsigned int>(__builtin_ctzll(static_cast<unsigned long long>(row_bytes)));
  // Row id staged for the slots past a bag's end: its row offset (2^32 - row_bytes, plus the
  // lane's column offset) and its scale offset both lie past the buffers' ends (the host admits
  // a table to the buffer path only if (rows + 1) * row_bytes <= 2^32), so those loads return
  // zeros without a memory request and the steps need no per-row test.
  const unsigned int r_pad = BUF ? 0xffffffffu >> shift : 0u;

  const int lane = lane_id();
  const int g = lane / LANES;   // subgroup inside the wavefront
  const int sl = lane % LANES;  // lane inside the subgroup
  const int64_t b0 = static_cast<int64_t>(local_tile) * NB;

  // Lane i describes bag b0 + i.
  const bool valid = lane < NB && b0 + lane < p.batch;
  int64_t start = 0, end = 0;
  if (valid) bag_range(p, gidx, b0 + lane, start, end);
  const int64_t L = end - start;
  const bool shortb = valid && L <= p.sub_threshold;  // empty bags too; sub_threshold < 2^24 (host)
  const bool medium = valid && L > p.sub_threshold && L <= p.block_threshold;
  const int n_short = __popcll(__ballot(shortb));
  // rank among the short bags: longer first, ties by position
  const int key = shortb ? static_cast<int>(L) : -1;
  int rank = 0;
  // unrolled by at most 8: each unrolled readlane holds a scalar register, and 32 or 64 of them
  // (tiles of narrow rows) would cap the wavefronts per SIMD by scalar registers
  constexpr int kRankUnroll = NB < 8 ? NB : 8;
#pragma unroll kRankUnroll
  for (int j = 0; j < NB; ++j) {
    const int kj = __builtin_amdgcn_readlane(key, j);
    rank += (kj > key || (kj == key && j < lane)) ? 1 : 0;
  }
  if (shortb) {
    s.order[rank] = lane;
    s.len[lane] = static_cast<int>(L);
    s.start[lane] = start;
  }
  __syncthreads();  // one wavefront per workgroup: orders the bag table before other lanes read it

  for (int r0 = 0; r0 < n_short; r0 += R) {
    const int slot = r0 + g;
    const bool has = slot < n_short;
    const int bi = has ? s.order[slot] : 0;
    const int Lb = has ? s.len[bi] : 0;
    const int64_t bs = has ? s.start[bi] : 0;
    float acc[S::NACC];
#pragma unroll
    for (int i = 0; i < S::NACC; ++i) acc[i] = 0.f;
    int64_t next_id = sl < Lb ? load_index(p, bs + sl) : 0;
    for (int c = 0; __ballot(c < Lb) != 0; c += LANES) {
      // this chunk's id was loaded one chunk ahead; the next chunk's id load is issued now, so
      // it completes under this chunk's row loads instead of costing its own round trip
      const int64_t id = next_id;
      if (c + LANES + sl < Lb) next_id = load_index(p, bs + c + LANES + sl);
      __syncthreads();  // orders this chunk's LDS writes after the last reads
      s.ids[lane] = c + sl < Lb ? static_cast<unsigned int>(clamp_i64(id, 0, max_row)) : r_pad;
      __syncthreads();
      const int live = Lb - c < LANES ? Lb - c : LANES;
      for (int k = 0; k < LANES; k += U) {
        if (__ballot(k < live) == 0) break;
        uint4 v[U][VPL];
        float sc[U];
        if constexpr (BUF) {
          // all U ids first, then branch-free loads (slots past the bag's end hold r_pad)
          unsigned int r[U];
#pragma unroll
          for (int u = 0; u < U; ++u) r[u] = s.ids[g * LANES + k + u];
          const unsigned int lane_off = static_cast<unsigned int>(sl * S::VB);
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const unsigned int o = (r[u] << shift) + lane_off;
#pragma unroll
            for (int q = 0; q < VPL; ++q) v[u][q] = buffer_load_vec<TT>(rsrc, o + q * LANES * S::VB);
            sc[u] = 1.f;
            if constexpr (Quantized<TT>::value) sc[u] = buffer_load_f32(srsrc, r[u] * 4u);
          }
          __builtin_amdgcn_sched_barrier(0);  // issue every load of the step before consuming any
        } else {
          load_step<TT, LANES, VPL>(table, row_scale, row_bytes, s.ids + g * LANES, sl, k, live, v, sc);
        }
        add_step<TT, LANES, VPL>(acc, v, sc);
      }
    }
    if (has) store_bag<TT, OT, LANES, VPL>(p, b0 + bi, out_col, Lb, acc);
  }

  for (uint64_t m = __ballot(medium); m;) {
    const int src = __ffsll(static_cast<long long>(m)) - 1;  // the bag's lane
    m &= m - 1;
    const int64_t bs = shfl_i64(start, src), be = shfl_i64(end, src);
    float pa[S::NACC];
#pragma unroll
    for (int i = 0; i < S::NACC; ++i) pa[i] = 0.f;
    __syncthreads();
    wave_slice_partial<TT, LANES, VPL>(p, table, row_scale, max_row, row_bytes, bs, be, pa, s.ids);
    if (g == 0) store_bag<TT, OT, LANES, VPL>(p, b0 + src, out_col, be - bs, pa);
  }
}

// ---------------------------------------------------------------------------------------------
// Streamed tile. A tile's bags are consecutive bags of one field, so with well-formed offsets
// their rows are one contiguous run of `values`. Here the whole wavefront walks the tile's rows in
// order, one 256-byte row per load instruction (each lane holds 4 bytes of every row), keeping K
// row loads in flight across bag boundaries: after it adds row r it issues row r + K into the
// same registers. A bag's sum is finished (and stored) when its last row has been added, so every
// bag is a sequential fp32 sum in element order, whatever its length. Row ids go one 64-row chunk
// at a time through a lane vector and are broadcast with readlane; the chunk after the current
// one is in flight meanwhile. Bags that are not one run (malformed offsets) are walked the same
// way, walk rows mapped to `values` positions by a search over the bags' ends.
// ---------------------------------------------------------------------------------------------
// The elements of a row that one 32-bit word holds (one fp32, or two bf16 / fp16), added in
// element order.
template <typename TT>
__device__ __forceinline__ void acc_word(float* a, uint32_t w) {
  if constexpr (__is_same(TT, float)) {
    a[0] += __uint_as_float(w);
  } else if constexpr (__is_same(TT, bf16_t)) {
    a[0] += __uint_as_float(w << 16);
    a[1] += __uint_as_float(w & 0xffff0000u);
  } else {
    a[0] += f16_bits_to_f32(w & 0xffffu);
    a[1] += f16_bits_to_f32(w >> 16);
  }
}

// E = 1 or 2 output elements of one lane (aligned to E * sizeof(OT) bytes); STREAM: non-temporal.
template <typename OT, int E, bool STREAM>
__device__ __forceinline__ void store_lane(OT* dst, const float* a) {
  if constexpr (E == 1) {
    if constexpr (sizeof(OT) == 4) put_as<STREAM>(reinterpret_cast<float*>(dst), a[0]);
    else if constexpr (__is_same(OT, bf16_t))
      put_as<STREAM>(reinterpret_cast<uint16_t*>(dst), static_cast<uint16_t>(pack_bf16x2(a[0], 0.f)));
    else put_as<STREAM>(reinterpret_cast<uint16_t*>(dst), static_cast<uint16_t>(f32_to_f16_bits(a[0])));
  } else if constexpr (sizeof(OT) == 4) {
    static_assert(E == 2, "two fp32 values");
    const u32x2 v = {__float_as_uint(a[0]), __float_as_uint(a[1])};
    put_as<STREAM>(reinterpret_cast<u32x2*>(dst), v);
  } else if constexpr (__is_same(OT, bf16_t)) {
    static_assert(E == 2, "two 16-bit values");
    put_as<STREAM>(reinterpret_cast<uint32_t*>(dst), pack_bf16x2(a[0], a[1]));
  } else {
    static_assert(E == 2, "two 16-bit values");
    put_as<STREAM>(reinterpret_cast<uint32_t*>(dst), pack_f16x2(a[0], a[1]));
  }
}

// Streamed tiles serve rows of 16 lane vectors read with buffer loads: 256-byte rows of fp32 / bf16
// / fp16 tables (4 bytes per lane) and 128-byte rows of int8 tables (2 bytes per lane, each row's
// scale read with it).
template <typename TT, int LANES, int VPL>
struct StreamShape {
  static constexpr bool ok = LANES == 16 && VPL == 1;
  static constexpr int BPL = LANES * Elem<TT>::kVecBytes / kWave;  // bytes of a row per lane
  static constexpr int K = 16;  // rows in flight: 16 VGPRs of row data (and 16 of scales)
};

// The BPL bytes of one lane's part of a row (loaded zero-extended into 32 bits) into the
// accumulators: fp32 / bf16 / fp16 as acc_word; int8 bytes as fma(q, s, acc) in element order.
template <typename TT, int BPL>
__device__ __forceinline__ void acc_lane(float* a, uint32_t w, float s) {
  if constexpr (Quantized<TT>::value) {
#pragma unroll
    for (int k = 0; k < BPL; ++k)
      a[k] = __builtin_fmaf(static_cast<float>(static_cast<int8_t>(w >> (8 * k))), s, a[k]);
  } else {
    static_assert(BPL == 4, "one 32-bit word of a 256-byte row");
    acc_word<TT>(a, w);
  }
}
template <int BPL>
__device__ __forceinline__ uint32_t load_lane(Rsrc r, unsigned int off) {
  if constexpr (BPL == 2) return static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
  else return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

// Raw ids of one 64-row chunk (one per lane), as loaded: converted only when the chunk is used,
// so the load stays in flight meanwhile.
template <typename IT>
struct RawIds;
template <>
struct RawIds<int32_t> {
  uint32_t lo;
  __device__ __forceinline__ void load(Rsrc r, unsigned int off) { lo = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0); }
  __device__ __forceinline__ int64_t value() const { return static_cast<int64_t>(static_cast<int32_t>(lo)); }
};
template <>
struct RawIds<int64_t> {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  u32x2 w;  // one register pair, as the 8-byte load writes it
  __device__ __forceinline__ void load(Rsrc r, unsigned int off) { w = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0); }
  __device__ __forceinline__ int64_t value() const { return static_cast<int64_t>(__builtin_bit_cast(uint64_t, w)); }
};

// Walks the rows of nb <= NB bags in order, bag after bag: lane i < nb describes bag i, the rows
// values[start, end). Each lane holds 4 bytes of every 256-byte row (read through `rsrc`, `shift`
// = log2 of the row stride); K row loads stay in flight across bag boundaries. When the last row
// of bag i has been added (at once for an empty bag) it calls store(i, r) with the bag's
// E = 4 / sizeof(TT) results of this lane (divided by the length for mean pooling), i rising.
// Walk rows are counted in 32 bits: the bags hold fewer than 2^31 rows in all (host).
template <typename TT, typename IT, int K, int NB, int BPL, typename Store>
__device__ __forceinline__ void stream_walk(const PoolParams& p, Rsrc rsrc, Rsrc srsrc, unsigned int shift,
                                            int64_t max_row, int nb, int64_t start, int64_t end, Store&& store) {
  static_assert(kWave % K == 0 && K <= kWave, "K divides the 64-row id chunk");
  static_assert(NB <= kWave, "one lane per bag");
  constexpr bool Q = Quantized<TT>::value;
  constexpr int E = BPL / Elem<TT>::kBytes;  // elements per lane and row
  const int lane = lane_id();
  const bool valid = lane < nb;
  if (nb <= 0) return;
  // Lane i < nb holds bag i's end in walk rows. With well-formed offsets (consecutive bags of one
  // field) bag i ends where bag i + 1 starts, walk row t is values[s0 + t] and bag i ends at
  // end_i - s0; otherwise the ends are the prefix sums of the lengths.
  const int64_t next_start = shfl_i64(start, lane + 1 < kWave ? lane + 1 : lane);
  const bool contiguous = __ballot(valid && lane < nb - 1 && end != next_start) == 0;
  const int64_t s0 = shfl_i64(start, 0);
  const int len = valid ? static_cast<int>(end - start) : 0;
  // mean pooling: lane i holds bag i's 1 / L (fp64, correctly rounded) and L (fp32), computed for
  // all the tile's bags at once; a bag's flush reads its pair with readlane (L there is this len)
  const bool mean = p.pooling == CTI_EBAG_MEAN;
  double inv_lane = 0.0;
  float len_f = 1.f;
  if (mean && len > 0) {
    inv_lane = 1.0 / static_cast<double>(len);
    len_f = static_cast<float>(len);
  }
  int cend = static_cast<int>(end - s0);
  if (!contiguous) {
    cend = len;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int t = shfl_i32(cend, lane >= d ? lane - d : lane);
      if (lane >= d) cend += t;
    }
  }
  const int T = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(cend, nb - 1));
  const int rel_end = valid ? cend : INT32_MAX;
  const int rel_start = cend - len;

  // Row ids through a buffer over `values` (the host admits nnz * sizeof(IT) < 2^32): positions
  // past nnz read as 0 without a memory request.
  const uint64_t vbase = reinterpret_cast<uint64_t>(p.values);
  const Rsrc vrsrc = make_rsrc(
      reinterpret_cast<const char*>(
          (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(vbase >> 32)))) << 32) |
          static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(vbase)))),
      static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(p.nnz * static_cast<int64_t>(sizeof(IT))))));
  // chunk of walk rows row0 .. row0 + 63 (row0 % 64 == 0), one per lane; lanes past the walk
  // request nothing (their ids are replaced by the pad id when the chunk is used)
  auto load_chunk = [&](RawIds<IT>& raw, int row0) {
    const int t = row0 + lane;
    int64_t at;
    if (contiguous) {
      at = s0 + t;
    } else {  // find the bag of walk row t
      int b = 0;
#pragma unroll
      for (int i = 0; i < NB; ++i) b += t >= __builtin_amdgcn_readlane(rel_end, i) ? 1 : 0;
      b = b < nb ? b : nb - 1;
      at = shfl_i64(start, b) + (t - shfl_i32(rel_start, b));
    }
    raw.load(vrsrc, t < T && at < p.nnz ? static_cast<unsigned int>(at * static_cast<int64_t>(sizeof(IT))) : 0xffffffffu);
  };

  const unsigned int r_pad = 0xffffffffu >> shift;  // offsets past the table: zeros, no request
  const unsigned int lane_off = static_cast<unsigned int>(lane * BPL);
  // int8 rows: a row's scale offset is its row offset >> (shift - 2) (past the scales for the pad
  // rows, whose row offsets lie past the table: the host admits only (rows + 1) * row_bytes <= 2^32)
  const unsigned int sshift = shift - 2;

  // clamped row ids of the chunk being issued; the next chunk's raw ids are in flight meanwhile
  RawIds<IT> raw, raw_next;
  load_chunk(raw, 0);
  load_chunk(raw_next, kWave);
  unsigned int ids = (lane < T ? static_cast<unsigned int>(clamp_i64(raw.value(), 0, max_row)) : r_pad) << shift;
  // int8 rows: the scales of a chunk's rows, one per lane, loaded when the chunk's ids are taken
  // (pad rows read zeros past the scales); a row's scale is read with readlane when it is added.
  // sc_issue: the chunk being issued; sc_add: the chunk of the rows being added (the previous
  // one for a step, after the issue has moved on to a new chunk)
  float sc_issue = 0.f, sc_add = 0.f;
  if constexpr (Q) {
    sc_issue = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(srsrc, ids >> sshift, 0, 0));
    sc_add = sc_issue;
  }

  uint32_t v[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const unsigned int r = static_cast<unsigned int>(__builtin_amdgcn_readlane(static_cast<int>(ids), k));
    v[k] = load_lane<BPL>(rsrc, r + lane_off);
  }

  float acc[E];
#pragma unroll
  for (int i = 0; i < E; ++i) acc[i] = 0.f;
  int bag = 0, prev_end = 0;
  int next_end = __builtin_amdgcn_readlane(rel_end, 0);
  // Finish the bag(s) ending at walk row `row_end` (bags of zero rows included).
  auto flush = [&](int row_end) {
    do {
      const int L = next_end - prev_end;
      float r[E];
#pragma unroll
      for (int i = 0; i < E; ++i) r[i] = acc[i];
      if (mean && L > 0) {
        const uint64_t iv = __builtin_bit_cast(uint64_t, inv_lane);
        const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(iv), bag));
        const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(iv >> 32), bag));
        const float fl = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, len_f), bag));
        div_by_count<E>(r, __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo), fl);
      }
      round_like_reference<TT, E>(p, r);
      store(bag, r);
#pragma unroll
      for (int i = 0; i < E; ++i) acc[i] = 0.f;
      prev_end = next_end;
      ++bag;
      next_end = bag < nb ? __builtin_amdgcn_readlane(rel_end, bag) : INT32_MAX;
    } while (next_end == row_end);
  };
  if (next_end == 0) flush(0);

  // Full steps: rows j .. j + K - 1 are added and rows j + K .. j + 2K - 1 issued (past the walk:
  // pad offsets, no request). The partial last step is outside the loop, so the loop carries the
  // row window in place (no register copies, which would wait for every load in flight).
  int j = 0;
  for (; j + K <= T; j += K) {
    const int c_issue = (j + K) & (kWave - 1);  // lane of walk row j + K in its id chunk
    const int c_add = j & (kWave - 1);          // lane of walk row j in its id chunk
    if constexpr (Q) {
      if (c_add == 0) sc_add = sc_issue;  // the rows added now are in the chunk issued since
    }
    if (c_issue == 0) {
      // rows j + K .. are in the next chunk: take it, and load the one after it
      ids = (j + K + lane < T ? static_cast<unsigned int>(clamp_i64(raw_next.value(), 0, max_row)) : r_pad) << shift;
      load_chunk(raw_next, j + K + kWave);
      if constexpr (Q) sc_issue = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(srsrc, ids >> sshift, 0, 0));
    }
    int dn = next_end - j - 1;  // step row after which the next bag ends
    unsigned int roff[K];       // this step's row offsets, uniform (scalar registers)
#pragma unroll
    for (int k = 0; k < K; ++k)
      roff[k] = static_cast<unsigned int>(__builtin_amdgcn_readlane(static_cast<int>(ids), c_issue + k));
#pragma unroll
    for (int k = 0; k < K; ++k) {
      float s = 0.f;
      if constexpr (Q) s = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc_add), c_add + k));
      acc_lane<TT, BPL>(acc, v[k], s);
      if (k == dn) {
        flush(j + k + 1);
        dn = next_end - j - 1;
      }
      v[k] = load_lane<BPL>(rsrc, roff[k] + lane_off);
    }
  }
  if (j < T) {  // the partial last step: rows j .. T - 1, nothing issued
    const int c_add = j & (kWave - 1);
    if constexpr (Q) {
      if (c_add == 0) sc_add = sc_issue;
    }
    int dn = next_end - j - 1;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      if (j + k < T) {
        float s = 0.f;
        if constexpr (Q) s = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc_add), c_add + k));
        acc_lane<TT, BPL>(acc, v[k], s);
        if (k == dn) {
          flush(j + k + 1);
          dn = next_end - j - 1;
        }
      }
    }
  }
}

// A tile of NB consecutive bags of one field, streamed (see stream_walk); STREAM_OUT: the results
// are stored non-temporally (the host sets it for output blocks of kStreamOutBytes and more).
template <typename TT, typename OT, typename IT, int K, int NB, int BPL, bool STREAM_OUT>
__device__ __forceinline__ void pool_tile_stream(const PoolParams& p, int fi, int local_tile) {
  constexpr int E = BPL / Elem<TT>::kBytes;
  const int lane = lane_id();
  const int64_t b0 = static_cast<int64_t>(local_tile) * NB;
  const int nb = static_cast<int>(p.batch - b0 < NB ? p.batch - b0 : NB);
  int64_t start = 0, end = 0;
  if (lane < nb) bag_range(p, p.f[fi].gidx, b0 + lane, start, end);
  const Rsrc rsrc = make_rsrc(p.f[fi].table, p.f[fi].span_bytes);
  const Rsrc srsrc = make_rsrc(reinterpret_cast<const char*>(p.f[fi].row_scale),
                               Quantized<TT>::value ? static_cast<uint32_t>((p.f[fi].max_row + 1) * 4) : 0u);
  const unsigned int shift =
      static_cast<unsigned int>(__builtin_ctzll(static_cast<unsigned long long>(p.f[fi].row_bytes)));
  // bags are stored in order, each once: the destination advances by one output row per bag
  OT* dst = reinterpret_cast<OT*>(p.out) + b0 * p.out_row_stride + p.f[fi].out_col + lane * E;
  stream_walk<TT, IT, K, NB, BPL>(p, rsrc, srsrc, shift, p.f[fi].max_row, nb, start, end, [&](int, const float* r) {
    store_lane<OT, E, STREAM_OUT>(dst, r);
    dst += p.out_row_stride;
  });
}

__device__ __forceinline__ void bin_handoff(const PoolParams& p) {
  if (p.bin_count && blockIdx.x == 0 && threadIdx.x == 0) {
    // hand the finished list lengths to the list kernel and zero the counters for the next call
#pragma unroll
    for (int k = 0; k < 4; k += 2) {
      const unsigned int n = __hip_atomic_load(p.bin_count + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(p.bin_total + k, n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(p.bin_count + k, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Dispatch order. Workgroups are dealt to the XCDs round-robin and xcd_contiguous() gives XCD x
// a contiguous range of tile positions, which it starts in order as wavefront slots free up. A
// launch ends with a drain: tiles of long bags that start late run on while the rest of the chip
// idles. Starting each XCD's tiles with the most rows per bag first removes most of that drain.
// The order of a batch is made one launch ahead: a launch given `next_order` runs order_blocks
// extra workgroups at the first dispatch positions (a multiple of 8, so every tile keeps its
// XCD), each sorting one chunk of kOrderChunk tiles of one XCD range of the next batch by rows per
// bag while the rest of the launch pools; the next launch on the stream reads it as `tile_order`. Only the sequence of each XCD's
// tiles changes and each output row keeps one writer, so results do not depend on the order.
//
// Order buffer (int32): [0] tiles of the launch it was made for, [1] kOrderMagic, [2..3] zero,
// [kOrderHeader + position] = tile. A launch follows an order only if [0] and [1] match it, and
// takes its own position for any entry outside its tiles, so no buffer can make it read or write
// out of bounds; an order written here for any launch of as many tiles is a permutation of them.
// kOrderMagic, kOrderHeader, kOrderChunk (an XCD range is sorted in chunks of this many tiles)
// and kOrderBuckets (rows per bag 63, 62, ..., 0; more count as 63) are shared with the host
// builder (ebag_internal.h).
constexpr int kOrderUnroll = 8;     // tiles per lane whose offsets are loaded together
static_assert(kOrderBuckets == kWave, "one bucket per lane in the prefix sum");

struct OrderLds {
  unsigned char bucket[kOrderChunk];
  unsigned int next[kOrderBuckets];
};

__device__ __forceinline__ int ordered_tile(const PoolParams& p, int pos) {
  if (!p.tile_order) return pos;
  // the host checked that the buffer holds kOrderHeader + num_tiles entries
  const int32_t n = p.tile_order[0], magic = p.tile_order[1], t = p.tile_order[kOrderHeader + pos];
  return n == p.num_tiles && magic == kOrderMagic && t >= 0 && t < p.num_tiles ? t : pos;
}

// tile / tiles_per_field for 0 <= tile < 2^31 without a division: hi32(tile * tpf_inv) with
// tpf_inv = floor((2^32 - 1) / d) is the quotient or one less, and one compare corrects it.
__device__ __forceinline__ int field_of_tile(const PoolParams& p, int tile) {
  const unsigned int t = static_cast<unsigned int>(tile), d = static_cast<unsigned int>(p.tiles_per_field);
  unsigned int q = __umulhi(t, p.tpf_inv);
  if ((q + 1u) * d <= t) ++q;
  return static_cast<int>(q);
}

// Rows of tile t (NB consecutive bags of one field) in the next batch, from its offsets alone. A
// launch that makes an order holds every field of its job in job order (the host checks it), so
// field fi's offsets start at fi * offsets_stride: no dependent load of the field's index, which
// would make each tile's offset loads wait for the previous tile's (loads complete in order).
__device__ __forceinline__ int64_t next_tile_rows(const PoolParams& p, int t, int nb) {
  const int fi = field_of_tile(p, t);
  const int64_t b0 = static_cast<int64_t>(t - fi * p.tiles_per_field) * nb;
  const int64_t b1 = b0 + nb < p.batch ? b0 + nb : p.batch;
  const int64_t i = static_cast<int64_t>(fi) * p.offsets_stride;
  return load_offset(p, p.next_offsets, i + b1) - load_offset(p, p.next_offsets, i + b0);  // val_base cancels
}

// One wavefront sorts chunk `chunk` of XCD range x of the next batch's tiles, most rows per bag
// first: a counting sort whose bucket of each tile is computed once and kept in LDS, so the
// positions it hands out are a permutation of the chunk whatever the offsets hold (the order
// inside a bucket is whatever the LDS atomics give).
template <int NB>
__device__ void order_next(const PoolParams& p, int x, int chunk, OrderLds& s) {
  const int n = p.num_tiles;
  const int q = n >> 3, r = n & 7;
  const int lo = x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q;
  const int cnt = q + (x < r ? 1 : 0);
  const int lane = lane_id();
  int32_t* const order = p.next_order + kOrderHeader;
  const int c0 = chunk * kOrderChunk;
  if (c0 < cnt) {
    const int m = cnt - c0 < kOrderChunk ? cnt - c0 : kOrderChunk;
    s.next[lane] = 0u;
    __syncthreads();
    for (int k0 = 0; k0 < m; k0 += kOrderUnroll * kWave) {
      int64_t rows[kOrderUnroll];
#pragma unroll
      for (int u = 0; u < kOrderUnroll; ++u) {
        const int k = k0 + u * kWave + lane;
        rows[u] = k < m ? next_tile_rows(p, lo + c0 + k, NB) : 0;
      }
#pragma unroll
      for (int u = 0; u < kOrderUnroll; ++u) {
        const int k = k0 + u * kWave + lane;
        if (k < m) {
          int64_t per_bag = rows[u] / NB;
          per_bag = per_bag < 0 ? 0 : (per_bag > kOrderBuckets - 1 ? kOrderBuckets - 1 : per_bag);
          const int b = kOrderBuckets - 1 - static_cast<int>(per_bag);
          s.bucket[k] = static_cast<unsigned char>(b);
          atomicAdd(&s.next[b], 1u);
        }
      }
    }
    __syncthreads();
    // exclusive prefix sum of the bucket counts, bucket = lane
    const unsigned int c = s.next[lane];
    unsigned int incl = c;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const unsigned int v = __shfl_up(incl, d);
      if (lane >= d) incl += v;
    }
    s.next[lane] = incl - c;
    __syncthreads();
    for (int k0 = 0; k0 < m; k0 += kOrderUnroll * kWave) {
      unsigned int at[kOrderUnroll];
#pragma unroll
      for (int u = 0; u < kOrderUnroll; ++u) {
        const int k = k0 + u * kWave + lane;
        at[u] = k < m ? atomicAdd(&s.next[s.bucket[k]], 1u) : 0u;  // in [0, m)
      }
#pragma unroll
      for (int u = 0; u < kOrderUnroll; ++u) {
        const int k = k0 + u * kWave + lane;
        if (k < m) order[lo + c0 + static_cast<int>(at[u])] = lo + c0 + k;
      }
    }
  }
  if (x == 0 && chunk == 0 && lane == 0) {
    p.next_order[0] = n;
    p.next_order[1] = kOrderMagic;
    p.next_order[2] = 0;
    p.next_order[3] = 0;
  }
}

// Main kernel: one wavefront per workgroup, one tile per workgroup (after the order workgroups,
// when the launch makes the next batch's order).
// Main kernel forms: tiles pooled by pool_tile, or streamed with int32 / int64 ids, the results
// stored plainly or (the Nt forms) non-temporally.
enum TileForm : int { kTileRanked = 0, kTileStream32 = 1, kTileStream64 = 2, kTileStream32Nt = 3, kTileStream64Nt = 4 };

template <typename TT, typename OT, int LANES, int VPL, bool BUF, int FORM>
__global__ void __launch_bounds__(kMainThreads) pool_kernel(const PoolParams p) {
  __shared__ union {
    TileLdsOf<TT, LANES, VPL> tile;
    OrderLds order;
  } s;
  bin_handoff(p);
  int pos = static_cast<int>(blockIdx.x);
  if (p.next_order) {
    if (pos < p.order_blocks) {
      order_next<TileShape<TT, LANES, VPL>::NB>(p, pos & 7, pos >> 3, s.order);
      return;
    }
    pos -= p.order_blocks;
  }
  const int tile = ordered_tile(p, xcd_position(pos, p.num_tiles));
  const int fi = field_of_tile(p, tile);
  if constexpr (FORM != kTileRanked) {
    using Stream = StreamShape<TT, LANES, VPL>;
    static_assert(BUF && Stream::ok, "streamed tiles need buffer loads and rows of 16 lane vectors");
    using IT = typename std::conditional<FORM == kTileStream32 || FORM == kTileStream32Nt, int32_t, int64_t>::type;
    constexpr bool kNt = FORM == kTileStream32Nt || FORM == kTileStream64Nt;
    pool_tile_stream<TT, OT, IT, Stream::K, TileShape<TT, LANES, VPL>::NB, Stream::BPL, kNt>(p, fi,
                                                                                           tile - fi * p.tiles_per_field);
  } else {
    pool_tile<TT, OT, LANES, VPL, BUF>(p, fi, tile - fi * p.tiles_per_field, s.tile);
  }
}

// Main kernel of a mixed-width launch: the fields' rows differ in width but each is one lane
// vector per lane (LANES = 1 << lanes_log2). Fields own consecutive ranges of tiles; a workgroup
// finds its tile's field (one compare per lane and a ballot) and runs that width's tile code, so
// fields of every width share one launch (and one binning pass and one list kernel).
template <typename TT, typename OT, bool BUF>
__global__ void __launch_bounds__(kMainThreads) pool_mixed_kernel(const PoolParams p) {
  __shared__ union {
    TileLdsOf<TT, 4, 1> l2;
    TileLdsOf<TT, 8, 1> l3;
    TileLdsOf<TT, 16, 1> l4;
    TileLdsOf<TT, 32, 1> l5;
    TileLdsOf<TT, 64, 1> l6;
  } s;
  bin_handoff(p);
  const int tile = block_tile();
  const int lane = lane_id();
  const int first = lane < p.num_fields ? p.f[lane].tile_begin : INT32_MAX;
  const int fi = __popcll(__ballot(first <= tile)) - 1;  // field 0 starts at tile 0
  const int local = tile - p.f[fi].tile_begin;
  switch (p.f[fi].lanes_log2) {
    case 2: pool_tile<TT, OT, 4, 1, BUF>(p, fi, local, s.l2); break;
    case 3: pool_tile<TT, OT, 8, 1, BUF>(p, fi, local, s.l3); break;
    case 4: pool_tile<TT, OT, 16, 1, BUF>(p, fi, local, s.l4); break;
    case 5: pool_tile<TT, OT, 32, 1, BUF>(p, fi, local, s.l5); break;
    default: pool_tile<TT, OT, 64, 1, BUF>(p, fi, local, s.l6); break;
  }
}

// ---------------------------------------------------------------------------------------------
// Pooling with the input LayerNorm fused into the writer (online_best/infer.py:1050-1076): one
// workgroup owns whole output rows, so the pooled row never goes to HBM before normalisation.
// One shared table (the reference's single nn.Embedding), uniform row width, one row vector per
// lane. The workgroup's bags (its samples x all fields) are dealt to its W wavefronts by length,
// so that each gets a like share; a wavefront pools its bags exactly as the main kernel pools a
// tile (length-ranked rounds, one lane group per short bag in element order, the whole
// wavefront for longer bags) and writes each result, rounded to the output type, into an LDS
// copy of the rows; the workgroup then normalises the rows (fp32 mean and variance, fixed
// reduction order) and stores each once.
constexpr int kFusedBags = kWave;  // samples per workgroup * fields <= 64: one lane per bag

// Wavefronts per fused workgroup for rows of `lanes` lanes (one 16-byte vector per lane).
// Measured (reference shape: 28 slots of 1 KiB rows, B = 4096; bf16-2m shape: 256-byte rows):
// 1 KiB rows 4 / 8 / 16 wavefronts 162.5 / 149.3 / 176.2 us; 256-byte rows 4 / 8: 40.7 / 50.8 us.
constexpr int fused_waves(int lanes) { return lanes >= 64 ? 8 : 4; }

struct FusedLds {  // one per wavefront
  unsigned int ids[kWave];
  int order[kFusedBags / 4];  // this wavefront's short bags in list order (at most 64 / 4 per wavefront)
  int len[kFusedBags];
  int64_t start[kFusedBags];
};

struct FusedNorm {
  const void* gamma;
  const void* beta;
  float eps;
};

// Orders this wavefront's LDS accesses (its lanes exchange row ids through LDS); the four
// wavefronts of a fused workgroup pool independently, so no workgroup barrier is used here.
__device__ __forceinline__ void wave_sync() { __builtin_amdgcn_wave_barrier(); }

template <typename TT, typename PT, int LANES, int SPW, bool BUF, int W = fused_waves(LANES)>
__global__ void __launch_bounds__(W * kWave) pool_norm_kernel(const PoolParams p, const FusedNorm fn) {
  using S = Shape<TT, LANES, 1>;
  constexpr int U = S::U;
  constexpr int R = S::R;
  static_assert(W >= 4, "a wavefront's list of short bags holds at most kFusedBags / 4 entries");
  extern __shared__ uint4 s_row_raw[];  // the output rows: SPW * F * D elements of TT
  __shared__ FusedLds s_w[W];
  __shared__ float s_red[W * SPW];
  TT* const row = reinterpret_cast<TT*>(s_row_raw);

  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  const int g = lane / LANES, sl = lane % LANES;
  const int64_t b0 = static_cast<int64_t>(block_tile()) * SPW;  // XCD x pools a contiguous sample range
  const int F = p.num_fields;
  const int D = p.f[0].dim;
  const char* const table = p.f[0].table;
  const int64_t max_row = p.f[0].max_row;
  const int64_t row_bytes = p.f[0].row_bytes;
  const Rsrc rsrc = make_rsrc(table, BUF ? p.f[0].span_bytes : 0u);
  const unsigned int shift = static_cast<unsigned int>(__builtin_ctzll(static_cast<unsigned long long>(row_bytes)));
  const unsigned int r_pad = BUF ? 0xffffffffu >> shift : 0u;
  FusedLds& s = s_w[wave];

  // Every wavefront describes all SPW * F bags of the workgroup, bag i on lane i (sample b0 + i / F,
  // field i % F; its pooled row goes to LDS row position i), ranks them by length (longest first,
  // ties by position) and keeps the ranks dealt to it: rank r goes to wavefront r % W when r / W
  // is even, W - 1 - r % W when odd, at position r / W of that wavefront's list. So each wavefront
  // gets a like share of the long and of the short bags and the workgroup's slowest wavefront (the
  // one the LayerNorm waits for) has about the average load. Each bag is pooled exactly as before
  // (one lane group in element order, or the whole wavefront above sub_threshold), so the pooled
  // rows do not depend on who pools them. Bags above sub_threshold have the first ranks, so they
  // come first in every list.
  const int nb = SPW * F;  // <= kFusedBags (host)
  bool valid = lane < nb;
  int64_t start = 0, end = 0;
  if (valid) {
    const int64_t bb = b0 + lane / F;
    valid = bb < p.batch;
    if (valid) bag_range(p, p.f[lane % F].gidx, bb, start, end);
  }
  const int64_t L = end - start;
  const int key = valid ? static_cast<int>(L < INT32_MAX ? L : INT32_MAX) : -1;
  int rank = 0;
  // unrolled by 8 only: each unrolled readlane holds a scalar register
#pragma unroll 8
  for (int j = 0; j < kFusedBags; ++j) {
    const int kj = __builtin_amdgcn_readlane(key, j);
    rank += (kj > key || (kj == key && j < lane)) ? 1 : 0;
  }
  const int rd = rank / W, rm = rank - rd * W;
  const bool mine = valid && ((rd & 1) ? W - 1 - rm : rm) == wave;
  const bool medium = mine && L > p.sub_threshold;
  const bool shortb = mine && L <= p.sub_threshold;
  const int n_medium = __popcll(__ballot(medium));
  const int n_short = __popcll(__ballot(shortb));
  if (shortb) {
    s.order[rd - n_medium] = lane;
    s.len[lane] = static_cast<int>(L);
    s.start[lane] = start;
  }
  wave_sync();

  auto write_row = [&](int bag, int64_t Lb, float* a) {
    float r[S::NACC];
#pragma unroll
    for (int i = 0; i < S::NACC; ++i) r[i] = a[i];
    if (p.pooling == CTI_EBAG_MEAN && Lb > 0)
      div_by_count<S::NACC>(r, 1.0 / static_cast<double>(Lb), static_cast<float>(Lb));
    store_out<S::VEC>(row + static_cast<int64_t>(bag) * D + sl * S::VEC, r, false);  // LDS row
  };

  for (int r0 = 0; r0 < n_short; r0 += R) {
    const int slot = r0 + g;
    const bool has = slot < n_short;
    const int bi = has ? s.order[slot] : 0;
    const int Lb = has ? s.len[bi] : 0;
    const int64_t bs = has ? s.start[bi] : 0;
    float acc[S::NACC];
#pragma unroll
    for (int i = 0; i < S::NACC; ++i) acc[i] = 0.f;
    // No id prefetch here (unlike pool_tile): its extra registers take this kernel from 63 to 67
    // VGPRs, one wavefront less per SIMD, and the launch from 41.9 to 49.3 us on bf16-2m.
    for (int c = 0; __ballot(c < Lb) != 0; c += LANES) {
      wave_sync();  // this chunk's LDS writes come after the last chunk's reads
      s.ids[lane] = c + sl < Lb ? static_cast<unsigned int>(clamp_i64(load_index(p, bs + c + sl), 0, max_row)) : r_pad;
      wave_sync();
      const int live = Lb - c < LANES ? Lb - c : LANES;
      for (int k = 0; k < LANES; k += U) {
        if (__ballot(k < live) == 0) break;
        uint4 v[U][1];
        float sc[U];
        if constexpr (BUF) {
          unsigned int r[U];
#pragma unroll
          for (int u = 0; u < U; ++u) r[u] = s.ids[g * LANES + k + u];
          const unsigned int lane_off = static_cast<unsigned int>(sl * S::VB);
#pragma unroll
          for (int u = 0; u < U; ++u) {
            v[u][0] = buffer_load_vec<TT>(rsrc, (r[u] << shift) + lane_off);
            sc[u] = 1.f;
          }
          __builtin_amdgcn_sched_barrier(0);  // issue every load of the step before consuming any
        } else {
          load_step<TT, LANES, 1>(table, nullptr, row_bytes, s.ids + g * LANES, sl, k, live, v, sc);
        }
        add_step<TT, LANES, 1>(acc, v, sc);
      }
    }
    if (has) write_row(bi, Lb, acc);
  }
  for (uint64_t m = __ballot(medium); m;) {
    const int src = __ffsll(static_cast<long long>(m)) - 1;  // the bag's lane
    m &= m - 1;
    const int64_t bs = shfl_i64(start, src), be = shfl_i64(end, src);
    float pa[S::NACC];
#pragma unroll
    for (int i = 0; i < S::NACC; ++i) pa[i] = 0.f;
    wave_sync();
    wave_slice_partial<TT, LANES, 1>(p, table, nullptr, max_row, row_bytes, bs, be, pa, s.ids);
    if (g == 0) write_row(src, be - bs, pa);
  }
  __syncthreads();  // the whole rows are in LDS

  // LayerNorm of each row (online_best/infer.py:843-856): fp32 mean, fp32 variance of the
  // deviations, y = (x - mean) * rstd * gamma + beta rounded once to the output type. The rows
  // of the workgroup's samples share each gamma / beta load.
  constexpr int VEC = 16 / Elem<TT>::kBytes;
  const int cols = F * D;
  const int nvec = cols / VEC;
  const int t = static_cast<int>(threadIdx.x);
  constexpr int THREADS = W * kWave;
  const char* const rb = reinterpret_cast<const char*>(row);
  const int64_t rstride = static_cast<int64_t>(cols) * Elem<TT>::kBytes;
  const float n = static_cast<float>(cols);
  // the SPW rows' sums share one workgroup reduction, then their squared deviations share one
  // (taking the sums while the rows are written held 4 more VGPRs: 7 wavefronts per SIMD)
  float mean[SPW], rstd[SPW];
#pragma unroll
  for (int j = 0; j < SPW; ++j) {
    float sum = 0.f;
    for (int i = t; i < nvec; i += THREADS) {
      float x[VEC];
      unpack16(load16(rb + j * rstride + i * 16), x, TT{});
#pragma unroll
      for (int e = 0; e < VEC; ++e) sum += x[e];
    }
    mean[j] = sum;
  }
  block_sum_n<W, SPW>(mean, s_red);
#pragma unroll
  for (int j = 0; j < SPW; ++j) {
    mean[j] /= n;
    float q = 0.f;
    for (int i = t; i < nvec; i += THREADS) {
      float x[VEC];
      unpack16(load16(rb + j * rstride + i * 16), x, TT{});
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float d = x[e] - mean[j];
        q += d * d;
      }
    }
    rstd[j] = q;
  }
  block_sum_n<W, SPW>(rstd, s_red);
#pragma unroll
  for (int j = 0; j < SPW; ++j) rstd[j] = 1.0f / __builtin_sqrtf(rstd[j] / n + fn.eps);
  with_stream(p.stream_out, [&](auto stream) {
    for (int i = t; i < nvec; i += THREADS) {
      float gm[VEC], bt[VEC];
      load_params<PT, VEC>(fn.gamma, static_cast<int64_t>(i) * VEC, gm);
      load_params<PT, VEC>(fn.beta, static_cast<int64_t>(i) * VEC, bt);
#pragma unroll
      for (int j = 0; j < SPW; ++j) {
        if (b0 + j >= p.batch) break;
        float x[VEC], r[VEC];
        unpack16(load16(rb + j * rstride + i * 16), x, TT{});
#pragma unroll
        for (int e = 0; e < VEC; ++e) r[e] = (x[e] - mean[j]) * rstd[j] * gm[e] + bt[e];
        store_out<VEC>(reinterpret_cast<TT*>(p.out) + (b0 + j) * p.out_row_stride + static_cast<int64_t>(i) * VEC, r,
                       decltype(stream)::value);
      }
    }
  });
}

// Length-binning pass: list the bags longer than block_threshold, those longer than
// split_threshold on the split list. grid (ceil(B/256), fields). The workgroup's wavefronts
// combine their counts in LDS, so each list costs one global atomic per workgroup.
__global__ void __launch_bounds__(kBinThreads) bin_kernel(const PoolParams p, LongList l) {
  constexpr int kWaves = kBinThreads / kWave;
  __shared__ unsigned int s_cnt[2][kWaves];
  __shared__ unsigned int s_base[2];
  const int fi = static_cast<int>(blockIdx.y);
  const int64_t b = static_cast<int64_t>(blockIdx.x) * kBinThreads + threadIdx.x;
  bool one = false, split = false;
  int64_t s = 0, e = 0;
  if (b < p.batch) {
    bag_range(p, p.f[fi].gidx, b, s, e);
    split = e - s > p.split_threshold;
    one = !split && e - s > p.block_threshold;
  }
  const int lane = lane_id();
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const uint64_t m1 = __ballot(one), m2 = __ballot(split);
  if (lane == 0) {
    s_cnt[0][wave] = static_cast<unsigned int>(__popcll(m1));
    s_cnt[1][wave] = static_cast<unsigned int>(__popcll(m2));
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    unsigned int n = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) n += s_cnt[threadIdx.x][w];
    s_base[threadIdx.x] = n ? atomicAdd(threadIdx.x == 0 ? l.count : l.count2, n) : 0u;
  }
  __syncthreads();
  unsigned int before1 = 0, before2 = 0;  // entries of the lower wavefronts of this workgroup
  for (int w = 0; w < wave; ++w) {
    before1 += s_cnt[0][w];
    before2 += s_cnt[1][w];
  }
  const uint64_t below = (1ull << lane) - 1ull;
  const int64_t entry = (static_cast<int64_t>(fi) << 40) | b;
  int64_t at = -1;
  if (one) at = s_base[0] + before1 + __popcll(m1 & below);
  if (split) at = l.capacity - 1 - (s_base[1] + before2 + __popcll(m2 & below));
  if (at >= 0) {
    l.bags[at] = entry;
    l.starts[at] = s;
    l.ends[at] = e;
  }
}

// Wave-uniform copy of a value every lane holds (list entries are read by all lanes alike).
__device__ __forceinline__ int64_t uniform_i64(int64_t v) {
  const uint64_t u = static_cast<uint64_t>(v);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

constexpr int64_t kSampleMask = (int64_t{1} << 40) - 1;

// One wavefront's share of a bag on the split list: its contiguous slice of [bs, be), partial
// sums through LDS, combined by wavefront 0 in wavefront order. Every wavefront of the workgroup
// calls this for the same bag.
template <typename TT, typename OT, int LANES, int VPL, int LW>
__device__ __forceinline__ void split_bag(const PoolParams& p, int fi, int64_t b, int64_t bs, int64_t be, int wave,
                                          float* s_red, unsigned int* ids) {
  using S = Shape<TT, LANES, VPL>;
  const int sl = lane_id() % LANES;
  const bool g0 = lane_id() < LANES;
  const int64_t per = (be - bs + LW - 1) / LW;
  const int64_t s0 = bs + wave * per < be ? bs + wave * per : be;
  const int64_t s1 = s0 + per < be ? s0 + per : be;
  float pa[S::NACC];
#pragma unroll
  for (int i = 0; i < S::NACC; ++i) pa[i] = 0.f;
  wave_slice_partial<TT, LANES, VPL>(p, p.f[fi].table, p.f[fi].row_scale, p.f[fi].max_row, p.f[fi].row_bytes, s0, s1,
                                     pa, ids);
  if (g0) {
#pragma unroll
    for (int q = 0; q < VPL; ++q) {
#pragma unroll
      for (int i = 0; i < S::VEC; ++i) s_red[wave * S::D + (q * LANES + sl) * S::VEC + i] = pa[q * S::VEC + i];
    }
  }
  __syncthreads();
  if (wave == 0 && g0) {
    float r[S::NACC];
#pragma unroll
    for (int q = 0; q < VPL; ++q) {
#pragma unroll
      for (int i = 0; i < S::VEC; ++i) {
        const int col = (q * LANES + sl) * S::VEC + i;
        float x = s_red[col];
#pragma unroll
        for (int w = 1; w < LW; ++w) x += s_red[w * S::D + col];
        r[q * S::VEC + i] = x;
      }
    }
    store_bag<TT, OT, LANES, VPL>(p, b, p.f[fi].out_col, be - bs, r);
  }
  __syncthreads();
}

// A bag on the one-wavefront list: the whole wavefront, lane groups taking interleaved rows.
template <typename TT, typename OT, int LANES, int VPL>
__device__ __forceinline__ void one_wave_bag(const PoolParams& p, int fi, int64_t b, int64_t bs, int64_t be,
                                             unsigned int* ids) {
  using S = Shape<TT, LANES, VPL>;
  float pa[S::NACC];
#pragma unroll
  for (int i = 0; i < S::NACC; ++i) pa[i] = 0.f;
  wave_slice_partial<TT, LANES, VPL>(p, p.f[fi].table, p.f[fi].row_scale, p.f[fi].max_row, p.f[fi].row_bytes, bs, be,
                                     pa, ids);
  if (lane_id() < LANES) store_bag<TT, OT, LANES, VPL>(p, b, p.f[fi].out_col, be - bs, pa);
}

// Row shape of the list kernel: one shape for every field of the launch ...
template <typename TT, typename OT, int LANES, int VPL, int LW>
struct FixedRows {
  static constexpr int DMAX = Shape<TT, LANES, VPL>::D;
  __device__ static __forceinline__ void split(const PoolParams& p, int fi, int64_t b, int64_t bs, int64_t be,
                                               int wave, float* s_red, unsigned int* ids) {
    split_bag<TT, OT, LANES, VPL, LW>(p, fi, b, bs, be, wave, s_red, ids);
  }
  __device__ static __forceinline__ void one(const PoolParams& p, int fi, int64_t b, int64_t bs, int64_t be,
                                             unsigned int* ids) {
    one_wave_bag<TT, OT, LANES, VPL>(p, fi, b, bs, be, ids);
  }
};

// wave_slice_partial for a row shape known only at run time: 1 << ll lanes of one vector each
// (4 to 64 lanes), four rows in flight per lane group. Every lane holds the same registers
// whatever the shape (one vector's accumulators), so one code path serves all shapes. Element
// order and the combine's order equal wave_slice_partial<TT, 1 << ll, 1>, so results do too.
template <typename TT>
__device__ __forceinline__ void wave_slice_partial_rt(const PoolParams& p, int fi, int ll, int64_t s0, int64_t s1,
                                                      float* pa, unsigned int* ids) {
  constexpr int VB = Elem<TT>::kVecBytes;
  constexpr int VEC = VB / Elem<TT>::kBytes;
  constexpr int U = 4;
  const char* const table = p.f[fi].table;
  const float* const row_scale = p.f[fi].row_scale;
  const int64_t max_row = p.f[fi].max_row;
  const int64_t row_bytes = p.f[fi].row_bytes;
  const int lane = lane_id();
  const int R = kWave >> ll;  // lane groups; U * R divides 64, so every row slot e below is < 64
  const int g = lane >> ll, sl = lane & ((1 << ll) - 1);
  int64_t next_id = s0 + lane < s1 ? load_index(p, s0 + lane) : 0;
  for (int64_t c = s0; c < s1; c += kWave) {
    const int64_t id = next_id;
    if (c + kWave + lane < s1) next_id = load_index(p, c + kWave + lane);
    ids[lane] = c + lane < s1 ? static_cast<unsigned int>(clamp_i64(id, 0, max_row)) : 0u;
    const int n = static_cast<int>(s1 - c < kWave ? s1 - c : kWave);
    for (int k = 0; k < n; k += U * R) {
      uint4 v[U];
      float sc[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int e = k + u * R + g;
        const char* row = table + static_cast<uint64_t>(ids[e]) * static_cast<uint64_t>(row_bytes);
        const bool act = e < n;
        v[u] = act ? load_row_vec<TT>(row + sl * VB) : make_uint4(0u, 0u, 0u, 0u);
        sc[u] = 1.f;
        if constexpr (Quantized<TT>::value) sc[u] = act ? row_scale[ids[e]] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) acc_row<TT>(pa, v[u], sc[u]);
    }
  }
  for (int mk = 1 << ll; mk < kWave; mk <<= 1) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) pa[i] += shfl_xor_f32(pa[i], mk);
  }
}

template <typename TT, typename OT>
__device__ __forceinline__ void store_bag_rt(const PoolParams& p, int64_t b, int out_col, int64_t L, int sl,
                                             const float* a) {
  constexpr int VEC = Elem<TT>::kVecBytes / Elem<TT>::kBytes;
  float r[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) r[i] = a[i];
  if (p.pooling == CTI_EBAG_MEAN && L > 0) div_by_count<VEC>(r, 1.0 / static_cast<double>(L), static_cast<float>(L));
  round_like_reference<TT, VEC>(p, r);
  store_out<VEC>(reinterpret_cast<OT*>(p.out) + b * p.out_row_stride + out_col + sl * VEC, r, p.stream_out);
}

// ... or, in a mixed launch, each field's own (one lane vector per lane, 1 << lanes_log2 lanes
// per row, kMixedLo <= lanes_log2 <= kMixedHi), chosen at run time.
template <typename TT, typename OT, int LW>
struct MixedRows {
  static constexpr int VEC = Elem<TT>::kVecBytes / Elem<TT>::kBytes;
  static constexpr int DMAX = Shape<TT, 1 << kMixedHi, 1>::D;
  __device__ static __forceinline__ void split(const PoolParams& p, int fi, int64_t b, int64_t bs, int64_t be,
                                               int wave, float* s_red, unsigned int* ids) {
    const int ll = p.f[fi].lanes_log2;
    const int D = VEC << ll;
    const int sl = lane_id() & ((1 << ll) - 1);
    const bool g0 = lane_id() < (1 << ll);
    const int64_t per = (be - bs + LW - 1) / LW;
    const int64_t s0 = bs + wave * per < be ? bs + wave * per : be;
    const int64_t s1 = s0 + per < be ? s0 + per : be;
    float pa[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) pa[i] = 0.f;
    wave_slice_partial_rt<TT>(p, fi, ll, s0, s1, pa, ids);
    if (g0) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) s_red[wave * D + sl * VEC + i] = pa[i];
    }
    __syncthreads();
    if (wave == 0 && g0) {
      float r[VEC];
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        float x = s_red[sl * VEC + i];
#pragma unroll
        for (int w = 1; w < LW; ++w) x += s_red[w * D + sl * VEC + i];
        r[i] = x;
      }
      store_bag_rt<TT, OT>(p, b, p.f[fi].out_col, be - bs, sl, r);
    }
    __syncthreads();
  }
  __device__ static __forceinline__ void one(const PoolParams& p, int fi, int64_t b, int64_t bs, int64_t be,
                                             unsigned int* ids) {
    const int ll = p.f[fi].lanes_log2;
    float pa[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) pa[i] = 0.f;
    wave_slice_partial_rt<TT>(p, fi, ll, bs, be, pa, ids);
    if (lane_id() < (1 << ll)) store_bag_rt<TT, OT>(p, b, p.f[fi].out_col, be - bs, lane_id(), pa);
  }
};

// List kernel: LW wavefronts per workgroup. Every bag on the split list is cut into LW contiguous
// slices, one per wavefront, combined through LDS in wavefront order; then every bag on the
// one-wavefront list is pooled by one wavefront (lane groups take interleaved rows). List entries
// carry their bag's range, and the entry of a wavefront's next bag is loaded while it pools the
// current one, so a bag costs no lookup round trip of its own.
template <typename TT, typename OT, int LW, typename Rows>
__global__ void __launch_bounds__(LW * kWave) pool_long_kernel(const PoolParams p, LongList l) {
  __shared__ float s_red[LW * Rows::DMAX];
  __shared__ unsigned int s_ids[LW * kWave];
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  unsigned int* const ids = s_ids + wave * kWave;

  const unsigned int n = __hip_atomic_load(l.total2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  int64_t item = 0, bs = 0, be = 0;
  if (blockIdx.x < n) {
    const int64_t at = l.capacity - 1 - blockIdx.x;
    item = l.bags[at];
    bs = l.starts[at];
    be = l.ends[at];
  }
  for (unsigned int j = blockIdx.x; j < n; j += gridDim.x) {
    const unsigned int jn = j + gridDim.x;
    int64_t item_n = 0, bs_n = 0, be_n = 0;
    if (jn < n) {  // the next bag's entry, in flight while this one is pooled
      const int64_t at = l.capacity - 1 - jn;
      item_n = l.bags[at];
      bs_n = l.starts[at];
      be_n = l.ends[at];
    }
    const int64_t it = uniform_i64(item);
    Rows::split(p, static_cast<int>(it >> 40), it & kSampleMask, uniform_i64(bs), uniform_i64(be), wave, s_red, ids);
    item = item_n;
    bs = bs_n;
    be = be_n;
  }

  const unsigned int n1 = __hip_atomic_load(l.total, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned int stride = gridDim.x * LW;
  unsigned int j = blockIdx.x * LW + static_cast<unsigned int>(wave);
  if (j < n1) {
    item = l.bags[j];
    bs = l.starts[j];
    be = l.ends[j];
  }
  for (; j < n1; j += stride) {
    const unsigned int jn = j + stride;
    int64_t item_n = 0, bs_n = 0, be_n = 0;
    if (jn < n1) {
      item_n = l.bags[jn];
      bs_n = l.starts[jn];
      be_n = l.ends[jn];
    }
    const int64_t it = uniform_i64(item);
    Rows::one(p, static_cast<int>(it >> 40), it & kSampleMask, uniform_i64(bs), uniform_i64(be), ids);
    item = item_n;
    bs = bs_n;
    be = be_n;
  }
}

// Element-wise kernel for any row width / alignment: one wavefront per bag, rows accumulated in
// order, 4 columns per lane per pass (int8 rows: fma with the row's scale).
template <typename TT, typename OT>
__global__ void __launch_bounds__(kMainThreads) pool_generic_kernel(const PoolParams p) {
  constexpr int NC = 4;
  const int tile = block_tile();
  const int fi = field_of_tile(p, tile);
  const char* const table = p.f[fi].table;
  const int64_t max_row = p.f[fi].max_row;
  const int64_t row_bytes = p.f[fi].row_bytes;
  const int dim = p.f[fi].dim;
  const int out_col = p.f[fi].out_col;
  const int lane = lane_id();
  const int64_t b = static_cast<int64_t>(tile - fi * p.tiles_per_field);
  if (b >= p.batch) return;
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
      float rsc = 0.f;
      if (c + lane < end) {
        const int64_t row = clamp_i64(load_index(p, c + lane), 0, max_row);
        roff = row * row_bytes;
        if constexpr (Quantized<TT>::value) rsc = p.f[fi].row_scale[row];
      }
      const int n = static_cast<int>(end - c < kWave ? end - c : kWave);
      for (int k = 0; k < n; ++k) {
        const int64_t ro = shfl_i64(roff, k);
        const float sk = Quantized<TT>::value ? __int_as_float(shfl_i32(__float_as_int(rsc), k)) : 1.f;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
          const int col = c0 + i * kWave + lane;
          if (col < dim) {
            const float x = Elem<TT>::load(table + ro + static_cast<int64_t>(col) * Elem<TT>::kBytes);
            if constexpr (Quantized<TT>::value) acc[i] = __builtin_fmaf(x, sk, acc[i]);
            else acc[i] += x;
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int col = c0 + i * kWave + lane;
      if (col < dim) {
        float r = acc[i];
        if (p.pooling == CTI_EBAG_MEAN && L > 0) r = r / static_cast<float>(L);
        round_like_reference<TT, 1>(p, &r);
        store_one(o + col, r, p.stream_out);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------------------
int lanes_of(int variant) { return variant <= 6 ? (1 << variant) : 64; }
int bags_per_tile(int variant) {
  if (variant == kVarGeneric) return 1;
  const int r = kWave / lanes_of(variant);
  return kRounds * r <= kWave ? kRounds * r : kWave;  // as TileShape::NB
}

// Default short-bag limit of the tile kernels: longer bags are split over the wavefront's lane
// groups. Measured with host-made orders (us per launch, limit 16 / 24 / 32 / 40 / 48): bf16-2m
// 35.2 / 34.5 / 34.8 / 35.3 / 35.7, fp32-1m 56.3 / 55.6 / 55.6 / 55.8 / 56.2; lazy-32k (no
// order) 276.5 / 273.5 / 273.0 / 273.0 / 272.9.
constexpr int64_t kSubThreshold = 24;
// With length binning the limit stays 48 (capped at the block threshold): hetero-bf16 (block
// threshold 32) ran 157.9 us at 24 against 150.6 at 32. The fused pooling + LayerNorm kernel keeps
// 48 too: 24 measured 41.7 against 40.7 us there.
constexpr int64_t kSubThresholdBinned = 48;
constexpr int64_t kFusedSubThreshold = 48;

int64_t default_sub_threshold(int variant, bool bins) {
  if (variant == kVarGeneric) return kNoLimit;  // the element-wise kernel never splits
  return bins ? kSubThresholdBinned : kSubThreshold;
}

// With binning, bags longer than this go to the long kernel.
constexpr int64_t kDefaultBlockThreshold = 512;
constexpr int64_t kDefaultSplitThreshold = 192;   // listed bags longer than this are split over a workgroup
// Longest bag pooled by one subgroup (longer ones are split over the wavefront).
constexpr int64_t kMaxShortBag = int64_t{1} << 24;

int pick_variant(const cti_ebag_table& t, int tb, int ob, const void* out, int64_t out_row_stride) {
  const int64_t row_bytes = static_cast<int64_t>(t.dim) * tb;
  const int vb = tb == 1 ? 8 : 16;  // lane vector bytes (Elem<TT>::kVecBytes; only int8 has 1-byte elements)
  const bool table_ok = (reinterpret_cast<uintptr_t>(t.data) % vb == 0) && ((t.row_stride * tb) % vb == 0);
  const int vec = vb / tb;
  const int align = vec * ob < 16 ? vec * ob : 16;
  const bool out_ok = (reinterpret_cast<uintptr_t>(out) % align == 0) &&
                      ((out_row_stride * ob) % align == 0) &&
                      ((static_cast<int64_t>(t.out_col) * ob) % align == 0);
  if (!table_ok || !out_ok || row_bytes % vb != 0) return kVarGeneric;
  const int64_t nvec = row_bytes / vb;
  for (int v = 0; v <= 6; ++v) {
    if (nvec == (int64_t{1} << v)) return v;
  }
  if (nvec == 128) return kVarL64V2;
  if (nvec == 256) return kVarL64V4;
  return kVarGeneric;
}

void launch_bins(const PoolParams& p, const LongList& l, hipStream_t s) {
  const dim3 bgrid(static_cast<unsigned>((p.batch + kBinThreads - 1) / kBinThreads), static_cast<unsigned>(p.num_fields));
  hipLaunchKernelGGL(bin_kernel, bgrid, dim3(kBinThreads), 0, s, p, l);
}

// Workgroups of the list kernel: at most min(bags, nnz / (block_threshold + 1)) bags can be
// listed, and the workgroups loop over the list.
unsigned list_blocks(const PoolParams& p) {
  int64_t most = p.nnz / (p.block_threshold + 1) + 1;
  const int64_t bags = p.batch * p.num_fields;
  if (most > bags) most = bags;
  return static_cast<unsigned>(most < kLongBlocksMax ? (most > 0 ? most : 1) : kLongBlocksMax);
}

template <typename TT, typename OT, int LANES, int VPL>
void launch_shape(const PoolParams& p, const LongList* l, hipStream_t s) {
  if (l) launch_bins(p, *l, s);
  const dim3 grid(static_cast<unsigned>(p.num_tiles) + (p.next_order ? static_cast<unsigned>(p.order_blocks) : 0u)),
      block(kMainThreads);
  constexpr bool kStream = StreamShape<TT, LANES, VPL>::ok;
  const bool stream = kStream && p.stream_ok && p.buffer_ok;
  if (stream && p.idx32 && p.stream_out)
    hipLaunchKernelGGL((pool_kernel<TT, OT, LANES, VPL, true, kStream ? kTileStream32Nt : kTileRanked>), grid, block, 0, s, p);
  else if (stream && p.idx32)
    hipLaunchKernelGGL((pool_kernel<TT, OT, LANES, VPL, true, kStream ? kTileStream32 : kTileRanked>), grid, block, 0, s, p);
  else if (stream && p.stream_out)
    hipLaunchKernelGGL((pool_kernel<TT, OT, LANES, VPL, true, kStream ? kTileStream64Nt : kTileRanked>), grid, block, 0, s, p);
  else if (stream)
    hipLaunchKernelGGL((pool_kernel<TT, OT, LANES, VPL, true, kStream ? kTileStream64 : kTileRanked>), grid, block, 0, s, p);
  else if (p.buffer_ok)
    hipLaunchKernelGGL((pool_kernel<TT, OT, LANES, VPL, true, kTileRanked>), grid, block, 0, s, p);
  else
    hipLaunchKernelGGL((pool_kernel<TT, OT, LANES, VPL, false, kTileRanked>), grid, block, 0, s, p);
  if (l) {
    constexpr int LW = VPL >= 4 ? 4 : 8;  // keeps the LDS partials at <= 32 KB
    hipLaunchKernelGGL((pool_long_kernel<TT, OT, LW, FixedRows<TT, OT, LANES, VPL, LW>>), dim3(list_blocks(p)),
                       dim3(LW * kWave), 0, s, p, *l);
  }
}

// A mixed-width launch: fields of several one-vector-per-lane row shapes in one sequence.
template <typename TT, typename OT>
void launch_mixed(const PoolParams& p, const LongList* l, hipStream_t s) {
  if (l) launch_bins(p, *l, s);
  const dim3 grid(static_cast<unsigned>(p.num_tiles)), block(kMainThreads);
  if (p.buffer_ok)
    hipLaunchKernelGGL((pool_mixed_kernel<TT, OT, true>), grid, block, 0, s, p);
  else
    hipLaunchKernelGGL((pool_mixed_kernel<TT, OT, false>), grid, block, 0, s, p);
  if (l) {
    constexpr int LW = 8;
    hipLaunchKernelGGL((pool_long_kernel<TT, OT, LW, MixedRows<TT, OT, LW>>), dim3(list_blocks(p)), dim3(LW * kWave), 0,
                       s, p, *l);
  }
}

template <typename TT, typename OT>
hipError_t launch_variant(int variant, const PoolParams& p, const LongList* l, hipStream_t s) {
  switch (variant) {
    case 0: launch_shape<TT, OT, 1, 1>(p, l, s); break;
    case 1: launch_shape<TT, OT, 2, 1>(p, l, s); break;
    case 2: launch_shape<TT, OT, 4, 1>(p, l, s); break;
    case 3: launch_shape<TT, OT, 8, 1>(p, l, s); break;
    case 4: launch_shape<TT, OT, 16, 1>(p, l, s); break;
    case 5: launch_shape<TT, OT, 32, 1>(p, l, s); break;
    case 6: launch_shape<TT, OT, 64, 1>(p, l, s); break;
    case kVarL64V2: launch_shape<TT, OT, 64, 2>(p, l, s); break;
    case kVarL64V4: launch_shape<TT, OT, 64, 4>(p, l, s); break;
    case kVarMixed: launch_mixed<TT, OT>(p, l, s); break;
    default:
      hipLaunchKernelGGL((pool_generic_kernel<TT, OT>), dim3(static_cast<unsigned>(p.num_tiles)), dim3(kMainThreads), 0, s, p);
      break;
  }
  return hipGetLastError();
}

hipError_t launch_typed(int tdt, int odt, int variant, const PoolParams& p, const LongList* l, hipStream_t s) {
  switch (tdt * 3 + odt) {
    case CTI_EBAG_F32 * 3 + CTI_EBAG_F32: return launch_variant<float, float>(variant, p, l, s);
    case CTI_EBAG_F32 * 3 + CTI_EBAG_BF16: return launch_variant<float, bf16_t>(variant, p, l, s);
    case CTI_EBAG_F32 * 3 + CTI_EBAG_F16: return launch_variant<float, f16_t>(variant, p, l, s);
    case CTI_EBAG_BF16 * 3 + CTI_EBAG_F32: return launch_variant<bf16_t, float>(variant, p, l, s);
    case CTI_EBAG_BF16 * 3 + CTI_EBAG_BF16: return launch_variant<bf16_t, bf16_t>(variant, p, l, s);
    case CTI_EBAG_BF16 * 3 + CTI_EBAG_F16: return launch_variant<bf16_t, f16_t>(variant, p, l, s);
    case CTI_EBAG_F16 * 3 + CTI_EBAG_F32: return launch_variant<f16_t, float>(variant, p, l, s);
    case CTI_EBAG_F16 * 3 + CTI_EBAG_BF16: return launch_variant<f16_t, bf16_t>(variant, p, l, s);
    case CTI_EBAG_F16 * 3 + CTI_EBAG_F16: return launch_variant<f16_t, f16_t>(variant, p, l, s);
    case CTI_EBAG_I8 * 3 + CTI_EBAG_F32: return launch_variant<i8_t, float>(variant, p, l, s);
    case CTI_EBAG_I8 * 3 + CTI_EBAG_BF16: return launch_variant<i8_t, bf16_t>(variant, p, l, s);
    default: return launch_variant<i8_t, f16_t>(variant, p, l, s);
  }
}

struct Job {
  const void* values;
  int32_t idx32;
  int64_t nnz;
  const void* offsets;
  const void* val_base;
  int32_t off32;
  int64_t offsets_stride;
  int64_t batch;
  int32_t num_fields;
  const cti_ebag_table* tables;
  int32_t tdt;
  int32_t pooling;
  void* out;
  int32_t odt;
  int64_t out_row_stride;
  int32_t sub_threshold;    // 0 = default, < 0 = split every non-empty bag
  int32_t use_bins;
  int32_t block_threshold;  // 0 = default (with bins)
  int32_t split_threshold;  // 0 = default (with bins)
  void* workspace;
  const int32_t* tile_order;  // optional dispatch order (kOrderMagic layout)
  int32_t* next_order;        // optional: make the next batch's order here
  const void* next_offsets;
  int64_t order_bytes;        // size of each order buffer
  int32_t round_bf16;         // int8 tables: results rounded to bf16 before the output type
};

int validate_tables(const Job& j) {
  for (int f = 0; f < j.num_fields; ++f) {
    const cti_ebag_table& t = j.tables[f];
    if (!t.data) return set_error(CTI_EBAG_EINVAL, "table %d: data is NULL", f);
    if (t.rows < 1) return set_error(CTI_EBAG_EINVAL, "table %d: rows must be >= 1 (got %lld)", f, (long long)t.rows);
    if (t.rows > INT32_MAX)
      return set_error(CTI_EBAG_EUNSUPPORTED, "table %d: more than 2^31 - 1 rows (%lld)", f, (long long)t.rows);
    if (t.dim < 1) return set_error(CTI_EBAG_EINVAL, "table %d: dim must be >= 1 (got %d)", f, t.dim);
    if (t.row_stride < t.dim) return set_error(CTI_EBAG_EINVAL, "table %d: row_stride %lld < dim %d", f, (long long)t.row_stride, t.dim);
    if (t.out_col < 0 || static_cast<int64_t>(t.out_col) + t.dim > j.out_row_stride)
      return set_error(CTI_EBAG_EINVAL, "table %d: columns [%d, %lld) fall outside the output row of %lld", f, t.out_col,
                       (long long)t.out_col + t.dim, (long long)j.out_row_stride);
    if (j.tdt == CTI_EBAG_I8 && !t.row_scale) return set_error(CTI_EBAG_EINVAL, "table %d: int8 table without row_scale", f);
  }
  return CTI_EBAG_OK;
}

int64_t workspace_bytes(int64_t batch, int32_t num_fields);

// The variant whose rows are 16 lane vectors (256 bytes of fp32 / bf16 / fp16, 128 bytes of int8):
// the streamed tiles' shape.
constexpr int kVarStream = 4;
static_assert(StreamShape<float, 1 << kVarStream, 1>::ok && StreamShape<bf16_t, 1 << kVarStream, 1>::ok &&
                  StreamShape<f16_t, 1 << kVarStream, 1>::ok && StreamShape<i8_t, 1 << kVarStream, 1>::ok &&
                  TileShape<bf16_t, 1 << kVarStream, 1>::NB == kRounds * (kWave / 16),
              "the streamed shape is variant kVarStream");

// Whether a job's fields of the streamed shape may take streamed tiles (launch_shape also needs
// buffer loads over every table of their launch): no binning, the default short-bag limit, and
// walks / id offsets that fit 32 bits.
bool stream_variant_allowed(const Job& j) {
  const int64_t nb = kRounds * (kWave / 16);  // bags per tile of the streamed shape
  return !j.use_bins && j.sub_threshold == 0 && j.nnz < INT32_MAX / nb && j.nnz * (j.idx32 ? 4 : 8) < (int64_t{1} << 32);
}

int run_job(const Job& j, hipStream_t stream) {
  if (j.batch == 0 || j.num_fields == 0) return CTI_EBAG_OK;
  const int tb = dtype_bytes(j.tdt), ob = dtype_bytes(j.odt);
  LongList list;
  if (j.use_bins) {
    if (!j.workspace) return set_error(CTI_EBAG_EWORKSPACE, "length binning requested without a workspace");
    char* ws = static_cast<char*>(j.workspace);
    list.count = reinterpret_cast<unsigned int*>(ws);
    list.total = reinterpret_cast<unsigned int*>(ws) + 1;
    list.count2 = reinterpret_cast<unsigned int*>(ws) + 2;
    list.total2 = reinterpret_cast<unsigned int*>(ws) + 3;
    list.capacity = (workspace_bytes(j.batch, j.num_fields) - kWorkspaceHeader) / 24;
    list.bags = reinterpret_cast<int64_t*>(ws + kWorkspaceHeader);
    list.starts = list.bags + list.capacity;
    list.ends = list.starts + list.capacity;
  }
  // Group fields by kernel variant; each group is one launch sequence (per 64 fields). Fields
  // whose rows are one lane vector per lane but of different widths form one mixed group.
  std::vector<int> var(j.num_fields);
  for (int f = 0; f < j.num_fields; ++f) var[f] = pick_variant(j.tables[f], tb, ob, j.out, j.out_row_stride);
  // Fields of the streamed shape that may take streamed tiles keep a launch of their own, so a field is
  // pooled the same way whatever other fields share the call.
  const bool stream_apart = stream_variant_allowed(j);
  int one_vec_shapes = 0;
  for (int v = kMixedLo; v <= kMixedHi; ++v) {
    if (stream_apart && v == kVarStream) continue;
    for (int f = 0; f < j.num_fields; ++f) {
      if (var[f] == v) {
        ++one_vec_shapes;
        break;
      }
    }
  }
  const bool mixed = one_vec_shapes > 1;
  // A dispatch order belongs to a job that is one main-kernel launch of one fixed row shape.
  const bool ordered = j.tile_order || j.next_order;
  if (ordered) {
    bool one_shape = j.num_fields <= kMaxFields && !j.use_bins && var[0] != kVarGeneric;
    for (int f = 1; f < j.num_fields; ++f) one_shape = one_shape && var[f] == var[0];
    if (!one_shape)
      return set_error(CTI_EBAG_EUNSUPPORTED,
                       "a dispatch order needs one row shape with aligned rows, at most %d fields and no binning",
                       kMaxFields);
    const int bpt = bags_per_tile(var[0]);
    const int64_t tiles = static_cast<int64_t>(j.num_fields) * ((j.batch + bpt - 1) / bpt);
    if (tiles > INT32_MAX / 2)
      return set_error(CTI_EBAG_EUNSUPPORTED, "batch of %lld samples has too many tiles to order", (long long)j.batch);
    if (j.order_bytes < (kOrderHeader + tiles) * 4)
      return set_error(CTI_EBAG_EINVAL, "order buffers of %lld bytes; this job needs %lld", (long long)j.order_bytes,
                       (long long)((kOrderHeader + tiles) * 4));
  }
  for (int v = 0; v <= kVarMixed; ++v) {
    std::vector<int> fields;
    if (v == kVarMixed) {
      if (!mixed) continue;
      // widest rows first (fewest bags per tile), so those tiles start first
      for (int w = kMixedHi; w >= kMixedLo; --w) {
        if (stream_apart && w == kVarStream) continue;
        for (int f = 0; f < j.num_fields; ++f) if (var[f] == w) fields.push_back(f);
      }
    } else {
      if (mixed && v >= kMixedLo && v <= kMixedHi && !(stream_apart && v == kVarStream)) continue;
      for (int f = 0; f < j.num_fields; ++f) if (var[f] == v) fields.push_back(f);
    }
    for (size_t c0 = 0; c0 < fields.size(); c0 += kMaxFields) {
      PoolParams p;
      memset(&p, 0, sizeof(p));
      p.values = j.values;
      p.offsets = j.offsets;
      p.val_base = j.val_base;
      p.out = static_cast<char*>(j.out);
      p.nnz = j.nnz;
      p.offsets_stride = j.offsets_stride;
      p.out_row_stride = j.out_row_stride;
      p.batch = j.batch;
      p.pooling = j.pooling;
      p.idx32 = j.idx32;
      p.off32 = j.off32;
      p.round_bf16 = j.round_bf16;
      const bool bins = j.use_bins && v != kVarGeneric;
      p.stream_ok = stream_variant_allowed(j) ? 1 : 0;
      p.stream_out = j.batch * j.out_row_stride * dtype_bytes(j.odt) >= kStreamOutBytes;
      if (v == kVarGeneric) p.sub_threshold = kNoLimit;
      else if (j.sub_threshold == 0) p.sub_threshold = default_sub_threshold(v, bins);
      else p.sub_threshold = j.sub_threshold < 0 ? 0 : j.sub_threshold;
      p.block_threshold = !bins ? kNoLimit : (j.block_threshold > 0 ? j.block_threshold : kDefaultBlockThreshold);
      p.split_threshold = !bins ? kNoLimit : (j.split_threshold > 0 ? j.split_threshold : kDefaultSplitThreshold);
      // a bag is pooled by exactly one kernel: never call a listed (long) bag short
      if (v != kVarGeneric && p.sub_threshold > p.block_threshold) p.sub_threshold = p.block_threshold;
      // short-bag lengths are kept in 32 bits on the device
      if (v != kVarGeneric && p.sub_threshold > kMaxShortBag) p.sub_threshold = kMaxShortBag;
      p.bin_count = bins ? list.count : nullptr;
      p.bin_total = bins ? list.total : nullptr;
      if (ordered) {  // the job's only launch: fields 0 .. F-1 in job order
        if (c0 != 0 || fields.size() != static_cast<size_t>(j.num_fields))
          return set_error(CTI_EBAG_EUNSUPPORTED, "internal: an ordered job must be one launch");
        p.tile_order = j.tile_order;
        p.next_order = j.next_order;
        p.next_offsets = j.next_offsets;
      }
      const size_t nf = fields.size() - c0 < static_cast<size_t>(kMaxFields) ? fields.size() - c0 : kMaxFields;
      p.num_fields = static_cast<int32_t>(nf);
      bool all_buf = true;
      int64_t tiles = 0;
      for (size_t i = 0; i < nf; ++i) {
        const int f = fields[c0 + i];
        const cti_ebag_table& t = j.tables[f];
        FieldDesc& d = p.f[i];
        const int bpt = bags_per_tile(var[f]);
        d.lanes_log2 = var[f] <= 6 ? var[f] : 0;
        d.tile_begin = static_cast<int32_t>(tiles < INT32_MAX ? tiles : INT32_MAX);
        tiles += (j.batch + bpt - 1) / bpt;
        d.table = static_cast<const char*>(t.data);
        d.row_scale = j.tdt == CTI_EBAG_I8 ? t.row_scale : nullptr;
        d.max_row = t.rows - 1;
        d.row_bytes = t.row_stride * tb;
        d.dim = t.dim;
        d.out_col = t.out_col;
        d.gidx = f;
        const int64_t span = (t.rows - 1) * d.row_bytes + static_cast<int64_t>(t.dim) * tb;
        const bool pow2 = (d.row_bytes & (d.row_bytes - 1)) == 0;
        // buffer path: power-of-two rows of >= 8 bytes and (rows + 1) * row_bytes <= 2^32, so the
        // pad row id 0xffffffff >> log2(row_bytes) addresses past both the rows and the scales
        const bool fits = d.row_bytes >= 8 && t.rows < (int64_t{1} << 32) / d.row_bytes;
        d.span_bytes = pow2 && fits ? static_cast<uint32_t>(span) : 0u;
        all_buf = all_buf && d.span_bytes != 0;
      }
      if (tiles > INT32_MAX)
        return set_error(CTI_EBAG_EUNSUPPORTED, "batch of %lld samples needs more than 2^31 tiles", (long long)j.batch);
      p.buffer_ok = all_buf ? 1 : 0;
      p.num_tiles = static_cast<int32_t>(tiles);
      // every field of a single-shape launch has the same number of tiles
      p.tiles_per_field = static_cast<int32_t>(tiles / static_cast<int64_t>(nf));
      p.tpf_inv = p.tiles_per_field > 0 ? 0xffffffffu / static_cast<uint32_t>(p.tiles_per_field) : 0u;
      if (p.next_order) {  // one workgroup per chunk of each XCD range
        const int64_t per_range = (tiles + 7) / 8;
        p.order_blocks = static_cast<int32_t>(8 * ((per_range + kOrderChunk - 1) / kOrderChunk));
      }
      const hipError_t e = launch_typed(j.tdt, j.odt, v, p, bins ? &list : nullptr, stream);
      if (e != hipSuccess) return set_error(CTI_EBAG_EHIP, "pooling kernel launch failed: %s", hipGetErrorString(e));
    }
  }
  return CTI_EBAG_OK;
}

bool dtype_ok(int32_t dt) { return dt == CTI_EBAG_F32 || dt == CTI_EBAG_BF16 || dt == CTI_EBAG_F16; }

// Header, then three arrays of one entry per bag of a launch (field / sample, start, end).
int64_t workspace_bytes(int64_t batch, int32_t num_fields) {
  const int64_t per_launch = num_fields < kMaxFields ? num_fields : kMaxFields;
  return kWorkspaceHeader + 24 * batch * per_launch;
}

}  // namespace
}  // namespace cti

using namespace cti;

namespace cti {
namespace {

// The reference-layout launch (one shared table, slot-local offsets, sum pooling) for any table
// type and index / offset width; `scale` is the int8 table's per-row scale.
int run_all_slots(const void* values, int32_t index_type, const void* val_offsets, const void* row_offsets,
                  int32_t offset_type, const void* weight, const float* scale, int32_t tdt, void* out, int32_t odt,
                  int64_t batch_size, int32_t num_slots, int32_t emb_dim, int64_t max_idx, int64_t nnz, void* stream,
                  const int32_t* tile_order = nullptr, int64_t order_bytes = 0) {
  if (index_type != CTI_EBAG_I64 && index_type != CTI_EBAG_I32)
    return set_error(CTI_EBAG_EINVAL, "unknown index type code %d", index_type);
  if (offset_type != CTI_EBAG_I64 && offset_type != CTI_EBAG_I32)
    return set_error(CTI_EBAG_EINVAL, "unknown offset type code %d", offset_type);
  if (batch_size < 0) return set_error(CTI_EBAG_EINVAL, "batch_size must be >= 0 (got %lld)", (long long)batch_size);
  if (num_slots < 0) return set_error(CTI_EBAG_EINVAL, "num_slots must be >= 0 (got %d)", num_slots);
  if (emb_dim < 1) return set_error(CTI_EBAG_EINVAL, "emb_dim must be >= 1 (got %d)", emb_dim);
  if (max_idx < 0) return set_error(CTI_EBAG_EINVAL, "max_idx must be >= 0 (got %lld)", (long long)max_idx);
  if (max_idx >= INT32_MAX) return set_error(CTI_EBAG_EUNSUPPORTED, "max_idx must be < 2^31 - 1 (got %lld)", (long long)max_idx);
  if (nnz < 0) return set_error(CTI_EBAG_EINVAL, "nnz must be >= 0 (got %lld)", (long long)nnz);
  if (batch_size == 0 || num_slots == 0) return CTI_EBAG_OK;
  if (!val_offsets || !row_offsets || !weight || !out || (nnz > 0 && !values) || (tdt == CTI_EBAG_I8 && !scale))
    return set_error(CTI_EBAG_EINVAL, "NULL device pointer among values/val_offsets/row_offsets/weight/scale/out");
  std::vector<cti_ebag_table> tables(num_slots);
  for (int s = 0; s < num_slots; ++s) {
    tables[s].data = weight;
    tables[s].rows = max_idx + 1;
    tables[s].row_stride = emb_dim;
    tables[s].dim = emb_dim;
    tables[s].out_col = s * emb_dim;
    tables[s].row_scale = scale;
  }
  Job j;
  memset(&j, 0, sizeof(j));
  j.values = values;
  j.idx32 = index_type == CTI_EBAG_I32;
  j.nnz = nnz;
  j.offsets = row_offsets;
  j.val_base = val_offsets;
  j.off32 = offset_type == CTI_EBAG_I32;
  j.offsets_stride = batch_size + 1;
  j.batch = batch_size;
  j.num_fields = num_slots;
  j.tables = tables.data();
  j.tdt = tdt;
  j.pooling = CTI_EBAG_SUM;
  j.out = out;
  j.odt = odt;
  j.out_row_stride = static_cast<int64_t>(num_slots) * emb_dim;
  // the reference's int8 kernel stores acc.to(tl.bfloat16) into an output of the table's dtype
  // (online_best/infer.py:941, :989-996): fp32 / fp16 outputs get the bf16-rounded value
  j.round_bf16 = tdt == CTI_EBAG_I8 && odt != CTI_EBAG_BF16;
  j.tile_order = tile_order;
  j.order_bytes = order_bytes;
  return run_job(j, static_cast<hipStream_t>(stream));
}

}  // namespace
}  // namespace cti

namespace cti {
namespace {

template <typename TT, typename PT, int LANES>
hipError_t launch_fused(const PoolParams& p, const FusedNorm& fn, int spw, size_t row_lds, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((p.batch + spw - 1) / spw)), block(fused_waves(LANES) * kWave);
  const size_t lds = row_lds * spw;
  switch (spw * 2 + (p.buffer_ok ? 1 : 0)) {
    case 2: hipLaunchKernelGGL((pool_norm_kernel<TT, PT, LANES, 1, false>), grid, block, lds, s, p, fn); break;
    case 3: hipLaunchKernelGGL((pool_norm_kernel<TT, PT, LANES, 1, true>), grid, block, lds, s, p, fn); break;
    case 4: hipLaunchKernelGGL((pool_norm_kernel<TT, PT, LANES, 2, false>), grid, block, lds, s, p, fn); break;
    case 5: hipLaunchKernelGGL((pool_norm_kernel<TT, PT, LANES, 2, true>), grid, block, lds, s, p, fn); break;
    case 8: hipLaunchKernelGGL((pool_norm_kernel<TT, PT, LANES, 4, false>), grid, block, lds, s, p, fn); break;
    default: hipLaunchKernelGGL((pool_norm_kernel<TT, PT, LANES, 4, true>), grid, block, lds, s, p, fn); break;
  }
  return hipGetLastError();
}

template <typename TT, typename PT>
hipError_t launch_fused_lanes(int lanes, const PoolParams& p, const FusedNorm& fn, int spw, size_t row_lds,
                              hipStream_t s) {
  switch (lanes) {
    case 4: return launch_fused<TT, PT, 4>(p, fn, spw, row_lds, s);
    case 8: return launch_fused<TT, PT, 8>(p, fn, spw, row_lds, s);
    case 16: return launch_fused<TT, PT, 16>(p, fn, spw, row_lds, s);
    case 32: return launch_fused<TT, PT, 32>(p, fn, spw, row_lds, s);
    default: return launch_fused<TT, PT, 64>(p, fn, spw, row_lds, s);
  }
}

constexpr int kFusedSamples = 2;  // measured: 1 / 2 / 4 samples per workgroup 45.7 / 40.5 / 44.6 us

// Samples per fused workgroup: up to kFusedSamples, while the workgroup's bags fit one lane each
// and the LDS rows stay within kFusedLdsMax.
constexpr int64_t kFusedLdsMax = 64 * 1024;
int fused_samples(int num_slots, int64_t row_out_bytes) {
  int spw = kFusedSamples;
  while (spw > 1 && (spw * num_slots > kFusedBags || spw * row_out_bytes > kFusedLdsMax / 2)) spw /= 2;
  return spw;
}

constexpr int64_t kFusedRowBytesMax = 64 * 1024;  // LDS copy of one output row
constexpr int kFusedMaxSlots = 64;

}  // namespace
}  // namespace cti

extern "C" int cti_ebag_fused_all_slots_layernorm(const void* values, int32_t index_type, const void* val_offsets,
                                                  const void* row_offsets, int32_t offset_type, const void* weight,
                                                  int32_t dtype, void* out, int64_t batch_size, int32_t num_slots,
                                                  int32_t emb_dim, int64_t max_idx, int64_t nnz, int32_t pooling,
                                                  const void* gamma, const void* beta, int32_t param_dtype, float eps,
                                                  void* stream) {
  clear_error();
  if (index_type != CTI_EBAG_I64 && index_type != CTI_EBAG_I32)
    return set_error(CTI_EBAG_EINVAL, "unknown index type code %d", index_type);
  if (offset_type != CTI_EBAG_I64 && offset_type != CTI_EBAG_I32)
    return set_error(CTI_EBAG_EINVAL, "unknown offset type code %d", offset_type);
  if (!dtype_ok(dtype)) return set_error(CTI_EBAG_EINVAL, "unknown dtype code %d", dtype);
  if (!dtype_ok(param_dtype)) return set_error(CTI_EBAG_EINVAL, "unknown parameter dtype code %d", param_dtype);
  if (pooling != CTI_EBAG_SUM && pooling != CTI_EBAG_MEAN) return set_error(CTI_EBAG_EINVAL, "unknown pooling code %d", pooling);
  if (batch_size < 0) return set_error(CTI_EBAG_EINVAL, "batch_size must be >= 0 (got %lld)", (long long)batch_size);
  if (num_slots < 0) return set_error(CTI_EBAG_EINVAL, "num_slots must be >= 0 (got %d)", num_slots);
  if (emb_dim < 1) return set_error(CTI_EBAG_EINVAL, "emb_dim must be >= 1 (got %d)", emb_dim);
  if (max_idx < 0) return set_error(CTI_EBAG_EINVAL, "max_idx must be >= 0 (got %lld)", (long long)max_idx);
  if (max_idx >= INT32_MAX) return set_error(CTI_EBAG_EUNSUPPORTED, "max_idx must be < 2^31 - 1 (got %lld)", (long long)max_idx);
  if (nnz < 0) return set_error(CTI_EBAG_EINVAL, "nnz must be >= 0 (got %lld)", (long long)nnz);
  if (!(eps >= 0.0f)) return set_error(CTI_EBAG_EINVAL, "eps must be >= 0");
  if (batch_size == 0 || num_slots == 0) return CTI_EBAG_OK;
  if (!val_offsets || !row_offsets || !weight || !out || !gamma || !beta || (nnz > 0 && !values))
    return set_error(CTI_EBAG_EINVAL, "NULL device pointer among values/val_offsets/row_offsets/weight/out/gamma/beta");
  // shapes the fused kernel covers; the caller runs pooling and LayerNorm separately otherwise
  const int tb = dtype_bytes(dtype);
  const int64_t row_bytes = static_cast<int64_t>(emb_dim) * tb;
  if (dtype == CTI_EBAG_F16 || param_dtype == CTI_EBAG_F16)
    return set_error(CTI_EBAG_EUNSUPPORTED, "fused LayerNorm: fp16 tables or parameters");
  if (num_slots > kFusedMaxSlots)
    return set_error(CTI_EBAG_EUNSUPPORTED, "fused LayerNorm: more than %d slots", kFusedMaxSlots);
  if (row_bytes < 64 || row_bytes > 1024 || (row_bytes & (row_bytes - 1)) != 0)
    return set_error(CTI_EBAG_EUNSUPPORTED, "fused LayerNorm: table rows of %lld bytes (64..1024, a power of two)",
                     (long long)row_bytes);
  if (row_bytes * num_slots > kFusedRowBytesMax)
    return set_error(CTI_EBAG_EUNSUPPORTED, "fused LayerNorm: output rows over %lld bytes", (long long)kFusedRowBytesMax);
  if (reinterpret_cast<uintptr_t>(weight) % 16 || reinterpret_cast<uintptr_t>(out) % 16 ||
      reinterpret_cast<uintptr_t>(gamma) % 16 || reinterpret_cast<uintptr_t>(beta) % 16)
    return set_error(CTI_EBAG_EUNSUPPORTED, "fused LayerNorm: weight, out, gamma and beta must be 16-byte aligned");
  const int lanes = static_cast<int>(row_bytes / 16);
  PoolParams p;
  memset(&p, 0, sizeof(p));
  p.values = values;
  p.idx32 = index_type == CTI_EBAG_I32;
  p.offsets = row_offsets;
  p.val_base = val_offsets;
  p.off32 = offset_type == CTI_EBAG_I32;
  p.offsets_stride = batch_size + 1;
  p.nnz = nnz;
  p.out = static_cast<char*>(out);
  p.out_row_stride = static_cast<int64_t>(num_slots) * emb_dim;
  p.batch = batch_size;
  p.pooling = pooling;
  p.num_fields = num_slots;
  p.stream_out = batch_size * p.out_row_stride * tb >= kStreamOutBytes;
  p.sub_threshold = kFusedSubThreshold;
  p.block_threshold = kNoLimit;
  p.split_threshold = kNoLimit;
  const int64_t rows = max_idx + 1;
  const int64_t span = (rows - 1) * row_bytes + row_bytes;
  const bool fits = rows < (int64_t{1} << 32) / row_bytes;
  for (int f = 0; f < num_slots; ++f) {
    FieldDesc& d = p.f[f];
    d.table = static_cast<const char*>(weight);
    d.max_row = max_idx;
    d.row_bytes = row_bytes;
    d.dim = emb_dim;
    d.out_col = f * emb_dim;
    d.gidx = f;
    d.span_bytes = fits ? static_cast<uint32_t>(span) : 0u;
  }
  p.buffer_ok = fits ? 1 : 0;
  if (batch_size > INT32_MAX) return set_error(CTI_EBAG_EUNSUPPORTED, "batch_size must be < 2^31");
  FusedNorm fn;
  fn.gamma = gamma;
  fn.beta = beta;
  fn.eps = eps;
  const size_t row_lds = static_cast<size_t>(row_bytes * num_slots);
  const int spw = fused_samples(num_slots, row_bytes * num_slots);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (dtype == CTI_EBAG_F32)
    e = param_dtype == CTI_EBAG_F32 ? launch_fused_lanes<float, float>(lanes, p, fn, spw, row_lds, st)
                                    : launch_fused_lanes<float, bf16_t>(lanes, p, fn, spw, row_lds, st);
  else
    e = param_dtype == CTI_EBAG_F32 ? launch_fused_lanes<bf16_t, float>(lanes, p, fn, spw, row_lds, st)
                                    : launch_fused_lanes<bf16_t, bf16_t>(lanes, p, fn, spw, row_lds, st);
  if (e != hipSuccess) return set_error(CTI_EBAG_EHIP, "fused pooling + LayerNorm launch failed: %s", hipGetErrorString(e));
  return CTI_EBAG_OK;
}

extern "C" int cti_ebag_fused_all_slots(const int64_t* values, const int64_t* val_offsets,
                                        const int64_t* row_offsets, const void* weight, int32_t dtype,
                                        void* out, int64_t batch_size, int32_t num_slots, int32_t emb_dim,
                                        int64_t max_idx, int64_t nnz, void* stream) {
  clear_error();
  if (!dtype_ok(dtype)) return set_error(CTI_EBAG_EINVAL, "unknown dtype code %d", dtype);
  return run_all_slots(values, CTI_EBAG_I64, val_offsets, row_offsets, CTI_EBAG_I64, weight, nullptr, dtype, out, dtype,
                       batch_size, num_slots, emb_dim, max_idx, nnz, stream);
}

extern "C" int cti_ebag_fused_all_slots_int8(const int64_t* values, const int64_t* val_offsets,
                                             const int64_t* row_offsets, const int8_t* weight_int8,
                                             const float* scale, void* out, int32_t out_dtype, int64_t batch_size,
                                             int32_t num_slots, int32_t emb_dim, int64_t max_idx, int64_t nnz,
                                             void* stream) {
  clear_error();
  if (!dtype_ok(out_dtype)) return set_error(CTI_EBAG_EINVAL, "unknown output dtype code %d", out_dtype);
  return run_all_slots(values, CTI_EBAG_I64, val_offsets, row_offsets, CTI_EBAG_I64, weight_int8, scale, CTI_EBAG_I8,
                       out, out_dtype, batch_size, num_slots, emb_dim, max_idx, nnz, stream);
}

extern "C" int cti_ebag_fused_all_slots_typed(const void* values, int32_t index_type, const void* val_offsets,
                                              const void* row_offsets, int32_t offset_type, const void* weight,
                                              int32_t table_dtype, const float* scale, void* out, int32_t out_dtype,
                                              int64_t batch_size, int32_t num_slots, int32_t emb_dim, int64_t max_idx,
                                              int64_t nnz, void* stream) {
  clear_error();
  if (!dtype_ok(table_dtype) && table_dtype != CTI_EBAG_I8)
    return set_error(CTI_EBAG_EINVAL, "unknown table dtype code %d", table_dtype);
  if (!dtype_ok(out_dtype)) return set_error(CTI_EBAG_EINVAL, "unknown output dtype code %d", out_dtype);
  return run_all_slots(values, index_type, val_offsets, row_offsets, offset_type, weight,
                       table_dtype == CTI_EBAG_I8 ? scale : nullptr, table_dtype, out, out_dtype, batch_size, num_slots,
                       emb_dim, max_idx, nnz, stream);
}

extern "C" int64_t cti_ebag_workspace_bytes(int64_t batch_size, int32_t num_fields) {
  if (batch_size < 0 || num_fields < 0) return -1;
  return workspace_bytes(batch_size, num_fields);
}

extern "C" int64_t cti_ebag_order_bytes(int64_t batch_size, int32_t num_fields) {
  if (batch_size < 0 || num_fields < 0) return -1;
  const int64_t per_launch = num_fields < kMaxFields ? num_fields : kMaxFields;
  return (kOrderHeader + batch_size * per_launch) * 4;  // at least one bag per tile
}

extern "C" int cti_ebag_forward(const void* values, int32_t index_type, int64_t nnz, const int64_t* offsets,
                                int64_t batch_size, int32_t num_fields, const cti_ebag_table* tables,
                                int32_t table_dtype, int32_t pooling, void* out, int32_t out_dtype,
                                int64_t out_row_stride, void* workspace, int64_t workspace_bytes_given,
                                const cti_ebag_options* opts, void* stream) {
  clear_error();
  if (index_type != CTI_EBAG_I64 && index_type != CTI_EBAG_I32)
    return set_error(CTI_EBAG_EINVAL, "unknown index type code %d", index_type);
  if (!dtype_ok(table_dtype) && table_dtype != CTI_EBAG_I8)
    return set_error(CTI_EBAG_EINVAL, "unknown table dtype code %d", table_dtype);
  if (!dtype_ok(out_dtype)) return set_error(CTI_EBAG_EINVAL, "unknown output dtype code %d", out_dtype);
  if (pooling != CTI_EBAG_SUM && pooling != CTI_EBAG_MEAN) return set_error(CTI_EBAG_EINVAL, "unknown pooling code %d", pooling);
  if (nnz < 0) return set_error(CTI_EBAG_EINVAL, "nnz must be >= 0 (got %lld)", (long long)nnz);
  if (batch_size < 0) return set_error(CTI_EBAG_EINVAL, "batch_size must be >= 0 (got %lld)", (long long)batch_size);
  if (num_fields < 0) return set_error(CTI_EBAG_EINVAL, "num_fields must be >= 0 (got %d)", num_fields);
  if (out_row_stride < 1) return set_error(CTI_EBAG_EINVAL, "out_row_stride must be >= 1 (got %lld)", (long long)out_row_stride);
  if (batch_size == 0 || num_fields == 0) return CTI_EBAG_OK;
  if (!tables) return set_error(CTI_EBAG_EINVAL, "tables (host array) is NULL");
  if (!offsets || !out || (nnz > 0 && !values)) return set_error(CTI_EBAG_EINVAL, "NULL device pointer among values/offsets/out");
  if (batch_size >= (int64_t{1} << 40)) return set_error(CTI_EBAG_EUNSUPPORTED, "batch_size must be < 2^40");
  Job j;
  memset(&j, 0, sizeof(j));
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
  j.workspace = workspace;
  if (opts) {
    j.sub_threshold = opts->long_threshold;
    j.use_bins = opts->use_bins != 0;
    j.block_threshold = opts->block_threshold;
    j.split_threshold = opts->split_threshold;
    j.tile_order = opts->tile_order;
    j.next_order = opts->next_order;
    j.next_offsets = opts->next_offsets;
    j.order_bytes = opts->order_bytes;
  }
  if (j.tile_order || j.next_order) {
    if (reinterpret_cast<uintptr_t>(j.tile_order) % 4 != 0 || reinterpret_cast<uintptr_t>(j.next_order) % 4 != 0)
      return set_error(CTI_EBAG_EINVAL, "order buffers must be 4-byte aligned");
    if (j.next_order && !j.next_offsets) return set_error(CTI_EBAG_EINVAL, "next_order given without next_offsets");
    if (j.order_bytes <= 0) return set_error(CTI_EBAG_EINVAL, "order_bytes must be > 0 (got %lld)", (long long)j.order_bytes);
    if (j.tile_order && j.next_order) {
      const uintptr_t a = reinterpret_cast<uintptr_t>(j.tile_order), b = reinterpret_cast<uintptr_t>(j.next_order);
      if (a < b + static_cast<uintptr_t>(j.order_bytes) && b < a + static_cast<uintptr_t>(j.order_bytes))
        return set_error(CTI_EBAG_EINVAL, "tile_order and next_order overlap (the launch reads one and writes the other)");
    }
  }
  if (j.use_bins) {
    const int64_t need = workspace_bytes(batch_size, num_fields);
    if (!workspace || workspace_bytes_given < need)
      return set_error(CTI_EBAG_EWORKSPACE, "length binning needs a zero-initialised workspace of %lld bytes (got %lld)",
                       (long long)need, (long long)(workspace ? workspace_bytes_given : 0));
    if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
      return set_error(CTI_EBAG_EINVAL, "workspace must be 256-byte aligned");
  }
  const int rc = validate_tables(j);
  if (rc != CTI_EBAG_OK) return rc;
  return run_job(j, static_cast<hipStream_t>(stream));
}

namespace cti {

int order_bags_per_tile(int32_t table_dtype, int32_t emb_dim) {
  // the row shape a launch takes for aligned buffers
  cti_ebag_table t;
  memset(&t, 0, sizeof(t));
  t.data = reinterpret_cast<const void*>(uintptr_t{256});
  t.rows = 1;
  t.row_stride = emb_dim;
  t.dim = emb_dim;
  const int variant = pick_variant(t, dtype_bytes(table_dtype), 4, reinterpret_cast<void*>(uintptr_t{256}),
                                   static_cast<int64_t>(emb_dim) * 4);
  return variant == kVarGeneric ? 0 : bags_per_tile(variant);
}

}  // namespace cti

extern "C" int cti_ebag_fused_all_slots_ordered(const void* values, int32_t index_type, const void* val_offsets,
                                                const void* row_offsets, int32_t offset_type, const void* weight,
                                                int32_t table_dtype, const float* scale, void* out, int32_t out_dtype,
                                                int64_t batch_size, int32_t num_slots, int32_t emb_dim,
                                                int64_t max_idx, int64_t nnz, const int32_t* tile_order,
                                                int64_t order_bytes, void* stream) {
  clear_error();
  if (!dtype_ok(table_dtype) && table_dtype != CTI_EBAG_I8)
    return set_error(CTI_EBAG_EINVAL, "unknown table dtype code %d", table_dtype);
  if (!dtype_ok(out_dtype)) return set_error(CTI_EBAG_EINVAL, "unknown output dtype code %d", out_dtype);
  if (tile_order) {
    if (reinterpret_cast<uintptr_t>(tile_order) % 4 != 0) return set_error(CTI_EBAG_EINVAL, "tile_order must be 4-byte aligned");
    if (order_bytes <= 0) return set_error(CTI_EBAG_EINVAL, "order_bytes must be > 0 (got %lld)", (long long)order_bytes);
  }
  return run_all_slots(values, index_type, val_offsets, row_offsets, offset_type, weight,
                       table_dtype == CTI_EBAG_I8 ? scale : nullptr, table_dtype, out, out_dtype, batch_size, num_slots,
                       emb_dim, max_idx, nnz, stream, tile_order, order_bytes);
}
