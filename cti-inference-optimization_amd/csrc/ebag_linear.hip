// The encoder's input LayerNorm followed by its Linear, on the matrix cores of gfx950 (MI355X).
//
// online_best/infer.py:1061-1085 normalises the pooled block [B, 28*D] (Triton kernel :829-858,
// output in the block's dtype) and maps it to d_model with nn.Linear (a library GEMM):
//   a[m, k] = bf16( ((x[m, k] - mean[m]) * rstd[m]) * gamma[k] + beta[k] )
//   y[m, n] = sum_k a[m, k] * w[n, k] + bias[n]              (fp32 accumulation, one rounding)
// Here both run in one kernel: the LayerNorm is applied while the pooled block's tiles are moved
// from HBM to LDS (each element normalised in fp32 as the LayerNorm kernel computes it and
// rounded to bf16 as that kernel stores it), so the normalised block never reaches HBM; the
// per-row mean and rstd come from the pooling or statistics pass (cti_ebag_layernorm with no
// output). Without statistics the kernel is the plain Linear.
//
// Two forms (the products on v_mfma_f32_16x16x32_bf16: lane l supplies A[l%16][8(l/16) .. +8)
// and B[8(l/16) .. +8)[l%16] and receives C[4(l/16) + r][l%16], r < 4; workgroups numbered so
// that the tiles of one row band run on one XCD, whose L2 then serves the band to each of them):
//   ln_linear_big_kernel  K a multiple of 128 (every encoder shape): 128 x 256 or 128 x 128 tiles
//                         of 8 wavefronts, both operands through LDS (XOR-swizzled rows);
//   ln_linear_kernel      any K (a multiple of 8): 64 x 256 tiles of 4 wavefronts, each owning 64
//                         columns, x through LDS and the weight's fragments straight to registers.
// Both walk K in steps of 64 with each step's loads issued two steps ahead into rotating register
// sets, x normalised on its way to LDS, two LDS buffers and one barrier per step. When the large
// form's tiles would leave CUs idle (few rows), K is split over several workgroups per tile: each
// writes its fp32 partial products to a caller's workspace and ln_linear_reduce_kernel adds the
// splits in split order, adds the bias and rounds once.
#include <stdint.h>

#include "ebag_device.h"
#include "ebag_internal.h"

namespace cti {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBK = 64;        // K per step
constexpr int kLds = kBK + 8;  // LDS row pitch in elements (144 bytes)
constexpr int kChunks = kBK / 8;  // 16-byte chunks per tile row
constexpr int kXcds = 8;
constexpr int kWaveCols = 64;  // output columns per wavefront
constexpr int64_t kSplitTarget = 256;  // split K until the large form has one workgroup per CU

struct LinearParams {
  const char* x;      // [M, K] bf16
  const float* mean;  // [M], NULL: no LayerNorm
  const float* rstd;  // [M]
  const void* gamma;  // [K]
  const void* beta;   // [K]
  const char* w;      // [N, K] bf16
  const void* bias;   // [N] or NULL
  char* y;            // [M, N]
  int64_t M;
  int32_t N;
  int32_t K;
  int32_t tiles_m;
  int32_t tiles_n;
  float* part;          // split K: fp32 partial products [splits, M, N] (no bias), NULL: no split
  int32_t split_steps;  // split K: steps of kBK per split (even); split s is blockIdx.y
};

// One bf16 chunk (8 elements) normalised: ((x - mean) * rstd) * g + b, rounded to bf16.
__device__ __forceinline__ uint4 normalise8(const uint4& raw, float mean, float rstd, const float* g, const float* b) {
  float v[8];
  unpack16(raw, v, bf16_t{});
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (v[e] - mean) * rstd * g[e] + b[e];
  return make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                    pack_bf16x2(v[6], v[7]));
}

template <typename OT>
__device__ __forceinline__ void store_y(char* y, int64_t idx, float v) {
  if constexpr (std::is_same<OT, float>::value) reinterpret_cast<float*>(y)[idx] = v;
  else reinterpret_cast<uint16_t*>(y)[idx] = static_cast<uint16_t>(pack_bf16x2(v, 0.f));
}

template <int BM, int WAVES, int U, bool LN, typename PT, typename BT, typename OT>
__global__ void __launch_bounds__(WAVES * kWave) ln_linear_kernel(const LinearParams p) {
  constexpr int THREADS = WAVES * kWave;
  constexpr int BN = WAVES * kWaveCols;
  constexpr int MI = BM / 16, NI = kWaveCols / 16;  // 16 x 16 products per wavefront
  constexpr int PA = BM * kChunks / THREADS;        // x chunks per thread and step
  constexpr int kRowStep = THREADS / kChunks;
  static_assert(PA >= 1 && BM * kChunks % THREADS == 0, "tile shape");
  __shared__ __align__(16) uint16_t sA[2][BM * kLds];

  // XCD-contiguous numbering: dispatch position i runs on XCD i % 8; give each XCD a contiguous
  // range of tiles, column tiles fastest, so a row band's tiles share that XCD's L2.
  const int total = p.tiles_m * p.tiles_n;
  const int i = static_cast<int>(blockIdx.x);
  int tile = i;
  if (total % kXcds == 0) tile = (i % kXcds) * (total / kXcds) + i / kXcds;
  const int64_t m0 = static_cast<int64_t>(tile / p.tiles_n) * BM;
  const int n0 = (tile % p.tiles_n) * BN;

  const int t = static_cast<int>(threadIdx.x);
  const int lane = t & (kWave - 1);
  const int wave = t / kWave;
  const int kc = t % kChunks;  // this thread's chunk of each x row of a step (fixed over K)
  const int r0 = t / kChunks;  // its first row of the band; then every kRowStep rows
  const int fr = lane & 15;        // fragment row (A) / column (B)
  const int fk = (lane >> 4) * 8;  // fragment k offset

  // Every load below reads a valid address (rows past M or N and chunks past K read the last
  // row / chunk) and its value is replaced by zero afterwards: no branch around a load, so the
  // loads of a step issue back to back and retire in order.
  float mean[PA], rstd[PA];
  bool row_ok[PA];
  const char* xrow[PA];
#pragma unroll
  for (int q = 0; q < PA; ++q) {
    const int64_t m = m0 + r0 + q * kRowStep;
    row_ok[q] = m < p.M;
    const int64_t mc = row_ok[q] ? m : p.M - 1;
    mean[q] = 0.f;
    rstd[q] = 1.f;
    if constexpr (LN) {
      mean[q] = p.mean[mc];
      rstd[q] = p.rstd[mc];
    }
    xrow[q] = p.x + mc * p.K * 2;
  }
  // this lane's weight rows (one per 16-column fragment of the wavefront)
  const char* wrow[NI];
  bool col_ok[NI];
#pragma unroll
  for (int c = 0; c < NI; ++c) {
    const int n = n0 + wave * kWaveCols + c * 16 + fr;
    col_ok[c] = n < p.N;
    wrow[c] = p.w + static_cast<int64_t>(col_ok[c] ? n : p.N - 1) * p.K * 2;
  }

  const int nk = (p.K + kBK - 1) / kBK;
  constexpr int PV = LN ? 2 * Elem<PT>::kBytes / 2 : 0;  // 16-byte vectors of gamma + beta per chunk
  // register sets: step s's x chunks (with their gamma / beta) and weight fragments live in set
  // s % U from when they are issued (U steps ahead) until they are used
  uint4 ra[U][PA];
  uint4 rp[U][PV > 0 ? PV : 1];
  bf16x8 wb[U][2][NI];
  const uint4 zero4 = make_uint4(0u, 0u, 0u, 0u);
  auto issue_x = [&](int ks, uint4 (&a)[PA], uint4 (&pp)[PV > 0 ? PV : 1]) {
    const int k = ks * kBK + kc * 8;
    const int kq = k < p.K ? k : p.K - 8;  // steps and chunks past K read the last chunk
#pragma unroll
    for (int q = 0; q < PA; ++q) a[q] = load16(xrow[q] + static_cast<int64_t>(kq) * 2);
    if constexpr (LN) {
      constexpr int H = Elem<PT>::kBytes / 2;  // 16-byte vectors per 8 parameters
#pragma unroll
      for (int h = 0; h < H; ++h) {
        pp[h] = load16(static_cast<const char*>(p.gamma) + static_cast<int64_t>(kq) * Elem<PT>::kBytes + h * 16);
        pp[H + h] = load16(static_cast<const char*>(p.beta) + static_cast<int64_t>(kq) * Elem<PT>::kBytes + h * 16);
      }
    }
  };
  auto issue_w = [&](int ks, bf16x8 (&b)[2][NI]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int k = ks * kBK + h * 32 + fk;
      const int kq = k < p.K ? k : p.K - 8;
#pragma unroll
      for (int c = 0; c < NI; ++c) b[h][c] = __builtin_bit_cast(bf16x8, load16(wrow[c] + static_cast<int64_t>(kq) * 2));
    }
  };
  // zero the weight fragments past K or N (after their loads have been waited for)
  auto mask_w = [&](int ks, bf16x8 (&b)[2][NI]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const bool kin = ks * kBK + h * 32 + fk < p.K;
#pragma unroll
      for (int c = 0; c < NI; ++c)
        if (!(kin && col_ok[c])) b[h][c] = __builtin_bit_cast(bf16x8, zero4);
    }
  };
  auto put_x = [&](int ks, int buf, const uint4 (&a)[PA], const uint4 (&pp)[PV > 0 ? PV : 1]) {
    const bool kin = ks * kBK + kc * 8 < p.K;
    float g[8], bt[8];
    if constexpr (LN) {
      constexpr int H = Elem<PT>::kBytes / 2;
#pragma unroll
      for (int h = 0; h < H; ++h) {
        unpack16(pp[h], g + h * (16 / Elem<PT>::kBytes), PT{});
        unpack16(pp[H + h], bt + h * (16 / Elem<PT>::kBytes), PT{});
      }
    }
#pragma unroll
    for (int q = 0; q < PA; ++q) {
      uint4 v = a[q];
      if constexpr (LN) v = normalise8(a[q], mean[q], rstd[q], g, bt);
      // rows past M and columns past K hold +0 (they must not add beta)
      if (!(row_ok[q] && kin)) v = zero4;
      *reinterpret_cast<uint4*>(&sA[buf][(r0 + q * kRowStep) * kLds + kc * 8]) = v;
    }
  };

  f32x4 acc[MI][NI];
#pragma unroll
  for (int a = 0; a < MI; ++a)
#pragma unroll
    for (int c = 0; c < NI; ++c) acc[a][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto multiply = [&](int buf, const bf16x8 (&b)[2][NI]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int a = 0; a < MI; ++a) {
        const bf16x8 fa = *reinterpret_cast<const bf16x8*>(&sA[buf][(a * 16 + fr) * kLds + h * 32 + fk]);
#pragma unroll
        for (int c = 0; c < NI; ++c) acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa, b[h][c], acc[a][c], 0, 0, 0);
      }
    }
  };

  // steps walked: nk rounded up to a multiple of U (the steps past nk load valid addresses and
  // multiply zeros), so that the unrolled body below holds no branch: the compiler then knows at
  // every use how many loads were issued after the one it waits for
  const int nks = (nk + U - 1) / U * U;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    issue_x(u, ra[u], rp[u]);
    issue_w(u, wb[u]);
  }
  put_x(0, 0, ra[0], rp[0]);
  issue_x(U, ra[0], rp[0]);
  __syncthreads();
  // iteration s writes step s + 1's x chunks (set (s + 1) % U) into the other LDS buffer and
  // refills that set with step s + 1 + U, multiplies step s (LDS buffer s % 2, weight set s % U)
  // and refills the weight set with step s + U; one barrier per step. The body is unrolled U
  // times so that every register set keeps its registers across the loop.
  for (int s0 = 0; s0 < nks; s0 += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = s0 + u;
      put_x(s + 1, (s + 1) & 1, ra[(u + 1) % U], rp[(u + 1) % U]);
      issue_x(s + 1 + U, ra[(u + 1) % U], rp[(u + 1) % U]);
      mask_w(s, wb[u]);
      multiply(s & 1, wb[u]);
      issue_w(s + U, wb[u]);
      __syncthreads();
    }
  }

  // epilogue: + bias, one rounding to the output type
#pragma unroll
  for (int c = 0; c < NI; ++c) {
    const int n = n0 + wave * kWaveCols + c * 16 + fr;
    if (n >= p.N) continue;
    const float bn = p.bias ? Elem<BT>::load(static_cast<const char*>(p.bias) + static_cast<int64_t>(n) * Elem<BT>::kBytes)
                            : 0.f;
#pragma unroll
    for (int a = 0; a < MI; ++a) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + a * 16 + (lane >> 4) * 4 + r;
        if (m < p.M) store_y<OT>(p.y, m * p.N + n, acc[a][c][r] + bn);
      }
    }
  }
}

// Raw buffer over a whole array: byte offsets (voffset from the lane, soffset from the step).
typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                           0x00020000);  // raw buffer, 32-bit data format
}
__device__ __forceinline__ uint4 bload16(Rsrc r, uint32_t voff, uint32_t soff) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// The large form (K a multiple of 128, byte offsets below 2^31): a workgroup of 8 wavefronts
// (2 x 4, each 64 x BN/4) owns a 128 x BN tile of y (BN = 256, or 128 when that leaves fewer
// than two tiles per CU); both
// operands pass through LDS, so each x element loaded feeds BN columns and each weight element
// 128 rows (the L2 -> CU traffic per product that the matrix cores can sustain). x chunks are
// normalised on their way to LDS, once per BN columns. Every load reads inside its array (rows
// past M or N read the last row: their products only reach accumulators that are not stored),
// buffer loads with the step in the scalar offset, U register sets rotating, two LDS buffers, one
// barrier per step, no branch in the loop.
template <int BN, int GN, int U, bool LN, typename PT, typename BT, typename OT>
__global__ void __launch_bounds__(2 * GN * kWave, GN == 2 ? 2 : 1) ln_linear_big_kernel(const LinearParams p) {
  constexpr int BM = 128, THREADS = 2 * GN * kWave;  // 2 x GN wavefronts
  constexpr int WN = BN / GN;                       // wavefront tile 64 x WN
  constexpr int MI = 4, NI = WN / 16;
  constexpr int PA = BM * kChunks / THREADS;        // x chunks per thread and step
  constexpr int PB = BN * kChunks / THREADS;        // weight chunks
  constexpr int kRowStep = THREADS / kChunks;
  constexpr int PV = LN ? Elem<PT>::kBytes : 0;     // 16-byte vectors of gamma + beta per chunk
  // LDS rows of 64 elements (128 bytes), no padding: chunk c of row r sits in slot c ^ (r & 7), so
  // the 16-byte chunk writes and the fragment reads meet no bank conflicts (2.75 M conflict cycles
  // per launch with rows padded to 72 elements)
  constexpr int kStageA = BM * kBK, kStageB = BN * kBK;
  __shared__ __align__(16) uint16_t sA[2][kStageA];
  __shared__ __align__(16) uint16_t sB[2][kStageB];

  const int total = p.tiles_m * p.tiles_n;
  const int i = static_cast<int>(blockIdx.x);
  int tile = i;
  if (total % kXcds == 0) tile = (i % kXcds) * (total / kXcds) + i / kXcds;
  const int64_t m0 = static_cast<int64_t>(tile / p.tiles_n) * BM;
  const int n0 = (tile % p.tiles_n) * BN;

  const int t = static_cast<int>(threadIdx.x);
  const int lane = t & (kWave - 1);
  const int wave = t / kWave;
  const int wm = wave / GN, wn = wave % GN;
  const int kc = t % kChunks, r0 = t / kChunks;
  const int fr = lane & 15, fk = (lane >> 4) * 8;

  const Rsrc xr = make_rsrc(p.x, static_cast<uint32_t>(p.M * p.K * 2));
  const Rsrc wr = make_rsrc(p.w, static_cast<uint32_t>(static_cast<int64_t>(p.N) * p.K * 2));
  const Rsrc gr = LN ? make_rsrc(p.gamma, static_cast<uint32_t>(p.K * Elem<PT>::kBytes)) : wr;
  const Rsrc br = LN ? make_rsrc(p.beta, static_cast<uint32_t>(p.K * Elem<PT>::kBytes)) : wr;
  const uint32_t poff = kc * 8 * Elem<PT>::kBytes;
  float mean[PA], rstd[PA];
  uint32_t xoff[PA], woff[PB];
#pragma unroll
  for (int q = 0; q < PA; ++q) {
    const int64_t m = m0 + r0 + q * kRowStep;
    const int64_t mc = m < p.M ? m : p.M - 1;
    mean[q] = 0.f;
    rstd[q] = 1.f;
    if constexpr (LN) {
      mean[q] = p.mean[mc];
      rstd[q] = p.rstd[mc];
    }
    xoff[q] = static_cast<uint32_t>((mc * p.K + kc * 8) * 2);
  }
#pragma unroll
  for (int q = 0; q < PB; ++q) {
    const int n = n0 + r0 + q * kRowStep;
    woff[q] = static_cast<uint32_t>((static_cast<int64_t>(n < p.N ? n : p.N - 1) * p.K + kc * 8) * 2);
  }

  // this workgroup's steps of K: all of them, or split blockIdx.y's range (an even count)
  const int nk_all = p.K / kBK;
  const int ks0 = p.part ? static_cast<int>(blockIdx.y) * p.split_steps : 0;
  const int nk = p.part ? (nk_all - ks0 < p.split_steps ? nk_all - ks0 : p.split_steps) : nk_all;
  uint4 ra[U][PA], rb[U][PB];
  uint4 rp[U][PV > 0 ? PV : 1];
  auto issue = [&](int ks, uint4 (&a)[PA], uint4 (&b)[PB], uint4 (&pp)[PV > 0 ? PV : 1]) {
    const uint32_t kq = static_cast<uint32_t>(ks0 + (ks < nk ? ks : nk - 1));  // later steps are never used
#pragma unroll
    for (int q = 0; q < PA; ++q) a[q] = bload16(xr, xoff[q], kq * kBK * 2);
    if constexpr (LN) {
      constexpr int HV = Elem<PT>::kBytes / 2;
#pragma unroll
      for (int h = 0; h < HV; ++h) {
        pp[h] = bload16(gr, poff + h * 16, kq * kBK * Elem<PT>::kBytes);
        pp[HV + h] = bload16(br, poff + h * 16, kq * kBK * Elem<PT>::kBytes);
      }
    }
#pragma unroll
    for (int q = 0; q < PB; ++q) b[q] = bload16(wr, woff[q], kq * kBK * 2);
  };
  auto put = [&](int buf, const uint4 (&a)[PA], const uint4 (&b)[PB], const uint4 (&pp)[PV > 0 ? PV : 1]) {
    float g[8], bt[8];
    if constexpr (LN) {
      constexpr int HV = Elem<PT>::kBytes / 2;
#pragma unroll
      for (int h = 0; h < HV; ++h) {
        unpack16(pp[h], g + h * (16 / Elem<PT>::kBytes), PT{});
        unpack16(pp[HV + h], bt + h * (16 / Elem<PT>::kBytes), PT{});
      }
    }
#pragma unroll
    for (int q = 0; q < PA; ++q) {
      uint4 v = a[q];
      if constexpr (LN) v = normalise8(a[q], mean[q], rstd[q], g, bt);
      *reinterpret_cast<uint4*>(&sA[buf][(r0 + q * kRowStep) * kBK + ((kc ^ (r0 & 7)) << 3)]) = v;
    }
#pragma unroll
    for (int q = 0; q < PB; ++q) *reinterpret_cast<uint4*>(&sB[buf][(r0 + q * kRowStep) * kBK + ((kc ^ (r0 & 7)) << 3)]) = b[q];
  };

  f32x4 acc[MI][NI];
#pragma unroll
  for (int a = 0; a < MI; ++a)
#pragma unroll
    for (int c = 0; c < NI; ++c) acc[a][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto multiply = [&](int buf) {
    // every fragment of the step is read first (16 LDS reads in flight), then the products; a
    // fragment row's r & 7 is fr & 7 (the other terms of the row are multiples of 8)
    bf16x8 fa[2][MI], fb[2][NI];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int c = 0; c < NI; ++c)
        fb[h][c] = *reinterpret_cast<const bf16x8*>(&sB[buf][(wn * WN + c * 16 + fr) * kBK + ((((h * 32 + fk) >> 3) ^ (fr & 7)) << 3)]);
#pragma unroll
      for (int a = 0; a < MI; ++a)
        fa[h][a] = *reinterpret_cast<const bf16x8*>(&sA[buf][(wm * 64 + a * 16 + fr) * kBK + ((((h * 32 + fk) >> 3) ^ (fr & 7)) << 3)]);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int a = 0; a < MI; ++a)
#pragma unroll
        for (int c = 0; c < NI; ++c)
          acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[h][a], fb[h][c], acc[a][c], 0, 0, 0);
  };

#pragma unroll
  for (int u = 0; u < U; ++u) issue(u, ra[u], rb[u], rp[u]);
  put(0, ra[0], rb[0], rp[0]);
  // kept after the write that reads set 0: hoisted above it, these loads would need registers
  // of their own, and the loop would begin with copies that wait for every load in flight
  __builtin_amdgcn_sched_barrier(0);
  issue(U, ra[0], rb[0], rp[0]);
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  // iteration s writes step s + 1 (set (s + 1) % U) into the other LDS buffer and refills that
  // set with step s + 1 + U, then multiplies step s; nk is a multiple of U, so the unrolled body
  // holds no branch and each register set keeps its registers across the loop (step nk's write
  // goes to a buffer that is not read again)
  for (int s0 = 0; s0 < nk; s0 += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = s0 + u;
      put((s + 1) & 1, ra[(u + 1) % U], rb[(u + 1) % U], rp[(u + 1) % U]);
      // the scheduling barriers keep each phase where it is written: loads moved next to
      // their use would be waited for at once
      __builtin_amdgcn_sched_barrier(0);
      issue(s + 1 + U, ra[(u + 1) % U], rb[(u + 1) % U], rp[(u + 1) % U]);
      __builtin_amdgcn_sched_barrier(0);
      multiply(s & 1);
      __syncthreads();
    }
  }

  if (p.part) {  // split K: this split's fp32 partial products, added up by the reduction kernel
    float* const part = p.part + static_cast<int64_t>(blockIdx.y) * p.M * p.N;
#pragma unroll
    for (int c = 0; c < NI; ++c) {
      const int n = n0 + wn * WN + c * 16 + fr;
      if (n >= p.N) continue;
#pragma unroll
      for (int a = 0; a < MI; ++a) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t m = m0 + wm * 64 + a * 16 + (lane >> 4) * 4 + r;
          if (m < p.M) part[m * p.N + n] = acc[a][c][r];
        }
      }
    }
    return;
  }
  // epilogue: + bias, one rounding to the output type
#pragma unroll
  for (int c = 0; c < NI; ++c) {
    const int n = n0 + wn * WN + c * 16 + fr;
    if (n >= p.N) continue;
    const float bn = p.bias ? Elem<BT>::load(static_cast<const char*>(p.bias) + static_cast<int64_t>(n) * Elem<BT>::kBytes)
                            : 0.f;
#pragma unroll
    for (int a = 0; a < MI; ++a) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + wm * 64 + a * 16 + (lane >> 4) * 4 + r;
        if (m < p.M) store_y<OT>(p.y, m * p.N + n, acc[a][c][r] + bn);
      }
    }
  }
}

// Split K: y[m, n] = (sum over splits, in split order, of the fp32 partials) + bias, one rounding.
// Four consecutive elements per thread (16-byte loads of each split's partials; M * N is a
// multiple of 4, so every split's block stays 16-byte aligned), the last thread taking the rest.
template <typename BT, typename OT>
__global__ void __launch_bounds__(256) ln_linear_reduce_kernel(const LinearParams p, int32_t splits) {
  const int64_t total = p.M * p.N;
  const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i0 >= total) return;
  float v[4];
  const int cnt = total - i0 < 4 ? static_cast<int>(total - i0) : 4;
  if (total % 4 == 0) {  // then cnt == 4
    const float4 q0 = *reinterpret_cast<const float4*>(p.part + i0);
    v[0] = q0.x;
    v[1] = q0.y;
    v[2] = q0.z;
    v[3] = q0.w;
    for (int sp = 1; sp < splits; ++sp) {
      const float4 q = *reinterpret_cast<const float4*>(p.part + static_cast<int64_t>(sp) * total + i0);
      v[0] += q.x;
      v[1] += q.y;
      v[2] += q.z;
      v[3] += q.w;
    }
  } else {
    for (int e = 0; e < cnt; ++e) v[e] = p.part[i0 + e];
    for (int sp = 1; sp < splits; ++sp)
      for (int e = 0; e < cnt; ++e) v[e] += p.part[static_cast<int64_t>(sp) * total + i0 + e];
  }
  for (int e = 0; e < cnt; ++e) {
    const int n = static_cast<int>((i0 + e) % p.N);
    const float bn = p.bias ? Elem<BT>::load(static_cast<const char*>(p.bias) + static_cast<int64_t>(n) * Elem<BT>::kBytes)
                            : 0.f;
    store_y<OT>(p.y, i0 + e, v[e] + bn);
  }
}

template <int BN, int GN, int U, bool LN, typename PT, typename BT, typename OT>
hipError_t launch_big(LinearParams p, int splits, hipStream_t s) {
  p.tiles_m = static_cast<int32_t>((p.M + 127) / 128);
  p.tiles_n = (p.N + BN - 1) / BN;
  const int64_t blocks = static_cast<int64_t>(p.tiles_m) * p.tiles_n;
  if (splits <= 1) p.part = nullptr;
  hipLaunchKernelGGL((ln_linear_big_kernel<BN, GN, U, LN, PT, BT, OT>),
                     dim3(static_cast<unsigned>(blocks), static_cast<unsigned>(splits > 1 ? splits : 1)),
                     dim3(2 * GN * kWave), 0, s, p);
  if (splits > 1) {
    const int64_t threads = (p.M * p.N + 3) / 4;
    hipLaunchKernelGGL((ln_linear_reduce_kernel<BT, OT>), dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256),
                       0, s, p, splits);
  }
  return hipGetLastError();
}

template <int BM, int WAVES, int U, bool LN, typename PT, typename BT, typename OT>
hipError_t launch_tile(LinearParams p, hipStream_t s) {
  p.tiles_m = static_cast<int32_t>((p.M + BM - 1) / BM);
  p.tiles_n = (p.N + WAVES * kWaveCols - 1) / (WAVES * kWaveCols);
  const int64_t blocks = static_cast<int64_t>(p.tiles_m) * p.tiles_n;
  hipLaunchKernelGGL((ln_linear_kernel<BM, WAVES, U, LN, PT, BT, OT>), dim3(static_cast<unsigned>(blocks)),
                     dim3(WAVES * kWave), 0, s, p);
  return hipGetLastError();
}

// The large form applies to K a multiple of 128 with byte offsets below 2^31 (every encoder shape:
// K = 28 * D).
bool big_form(int64_t M, int32_t N, int32_t K) {
  return K % (2 * kBK) == 0 && (M + 128) * K * 2 < (int64_t{1} << 31) && static_cast<int64_t>(N) * K * 2 < (int64_t{1} << 31);
}

// Split K for the large form: enough splits that its 128 x 128 tiles give one workgroup per CU
// (each split at least two steps of kBK, an even count), as many as `ws_bytes` of fp32 partials
// hold; 1 = no split. `steps` receives the steps per split. (Two workgroups per CU measured
// slower: M = 1024, K = 3584, N = 512 took 28.0 against 18.7 us, the partials' HBM traffic
// outweighing the extra parallelism.)
int split_count(int64_t M, int32_t N, int32_t K, int64_t ws_bytes, int* steps) {
  const int nk = K / kBK;
  *steps = nk;
  const int64_t tiles = (M + 127) / 128 * ((N + 127) / 128);
  if (tiles >= kSplitTarget || nk < 4) return 1;
  int64_t want = (kSplitTarget + tiles - 1) / tiles;
  const int64_t fit = ws_bytes / (M * N * 4);
  if (want > fit) want = fit;
  if (want > nk / 2) want = nk / 2;
  if (want <= 1) return 1;
  const int per = static_cast<int>(((nk + want - 1) / want + 1) / 2 * 2);  // even steps per split
  *steps = per;
  return (nk + per - 1) / per;
}

// 128 x 256 tiles when there are at least two per CU, else 128 x 128 (split over K when even
// those leave CUs idle); the general form for the rest.
template <bool LN, typename PT, typename BT, typename OT>
hipError_t launch_linear(const LinearParams& p, int64_t ws_bytes, hipStream_t s) {
  if (big_form(p.M, p.N, p.K)) {
    if ((p.M + 127) / 128 * ((p.N + 255) / 256) >= 2 * 256) return launch_big<256, 4, 2, LN, PT, BT, OT>(p, 1, s);
    LinearParams q = p;
    int steps = 0;
    const int splits = p.part ? split_count(p.M, p.N, p.K, ws_bytes, &steps) : 1;
    q.split_steps = steps;
    return launch_big<128, 4, 2, LN, PT, BT, OT>(q, splits, s);
  }
  return launch_tile<64, 4, 2, LN, PT, BT, OT>(p, s);
}

template <bool LN, typename PT, typename BT>
hipError_t launch_out(int32_t odt, const LinearParams& p, int64_t ws, hipStream_t s) {
  return odt == CTI_EBAG_F32 ? launch_linear<LN, PT, BT, float>(p, ws, s) : launch_linear<LN, PT, BT, bf16_t>(p, ws, s);
}

template <bool LN, typename PT>
hipError_t launch_bias(int32_t bdt, int32_t odt, const LinearParams& p, int64_t ws, hipStream_t s) {
  return bdt == CTI_EBAG_F32 ? launch_out<LN, PT, float>(odt, p, ws, s) : launch_out<LN, PT, bf16_t>(odt, p, ws, s);
}

}  // namespace
}  // namespace cti

using namespace cti;

extern "C" int64_t cti_ebag_layernorm_linear_workspace_bytes(int64_t rows, int32_t cols, int32_t out_features) {
  if (rows < 1 || cols < 1 || out_features < 1 || !big_form(rows, out_features, cols)) return 0;
  int steps = 0;
  const int splits = split_count(rows, out_features, cols, INT64_MAX, &steps);
  return splits > 1 ? static_cast<int64_t>(splits) * rows * out_features * 4 : 0;
}

extern "C" int cti_ebag_layernorm_linear(const void* x, int64_t rows, int32_t cols, const float* mean,
                                         const float* rstd, const void* gamma, const void* beta, int32_t param_dtype,
                                         const void* weight, int32_t out_features, const void* bias,
                                         int32_t bias_dtype, void* y, int32_t y_dtype, void* workspace,
                                         int64_t workspace_bytes, void* stream) {
  clear_error();
  if (rows < 0) return set_error(CTI_EBAG_EINVAL, "rows must be >= 0 (got %lld)", (long long)rows);
  if (cols < 1 || out_features < 1)
    return set_error(CTI_EBAG_EINVAL, "cols and out_features must be >= 1 (got %d, %d)", cols, out_features);
  if (cols % 8 != 0)
    return set_error(CTI_EBAG_EUNSUPPORTED, "cols must be a multiple of 8 (16-byte rows; got %d)", cols);
  const bool ln = mean != nullptr || rstd != nullptr || gamma != nullptr || beta != nullptr;
  if (ln && !(mean && rstd && gamma && beta))
    return set_error(CTI_EBAG_EINVAL, "mean, rstd, gamma and beta must be given together (or none of them)");
  if (ln && param_dtype != CTI_EBAG_F32 && param_dtype != CTI_EBAG_BF16)
    return set_error(CTI_EBAG_EINVAL, "gamma / beta must be fp32 or bf16 (dtype code %d)", param_dtype);
  if (bias && bias_dtype != CTI_EBAG_F32 && bias_dtype != CTI_EBAG_BF16)
    return set_error(CTI_EBAG_EINVAL, "bias must be fp32 or bf16 (dtype code %d)", bias_dtype);
  if (y_dtype != CTI_EBAG_F32 && y_dtype != CTI_EBAG_BF16)
    return set_error(CTI_EBAG_EINVAL, "the output must be fp32 or bf16 (dtype code %d)", y_dtype);
  if (rows == 0) return CTI_EBAG_OK;
  if (!x || !weight || !y) return set_error(CTI_EBAG_EINVAL, "NULL device pointer among x / weight / y");
  const auto a16 = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
  if (!a16(x) || !a16(weight) || (ln && (!a16(gamma) || !a16(beta))))
    return set_error(CTI_EBAG_EINVAL, "x, weight, gamma and beta must be 16-byte aligned");
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace))
    return set_error(CTI_EBAG_EINVAL, "workspace_bytes %lld without a workspace", (long long)workspace_bytes);
  if (workspace && !a16(workspace)) return set_error(CTI_EBAG_EINVAL, "the workspace must be 16-byte aligned");
  if (rows > (int64_t{INT32_MAX} / 2) * 64 || (rows + 63) / 64 * ((out_features + 255) / 256) > INT32_MAX)
    return set_error(CTI_EBAG_EUNSUPPORTED, "%lld rows x %d outputs need too many tiles", (long long)rows, out_features);
  LinearParams p{};
  p.x = static_cast<const char*>(x);
  p.mean = mean;
  p.rstd = rstd;
  p.gamma = gamma;
  p.beta = beta;
  p.w = static_cast<const char*>(weight);
  p.bias = bias;
  p.y = static_cast<char*>(y);
  p.M = rows;
  p.N = out_features;
  p.K = cols;
  p.part = workspace_bytes > 0 ? static_cast<float*>(workspace) : nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  const int32_t bdt = bias ? bias_dtype : CTI_EBAG_F32;
  const int64_t ws = p.part ? workspace_bytes : 0;
  if (!ln) e = launch_bias<false, float>(bdt, y_dtype, p, ws, s);
  else if (param_dtype == CTI_EBAG_F32) e = launch_bias<true, float>(bdt, y_dtype, p, ws, s);
  else e = launch_bias<true, bf16_t>(bdt, y_dtype, p, ws, s);
  if (e != hipSuccess) return set_error(CTI_EBAG_EHIP, "layernorm-linear launch failed: %s", hipGetErrorString(e));
  return CTI_EBAG_OK;
}
