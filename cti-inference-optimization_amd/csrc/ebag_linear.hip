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
// Mapping: workgroups of 4 wavefronts own a BM x BN tile of y (wavefronts 2 x 2, each
// (BM/2) x (BN/2)) and walk K in steps of 64: the next step's x and w tiles are loaded into
// registers while the matrix cores work on the current one from LDS (rows padded to 72
// elements, so the 16-byte fragment reads of 16 rows hit distinct banks). The products are
// v_mfma_f32_16x16x32_bf16: lane l supplies A[l%16][8(l/16) .. +8) and B[8(l/16) .. +8)[l%16]
// and receives C[4(l/16) + r][l%16], r < 4. Workgroups are numbered so that the tiles of one
// row band of x run on one XCD (its L2 then serves x's rows to every column tile of the band).
#include <stdint.h>

#include "ebag_device.h"
#include "ebag_internal.h"

namespace cti {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kLinThreads = 256;          // 4 wavefronts
constexpr int kBK = 64;                   // K per step
constexpr int kLds = kBK + 8;             // LDS row pitch in elements (144 bytes)
constexpr int kChunks = kBK / 8;          // 16-byte chunks per tile row
constexpr int kXcds = 8;

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
};

template <typename PT>
__device__ __forceinline__ void load_param8(const void* p, int32_t k, bool live, float* out) {
  if (!live) {
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = 0.f;
    return;
  }
  load_params<PT, 8>(p, k, out);
}

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

template <int BM, int BN, bool LN, typename PT, typename BT, typename OT>
__global__ void __launch_bounds__(kLinThreads) ln_linear_kernel(const LinearParams p) {
  constexpr int WM = BM / 2, WN = BN / 2;     // wavefront tile
  constexpr int MI = WM / 16, NI = WN / 16;   // 16 x 16 products per wavefront
  constexpr int PA = BM * kChunks / kLinThreads;  // x chunks per thread and step
  constexpr int PB = BN * kChunks / kLinThreads;  // w chunks per thread and step
  static_assert(PA >= 1 && PB >= 1 && MI >= 1 && NI >= 1, "tile shape");
  __shared__ __align__(16) uint16_t sA[BM * kLds];
  __shared__ __align__(16) uint16_t sB[BN * kLds];

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
  const int wm = wave >> 1, wn = wave & 1;
  const int kc = t % kChunks;  // this thread's chunk of each tile row (fixed over the K loop)
  const int r0 = t / kChunks;  // its first tile row; then every kLinThreads / kChunks rows
  constexpr int kRowStep = kLinThreads / kChunks;

  float mean[PA], rstd[PA];
#pragma unroll
  for (int q = 0; q < PA; ++q) {
    const int64_t m = m0 + r0 + q * kRowStep;
    mean[q] = 0.f;
    rstd[q] = 1.f;
    if constexpr (LN) {
      if (m < p.M) {
        mean[q] = p.mean[m];
        rstd[q] = p.rstd[m];
      }
    }
  }

  uint4 ra[PA], rb[PB];
  float g[8], b[8];
  const int nk = (p.K + kBK - 1) / kBK;
  auto load_step = [&](int ks) {
    const int k = ks * kBK + kc * 8;
    const bool kin = k < p.K;
#pragma unroll
    for (int q = 0; q < PA; ++q) {
      const int64_t m = m0 + r0 + q * kRowStep;
      ra[q] = (kin && m < p.M) ? load16(p.x + (m * p.K + k) * 2) : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int q = 0; q < PB; ++q) {
      const int n = n0 + r0 + q * kRowStep;
      rb[q] = (kin && n < p.N) ? load16(p.w + (static_cast<int64_t>(n) * p.K + k) * 2) : make_uint4(0u, 0u, 0u, 0u);
    }
    if constexpr (LN) {
      load_param8<PT>(p.gamma, k, kin, g);
      load_param8<PT>(p.beta, k, kin, b);
    }
  };
  auto store_step = [&](int ks) {
    const int k = ks * kBK + kc * 8;
#pragma unroll
    for (int q = 0; q < PA; ++q) {
      const int row = r0 + q * kRowStep;
      uint4 v = ra[q];
      if constexpr (LN) {
        // rows past M and columns past K hold +0 (they must not add beta)
        if (m0 + row < p.M && k < p.K) v = normalise8(ra[q], mean[q], rstd[q], g, b);
      }
      *reinterpret_cast<uint4*>(&sA[row * kLds + kc * 8]) = v;
    }
#pragma unroll
    for (int q = 0; q < PB; ++q) {
      const int row = r0 + q * kRowStep;
      *reinterpret_cast<uint4*>(&sB[row * kLds + kc * 8]) = rb[q];
    }
  };

  f32x4 acc[MI][NI];
#pragma unroll
  for (int a = 0; a < MI; ++a)
#pragma unroll
    for (int c = 0; c < NI; ++c) acc[a][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  load_step(0);
  store_step(0);
  __syncthreads();
  const int fr = lane & 15;        // fragment row (A) / column (B)
  const int fk = (lane >> 4) * 8;  // fragment k offset
  for (int ks = 0; ks < nk; ++ks) {
    if (ks + 1 < nk) load_step(ks + 1);
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 32) {
      bf16x8 fa[MI], fb[NI];
#pragma unroll
      for (int a = 0; a < MI; ++a)
        fa[a] = *reinterpret_cast<const bf16x8*>(&sA[(wm * WM + a * 16 + fr) * kLds + kk + fk]);
#pragma unroll
      for (int c = 0; c < NI; ++c)
        fb[c] = *reinterpret_cast<const bf16x8*>(&sB[(wn * WN + c * 16 + fr) * kLds + kk + fk]);
#pragma unroll
      for (int a = 0; a < MI; ++a)
#pragma unroll
        for (int c = 0; c < NI; ++c) acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[a], fb[c], acc[a][c], 0, 0, 0);
    }
    __syncthreads();
    if (ks + 1 < nk) {
      store_step(ks + 1);
      __syncthreads();
    }
  }

  // epilogue: + bias, one rounding to the output type
#pragma unroll
  for (int c = 0; c < NI; ++c) {
    const int n = n0 + wn * WN + c * 16 + (lane & 15);
    if (n >= p.N) continue;
    const float bn = p.bias ? Elem<BT>::load(static_cast<const char*>(p.bias) + static_cast<int64_t>(n) * Elem<BT>::kBytes)
                            : 0.f;
#pragma unroll
    for (int a = 0; a < MI; ++a) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + wm * WM + a * 16 + (lane >> 4) * 4 + r;
        if (m < p.M) store_y<OT>(p.y, m * p.N + n, acc[a][c][r] + bn);
      }
    }
  }
}

template <int BM, int BN, bool LN, typename PT, typename BT, typename OT>
hipError_t launch_tile(LinearParams p, hipStream_t s) {
  p.tiles_m = static_cast<int32_t>((p.M + BM - 1) / BM);
  p.tiles_n = (p.N + BN - 1) / BN;
  const int64_t blocks = static_cast<int64_t>(p.tiles_m) * p.tiles_n;
  hipLaunchKernelGGL((ln_linear_kernel<BM, BN, LN, PT, BT, OT>), dim3(static_cast<unsigned>(blocks)),
                     dim3(kLinThreads), 0, s, p);
  return hipGetLastError();
}

// Tile shape by the number of tiles it makes: 128 x 128 when that fills the chip (256 CUs) at
// least once, else 64 x 128.
template <bool LN, typename PT, typename BT, typename OT>
hipError_t launch_linear(const LinearParams& p, hipStream_t s) {
  const int64_t big = ((p.M + 127) / 128) * ((p.N + 127) / 128);
  if (big >= 256) return launch_tile<128, 128, LN, PT, BT, OT>(p, s);
  return launch_tile<64, 128, LN, PT, BT, OT>(p, s);
}

template <bool LN, typename PT, typename BT>
hipError_t launch_out(int32_t odt, const LinearParams& p, hipStream_t s) {
  return odt == CTI_EBAG_F32 ? launch_linear<LN, PT, BT, float>(p, s) : launch_linear<LN, PT, BT, bf16_t>(p, s);
}

template <bool LN, typename PT>
hipError_t launch_bias(int32_t bdt, int32_t odt, const LinearParams& p, hipStream_t s) {
  return bdt == CTI_EBAG_F32 ? launch_out<LN, PT, float>(odt, p, s) : launch_out<LN, PT, bf16_t>(odt, p, s);
}

}  // namespace
}  // namespace cti

using namespace cti;

extern "C" int cti_ebag_layernorm_linear(const void* x, int64_t rows, int32_t cols, const float* mean,
                                         const float* rstd, const void* gamma, const void* beta, int32_t param_dtype,
                                         const void* weight, int32_t out_features, const void* bias,
                                         int32_t bias_dtype, void* y, int32_t y_dtype, void* stream) {
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
  if (rows > (int64_t{INT32_MAX} / 2) * 64 || (rows + 63) / 64 * ((out_features + 127) / 128) > INT32_MAX)
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
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  const int32_t bdt = bias ? bias_dtype : CTI_EBAG_F32;
  if (!ln) e = launch_bias<false, float>(bdt, y_dtype, p, s);
  else if (param_dtype == CTI_EBAG_F32) e = launch_bias<true, float>(bdt, y_dtype, p, s);
  else e = launch_bias<true, bf16_t>(bdt, y_dtype, p, s);
  if (e != hipSuccess) return set_error(CTI_EBAG_EHIP, "layernorm-linear launch failed: %s", hipGetErrorString(e));
  return CTI_EBAG_OK;
}
