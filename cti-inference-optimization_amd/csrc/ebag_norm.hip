// Row LayerNorm over the pooled block [rows, cols] (the encoder's input norm) for MI355X (gfx950).
//
// Semantics follow the reference kernel online_best/infer.py:829-858:
//   mean = sum(x) / cols;  var = sum((x - mean)^2) / cols;  rstd = 1 / sqrt(var + eps)
//   y = (x - mean) * rstd * gamma + beta
// in fp32, with one rounding to the output type; the per-row mean and rstd are optional outputs.
//
// This is an HBM-bound pass (read the row once, write it once): one workgroup per row holds the
// row in registers as 16-byte vectors (up to 8 per thread): one wavefront for rows of up to 512
// vectors (4,096 bf16 columns; the reductions are then lane shuffles only), four wavefronts for
// rows of up to 2,048 vectors (16,384 bf16 or 8,192 fp32 columns). The two reductions combine
// per-thread partial sums through an xor butterfly and, across wavefronts, LDS in a fixed order,
// so results are deterministic. gamma and beta are read as 16-byte vectors. Rows that are not
// whole 16-byte vectors, misaligned buffers or longer rows use a loop kernel that reads the row
// three times.
#include <stdint.h>

#include "ebag_device.h"
#include "ebag_internal.h"

namespace cti {
namespace {

constexpr int kNormThreads = 256;  // the loop kernel and the widest register kernel
constexpr int kNormWaves = kNormThreads / kWave;
constexpr int kNormMaxVecs = 8;  // 16-byte vectors per thread held in registers

struct NormParams {
  const char* x;
  char* y;
  const void* gamma;
  const void* beta;
  float* mean_out;
  float* rstd_out;
  int64_t rows;
  int64_t cols;
  float eps;
  int32_t stream_out;  // the output is at least kStreamOutBytes: non-temporal stores
};

template <typename PT>
__device__ __forceinline__ float load_param(const void* p, int64_t i) {
  return Elem<PT>::load(static_cast<const char*>(p) + i * Elem<PT>::kBytes);
}

// One row per workgroup of WAVES wavefronts, the row in registers: thread t holds vectors
// t, t + THREADS, ... (K of them).
template <typename T, typename PT, int K, int WAVES>
__global__ void __launch_bounds__(WAVES * kWave) norm_rows_kernel(const NormParams p) {
  constexpr int VEC = 16 / Elem<T>::kBytes;
  constexpr int THREADS = WAVES * kWave;
  __shared__ float s_red[WAVES];
  const int64_t row = blockIdx.x;
  const int t = static_cast<int>(threadIdx.x);
  const int nvec = static_cast<int>(p.cols / VEC);
  const char* xr = p.x + row * p.cols * Elem<T>::kBytes;

  float v[K][VEC];
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int i = t + k * THREADS;
    const uint4 raw = i < nvec ? load16(xr + static_cast<int64_t>(i) * 16) : make_uint4(0u, 0u, 0u, 0u);
    unpack16(raw, v[k], T{});
#pragma unroll
    for (int e = 0; e < VEC; ++e) s += v[k][e];  // padding vectors hold +0
  }
  const float n = static_cast<float>(p.cols);
  const float mean = block_sum<WAVES>(s, s_red) / n;
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const bool live = t + k * THREADS < nvec;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      v[k][e] = live ? v[k][e] - mean : 0.f;
      q += v[k][e] * v[k][e];
    }
  }
  const float var = block_sum<WAVES>(q, s_red) / n;
  const float rstd = 1.0f / __builtin_sqrtf(var + p.eps);
  if (t == 0) {
    if (p.mean_out) p.mean_out[row] = mean;
    if (p.rstd_out) p.rstd_out[row] = rstd;
  }
  if (!p.y) return;  // statistics only
  T* yr = reinterpret_cast<T*>(p.y + row * p.cols * Elem<T>::kBytes);
  with_stream(p.stream_out, [&](auto stream) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int i = t + k * THREADS;
      if (i < nvec) {
        float gm[VEC], bt[VEC], r[VEC];
        load_params<PT, VEC>(p.gamma, static_cast<int64_t>(i) * VEC, gm);
        load_params<PT, VEC>(p.beta, static_cast<int64_t>(i) * VEC, bt);
#pragma unroll
        for (int e = 0; e < VEC; ++e) r[e] = v[k][e] * rstd * gm[e] + bt[e];
        store_out<VEC>(yr + static_cast<int64_t>(i) * VEC, r, decltype(stream)::value);
      }
    }
  });
}

// Any width and alignment: three passes over the row (sum, squared deviations, output).
template <typename T, typename PT>
__global__ void __launch_bounds__(kNormThreads) norm_rows_loop_kernel(const NormParams p) {
  __shared__ float s_red[kNormWaves];
  const int64_t row = blockIdx.x;
  const char* xr = p.x + row * p.cols * Elem<T>::kBytes;
  float s = 0.f;
  for (int64_t c = threadIdx.x; c < p.cols; c += kNormThreads) s += Elem<T>::load(xr + c * Elem<T>::kBytes);
  const float n = static_cast<float>(p.cols);
  const float mean = block_sum<kNormWaves>(s, s_red) / n;
  float q = 0.f;
  for (int64_t c = threadIdx.x; c < p.cols; c += kNormThreads) {
    const float d = Elem<T>::load(xr + c * Elem<T>::kBytes) - mean;
    q += d * d;
  }
  const float var = block_sum<kNormWaves>(q, s_red) / n;
  const float rstd = 1.0f / __builtin_sqrtf(var + p.eps);
  if (threadIdx.x == 0) {
    if (p.mean_out) p.mean_out[row] = mean;
    if (p.rstd_out) p.rstd_out[row] = rstd;
  }
  if (!p.y) return;  // statistics only
  T* yr = reinterpret_cast<T*>(p.y + row * p.cols * Elem<T>::kBytes);
  with_stream(p.stream_out, [&](auto stream) {
    for (int64_t c = threadIdx.x; c < p.cols; c += kNormThreads) {
      const float d = Elem<T>::load(xr + c * Elem<T>::kBytes) - mean;
      store_one(yr + c, d * rstd * load_param<PT>(p.gamma, c) + load_param<PT>(p.beta, c), decltype(stream)::value);
    }
  });
}

template <typename T, typename PT>
hipError_t launch_norm(const NormParams& p, hipStream_t s) {
  constexpr int VEC = 16 / Elem<T>::kBytes;
  const auto a16 = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
  const bool aligned = a16(p.x) && (!p.y || (a16(p.y) && a16(p.gamma) && a16(p.beta))) && p.cols % VEC == 0;
  const int64_t nvec = p.cols / VEC;
  const dim3 grid(static_cast<unsigned>(p.rows));
  const dim3 one(kWave), four(4 * kWave);
  if (!aligned || nvec > int64_t{4 * kWave} * kNormMaxVecs) {
    hipLaunchKernelGGL((norm_rows_loop_kernel<T, PT>), grid, dim3(kNormThreads), 0, s, p);
  } else if (nvec <= 2 * kWave) {
    hipLaunchKernelGGL((norm_rows_kernel<T, PT, 2, 1>), grid, one, 0, s, p);
  } else if (nvec <= 4 * kWave) {
    hipLaunchKernelGGL((norm_rows_kernel<T, PT, 4, 1>), grid, one, 0, s, p);
  } else if (nvec <= 8 * kWave) {
    hipLaunchKernelGGL((norm_rows_kernel<T, PT, 8, 1>), grid, one, 0, s, p);
  } else if (nvec <= 16 * kWave) {
    hipLaunchKernelGGL((norm_rows_kernel<T, PT, 4, 4>), grid, four, 0, s, p);
  } else {
    hipLaunchKernelGGL((norm_rows_kernel<T, PT, 8, 4>), grid, four, 0, s, p);
  }
  return hipGetLastError();
}

template <typename T>
hipError_t launch_norm_typed(int32_t pdt, const NormParams& p, hipStream_t s) {
  switch (pdt) {
    case CTI_EBAG_F32: return launch_norm<T, float>(p, s);
    case CTI_EBAG_BF16: return launch_norm<T, bf16_t>(p, s);
    default: return launch_norm<T, f16_t>(p, s);
  }
}

bool norm_dtype_ok(int32_t dt) { return dt == CTI_EBAG_F32 || dt == CTI_EBAG_BF16 || dt == CTI_EBAG_F16; }

}  // namespace
}  // namespace cti

using namespace cti;

extern "C" int cti_ebag_layernorm(const void* x, void* y, int64_t rows, int64_t cols, int32_t dtype,
                                  const void* gamma, const void* beta, int32_t param_dtype, float eps,
                                  float* mean_out, float* rstd_out, void* stream) {
  clear_error();
  if (rows < 0) return set_error(CTI_EBAG_EINVAL, "rows must be >= 0 (got %lld)", (long long)rows);
  if (cols < 1) return set_error(CTI_EBAG_EINVAL, "cols must be >= 1 (got %lld)", (long long)cols);
  if (!norm_dtype_ok(dtype)) return set_error(CTI_EBAG_EINVAL, "unknown dtype code %d", dtype);
  if (!norm_dtype_ok(param_dtype)) return set_error(CTI_EBAG_EINVAL, "unknown parameter dtype code %d", param_dtype);
  if (!(eps >= 0.f)) return set_error(CTI_EBAG_EINVAL, "eps must be >= 0");
  if (rows == 0) return CTI_EBAG_OK;
  if (rows > INT32_MAX) return set_error(CTI_EBAG_EUNSUPPORTED, "more than 2^31 - 1 rows (%lld)", (long long)rows);
  if (!x) return set_error(CTI_EBAG_EINVAL, "x is NULL");
  if (!y && !(mean_out && rstd_out))
    return set_error(CTI_EBAG_EINVAL, "y is NULL: a statistics-only call needs both mean_out and rstd_out");
  if (y && (!gamma || !beta)) return set_error(CTI_EBAG_EINVAL, "NULL device pointer among gamma/beta");
  NormParams p;
  p.x = static_cast<const char*>(x);
  p.y = static_cast<char*>(y);
  p.gamma = gamma;
  p.beta = beta;
  p.mean_out = mean_out;
  p.rstd_out = rstd_out;
  p.rows = rows;
  p.cols = cols;
  p.eps = eps;
  p.stream_out = rows * cols * dtype_bytes(dtype) >= kStreamOutBytes;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  switch (dtype) {
    case CTI_EBAG_F32: e = launch_norm_typed<float>(param_dtype, p, s); break;
    case CTI_EBAG_BF16: e = launch_norm_typed<bf16_t>(param_dtype, p, s); break;
    default: e = launch_norm_typed<f16_t>(param_dtype, p, s); break;
  }
  if (e != hipSuccess) return set_error(CTI_EBAG_EHIP, "layernorm launch failed: %s", hipGetErrorString(e));
  return CTI_EBAG_OK;
}
