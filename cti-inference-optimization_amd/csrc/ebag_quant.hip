// Row quantisation of an embedding table to int8 for MI355X (gfx950), as the reference's
// quantize_embedding_int8 (online_best/infer.py:895-901) evaluates on the device:
//   m = max_j |w[r, j]|                 (fp32; exact in any order)
//   s = max(m * RN32(1/127), 1e-8)      (torch divides a device tensor by a Python scalar as a
//                                        multiply by the scalar's fp32 reciprocal; then
//                                        torch.clamp(scale, min=1e-8))
//   q[r, j] = clamp(rint(w[r, j] / s), -128, 127)   (IEEE fp32 division, round half to even)
// One wavefront per row; results are bit-identical to that expression for finite tables.
#include <stdint.h>

#include "ebag_device.h"
#include "ebag_internal.h"

namespace cti {
namespace {

constexpr int kQuantThreads = 256;
constexpr int kQuantRowsPerBlock = kQuantThreads / kWave;

template <typename T>
__global__ void __launch_bounds__(kQuantThreads) quantize_rows_kernel(const char* w, int64_t rows, int64_t dim,
                                                                       int64_t row_stride, int8_t* q, float* scale) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kQuantRowsPerBlock + threadIdx.x / kWave;
  if (row >= rows) return;  // uniform over the wavefront
  const int lane = lane_id();
  const char* wr = w + row * row_stride * Elem<T>::kBytes;
  float m = 0.f;
  for (int64_t c = lane; c < dim; c += kWave) m = fmaxf(m, fabsf(Elem<T>::load(wr + c * Elem<T>::kBytes)));
#pragma unroll
  for (int k = 1; k < kWave; k <<= 1) m = fmaxf(m, shfl_xor_f32(m, k));
  float s = m * (1.0f / 127.0f);
  s = s < 1e-8f ? 1e-8f : s;
  if (lane == 0) scale[row] = s;
  int8_t* qr = q + row * dim;
  for (int64_t c = lane; c < dim; c += kWave) {
    float v = rintf(Elem<T>::load(wr + c * Elem<T>::kBytes) / s);
    v = v < -128.f ? -128.f : (v > 127.f ? 127.f : v);
    qr[c] = static_cast<int8_t>(v);
  }
}

}  // namespace
}  // namespace cti

using namespace cti;

extern "C" int cti_ebag_quantize_int8(const void* weight, int32_t dtype, int64_t rows, int64_t dim,
                                      int64_t row_stride, int8_t* q, float* scale, void* stream) {
  clear_error();
  if (dtype != CTI_EBAG_F32 && dtype != CTI_EBAG_BF16 && dtype != CTI_EBAG_F16)
    return set_error(CTI_EBAG_EINVAL, "unknown dtype code %d", dtype);
  if (rows < 0) return set_error(CTI_EBAG_EINVAL, "rows must be >= 0 (got %lld)", (long long)rows);
  if (dim < 1) return set_error(CTI_EBAG_EINVAL, "dim must be >= 1 (got %lld)", (long long)dim);
  if (row_stride < dim) return set_error(CTI_EBAG_EINVAL, "row_stride %lld < dim %lld", (long long)row_stride, (long long)dim);
  if (rows == 0) return CTI_EBAG_OK;
  if (!weight || !q || !scale) return set_error(CTI_EBAG_EINVAL, "NULL device pointer among weight/q/scale");
  const int64_t blocks = (rows + kQuantRowsPerBlock - 1) / kQuantRowsPerBlock;
  if (blocks > INT32_MAX) return set_error(CTI_EBAG_EUNSUPPORTED, "too many rows (%lld)", (long long)rows);
  const dim3 grid(static_cast<unsigned>(blocks)), block(kQuantThreads);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const char* w = static_cast<const char*>(weight);
  switch (dtype) {
    case CTI_EBAG_F32: hipLaunchKernelGGL((quantize_rows_kernel<float>), grid, block, 0, s, w, rows, dim, row_stride, q, scale); break;
    case CTI_EBAG_BF16: hipLaunchKernelGGL((quantize_rows_kernel<bf16_t>), grid, block, 0, s, w, rows, dim, row_stride, q, scale); break;
    default: hipLaunchKernelGGL((quantize_rows_kernel<f16_t>), grid, block, 0, s, w, rows, dim, row_stride, q, scale); break;
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(CTI_EBAG_EHIP, "quantize launch failed: %s", hipGetErrorString(e));
  return CTI_EBAG_OK;
}
