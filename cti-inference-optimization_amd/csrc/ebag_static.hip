// Allocation-free form of the general pooling entry point (cti_ebag_forward_static).
//
// cti_ebag_forward takes its length-binning workspace from the caller, who must allocate it.
// Callers that cannot allocate device memory (HIP graph capture, tight serving loops, hosts that
// forbid it) use this entry instead: the workspace is `scratch` below, a static device array
// that the loader places once in each GPU's copy of the code object, where it stays until the
// process ends. Host code never passes the array's name as an address (on the host it names a
// stand-in): each device's address comes from hipGetSymbolAddress, taken once per device with
// that device current, and only that address reaches the kernels.
//
// Every call on one GPU shares that GPU's copy, which keeps the last call's lists; the two list
// counters are zeroed (by a fill kernel on the caller's stream) when a device's address is first
// looked up, and every call leaves them zero again. Calls that overlap in time on one GPU race.
#include <mutex>

#include "ebag_device.h"
#include "ebag_internal.h"

namespace cti {
namespace {

static __device__ __align__(256) unsigned char scratch[CTI_EBAG_STATIC_WORKSPACE_BYTES];

constexpr int kMaxDevices = 64;
constexpr int kCounterWords = 4;  // the workspace header's list counters: count, total, count2, total2

__global__ void zero_counters_kernel(unsigned int* p) {
  if (static_cast<int>(threadIdx.x) < kCounterWords) p[threadIdx.x] = 0u;
}

std::mutex g_mutex;
void* g_scratch[kMaxDevices];  // per-device address of `scratch`, NULL until looked up

// The current device's copy of `scratch`.
int device_scratch(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(CTI_EBAG_EHIP, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(CTI_EBAG_EUNSUPPORTED, "device %d: the static workspace serves devices 0..%d", dev, kMaxDevices - 1);
  std::lock_guard<std::mutex> lock(g_mutex);
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return set_error(CTI_EBAG_EHIP, "hipGetSymbolAddress(scratch) on device %d failed: %s", dev, hipGetErrorString(e));
    hipLaunchKernelGGL(zero_counters_kernel, dim3(1), dim3(kWave), 0, stream, static_cast<unsigned int*>(ptr));
    e = hipGetLastError();
    if (e != hipSuccess) return set_error(CTI_EBAG_EHIP, "zeroing the static workspace failed: %s", hipGetErrorString(e));
    g_scratch[dev] = ptr;
  }
  *out = g_scratch[dev];
  return CTI_EBAG_OK;
}

}  // namespace
}  // namespace cti

using namespace cti;

extern "C" int cti_ebag_forward_static(const void* values, int32_t index_type, int64_t nnz, const int64_t* offsets,
                                       int64_t batch_size, int32_t num_fields, const cti_ebag_table* tables,
                                       int32_t table_dtype, int32_t pooling, void* out, int32_t out_dtype,
                                       int64_t out_row_stride, const cti_ebag_options* opts, void* stream) {
  clear_error();
  if (opts && opts->use_bins && batch_size > 0 && num_fields > 0) {
    const int64_t need = cti_ebag_workspace_bytes(batch_size, num_fields);
    if (need > CTI_EBAG_STATIC_WORKSPACE_BYTES)
      return set_error(CTI_EBAG_EWORKSPACE,
                       "length binning of %lld samples x %d fields needs %lld bytes of workspace; the allocation-free "
                       "entry holds %lld (batch_size * min(num_fields, 64) <= %lld)",
                       (long long)batch_size, num_fields, (long long)need, (long long)CTI_EBAG_STATIC_WORKSPACE_BYTES,
                       (long long)((CTI_EBAG_STATIC_WORKSPACE_BYTES - 256) / 24));
  }
  // the arguments are checked by cti_ebag_forward; an empty job launches nothing
  if (batch_size <= 0 || num_fields <= 0)
    return cti_ebag_forward(values, index_type, nnz, offsets, batch_size, num_fields, tables, table_dtype, pooling,
                            out, out_dtype, out_row_stride, nullptr, 0, opts, stream);
  void* ws = nullptr;
  const int rc = device_scratch(static_cast<hipStream_t>(stream), &ws);
  if (rc != CTI_EBAG_OK) return rc;
  return cti_ebag_forward(values, index_type, nnz, offsets, batch_size, num_fields, tables, table_dtype, pooling, out,
                          out_dtype, out_row_stride, ws, CTI_EBAG_STATIC_WORKSPACE_BYTES, opts, stream);
}
