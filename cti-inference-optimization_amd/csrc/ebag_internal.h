// Host-side internals shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cti_ebag.h"

namespace cti {

// Record `msg` (printf-style) as this thread's last error and return `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Map the status of the most recent launch to a CTI status code.
int check_launch(const char* what);

// Bags per tile of a launch whose rows are `emb_dim` elements of `table_dtype` (aligned
// buffers), or 0 when such rows take the element-wise kernel, which follows no tile order.
int order_bags_per_tile(int32_t table_dtype, int32_t emb_dim);

// Dispatch-order buffer layout shared by the device pass and the host builder:
// [0] tiles of the launch, [1] kOrderMagic, [2..3] zero, [kOrderHeader + position] = tile; each
// XCD's contiguous range of positions is sorted in chunks of kOrderChunk tiles into kOrderBuckets
// buckets of rows per bag (63 or more first).
constexpr int32_t kOrderMagic = 0x4f524452;
constexpr int kOrderHeader = 4;
constexpr int kOrderChunk = 2048;
constexpr int kOrderBuckets = 64;
constexpr int kOrderMaxFields = 64;

inline int dtype_bytes(int32_t dt) {
  switch (dt) {
    case CTI_EBAG_F32: return 4;
    case CTI_EBAG_BF16: return 2;
    case CTI_EBAG_F16: return 2;
    case CTI_EBAG_I8: return 1;
    default: return 0;
  }
}

}  // namespace cti
