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
