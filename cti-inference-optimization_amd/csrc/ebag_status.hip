// Error reporting and version query of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "ebag_internal.h"

namespace cti {

namespace {
thread_local char g_last_error[512] = "";
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return set_error(CTI_EBAG_EHIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  }
  return CTI_EBAG_OK;
}

}  // namespace cti

extern "C" int cti_ebag_abi_version(void) { return CTI_EBAG_ABI_VERSION; }

extern "C" const char* cti_ebag_last_error(void) { return cti::g_last_error; }
