// Status and error-message plumbing for the libcdx C-ABI.
#include <stdarg.h>
#include <stdio.h>

#include "cdx_common.h"

namespace cdx {

static thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

void clear_error() { g_last_error.clear(); }

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(CDX_ELAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(err));
  }
  return CDX_OK;
}

}  // namespace cdx

extern "C" int cdx_version(void) { return 100; }

extern "C" const char* cdx_last_error(void) { return cdx::g_last_error.c_str(); }
