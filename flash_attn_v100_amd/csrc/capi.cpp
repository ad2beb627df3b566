// Error reporting and version entry points of the C ABI.
#include <stdio.h>

#include <string>

#include "capi_internal.h"

namespace fa {

static thread_local std::string g_last_error;

int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error.assign(buf);
  return code;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return set_error(FA_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(err));
  }
  return FA_OK;
}

}  // namespace fa

extern "C" const char* fa_last_error(void) { return fa::g_last_error.c_str(); }

extern "C" const char* fa_version(void) { return "0.1.0 gfx950"; }
