// C-ABI plumbing shared by every entry point: error recording and launch checks.
#include <stdarg.h>
#include <stdio.h>

#include <string>

#include "gdn_common.h"

namespace {
thread_local std::string g_last_error;
}

namespace zgdn {

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(ZGDN_EHIP, "%s: kernel launch failed: %s", what, hipGetErrorString(err));
  g_last_error.clear();
  return ZGDN_OK;
}

}  // namespace zgdn

extern "C" const char* zgdn_last_error(void) { return g_last_error.c_str(); }

extern "C" int zgdn_abi_version(void) { return 2; }
