// Host-side error reporting shared by every C-ABI entry point.

#include <stdarg.h>
#include <stdio.h>

#include "kvc_common.h"

namespace kvc {

namespace {
thread_local char g_last_error[512] = "";
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(static_cast<int>(e), "%s: launch failed: %s", what, hipGetErrorString(e));
  return 0;
}

}  // namespace kvc

extern "C" int kvc_abi_version(void) { return KVC_ABI_VERSION; }

extern "C" const char* kvc_last_error(void) { return kvc::g_last_error; }
