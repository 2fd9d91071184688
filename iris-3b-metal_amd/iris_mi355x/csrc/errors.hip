// Thread-local error state of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "iris_common.hpp"

namespace {
thread_local char g_message[512] = "";
}

namespace iris {

int fail(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_message, sizeof(g_message), fmt, args);
  va_end(args);
  return code;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(IRIS_E_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(err));
  return IRIS_OK;
}

}  // namespace iris

extern "C" const char* iris_last_error(void) { return g_message; }

extern "C" int iris_abi_version(void) { return 3; }
