// Error state and small C-ABI entry points that launch nothing.
#include <cstdarg>
#include <cstdio>

#include "as_internal.h"

namespace as {

namespace {
thread_local char g_message[512] = {0};
}

int fail(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  std::vsnprintf(g_message, sizeof(g_message), fmt, args);
  va_end(args);
  return code;
}

void clear_error() { g_message[0] = '\0'; }

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(AS_ERR_LAUNCH, "%s: HIP launch failed: %s", what, hipGetErrorString(err));
  }
  return AS_OK;
}

}  // namespace as

extern "C" {

const char* as_last_error(void) { return as::g_message; }

int as_abi_version(void) { return AS_ABI_VERSION; }

}  // extern "C"
