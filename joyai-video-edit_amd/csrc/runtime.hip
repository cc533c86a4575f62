// Error reporting and version entry points of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "jo_host.hpp"

namespace jo {
namespace {
thread_local char g_last_error[512] = {0};
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = 0; }

int launch_status(const char* op) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", op, hipGetErrorString(e));
    return JO_ERR_HIP;
  }
  return JO_OK;
}

}  // namespace jo

extern "C" const char* jo_last_error(void) { return jo::g_last_error; }

extern "C" int jo_abi_version(void) { return JO_ABI_VERSION; }
