// Error reporting, version and launch-override entry points of the C ABI.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <atomic>

#include "jo_host.hpp"

namespace jo {
namespace {
thread_local char g_last_error[512] = {0};

constexpr int kKnobs = 3;

// Each knob's environment variable is read once, when the library is loaded.
int knob_from_env(const char* name) {
  const char* v = getenv(name);
  return (v && *v) ? atoi(v) : -1;
}
std::atomic<int> g_knobs[kKnobs] = {{knob_from_env("JO_QK_SPLIT")},
                                    {knob_from_env("JO_KV_SPLIT")},
                                    {knob_from_env("JO_GEMM_SHAPE")}};
}  // namespace

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

int launch_knob(int knob) {
  return (knob >= 0 && knob < kKnobs) ? g_knobs[knob].load(std::memory_order_relaxed) : -1;
}

}  // namespace jo

extern "C" const char* jo_last_error(void) { return jo::g_last_error; }

extern "C" int jo_abi_version(void) { return JO_ABI_VERSION; }

extern "C" int jo_set_launch_override(int knob, int value) {
  JO_REQUIRE(knob >= 0 && knob < jo::kKnobs, "jo_set_launch_override: unknown knob %d", knob);
  JO_REQUIRE(value >= -1 && value <= 64, "jo_set_launch_override: value %d out of range", value);
  jo::g_knobs[knob].store(value, std::memory_order_relaxed);
  return JO_OK;
}
