// Error reporting, version and launch-override entry points of the C ABI.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <atomic>

#include "jo_host.hpp"

namespace jo {
namespace {
thread_local char g_last_error[512] = {0};

constexpr int kKnobs = 4;

// The values each knob accepts besides -1 (the library's own choice):
// QK waves per token 1, 2, 4, 6, 8; KV rows on 1 or 2 waves; GEMM shapes 0-9;
// GEMM K splits 1, 2, 4, 8.
bool knob_value_ok(int knob, int v) {
  if (v == -1) return true;
  switch (knob) {
    case JO_KNOB_QK_SPLIT: return v == 1 || v == 2 || v == 4 || v == 6 || v == 8;
    case JO_KNOB_KV_SPLIT: return v == 1 || v == 2;
    case JO_KNOB_GEMM_SHAPE: return v >= 0 && v <= 11;
    case JO_KNOB_GEMM_SPLIT: return v == 1 || v == 2 || v == 4 || v == 8;
    default: return false;
  }
}

// Each knob's environment variable is read once, when the library is loaded.
// A value the knob does not accept is ignored (with a message on stderr), so a
// mistyped override never silently selects another kernel.
int knob_from_env(int knob, const char* name) {
  const char* v = getenv(name);
  if (!v || !*v) return -1;
  char* end = nullptr;
  const long x = strtol(v, &end, 10);
  if (*end != 0 || x < -1 || x > 64 || !knob_value_ok(knob, static_cast<int>(x))) {
    fprintf(stderr, "joyomni_hip: ignoring %s=%s (not a value this knob accepts)\n", name, v);
    return -1;
  }
  return static_cast<int>(x);
}
std::atomic<int> g_knobs[kKnobs] = {{knob_from_env(JO_KNOB_QK_SPLIT, "JO_QK_SPLIT")},
                                    {knob_from_env(JO_KNOB_KV_SPLIT, "JO_KV_SPLIT")},
                                    {knob_from_env(JO_KNOB_GEMM_SHAPE, "JO_GEMM_SHAPE")},
                                    {knob_from_env(JO_KNOB_GEMM_SPLIT, "JO_GEMM_SPLIT")}};
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
  JO_REQUIRE(jo::knob_value_ok(knob, value),
             "jo_set_launch_override: value %d is not one knob %d accepts", value, knob);
  jo::g_knobs[knob].store(value, std::memory_order_relaxed);
  return JO_OK;
}
