// Host-side helpers for the C ABI: per-thread error messages, argument
// validation and the row-shape dispatch shared by every row kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "joyomni_hip.h"

namespace jo {

// Records a printf-style message as the calling thread's last error.
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// Converts the launch status of the kernel just enqueued into a JO_ status.
int launch_status(const char* op);

// Launch-shape override of a JO_KNOB_* knob: -1 (automatic choice) unless the
// environment set it when the library was loaded (JO_QK_SPLIT, JO_KV_SPLIT,
// JO_GEMM_SHAPE) or jo_set_launch_override() changed it since. Results never
// depend on a knob, only the launch shape does.
int launch_knob(int knob);

#define JO_REQUIRE(cond, ...)      \
  do {                             \
    if (!(cond)) {                 \
      ::jo::set_error(__VA_ARGS__); \
      return JO_ERR_INVALID;       \
    }                              \
  } while (0)

inline bool aligned(const void* p, int64_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) % static_cast<uintptr_t>(bytes)) == 0;
}

// Most rows a row-kernel launch takes: at one 256-thread workgroup per row
// (the generic kernels, and rows wider than a wave) the launch's work-item
// count must stay below 2^32.
constexpr int64_t kMaxRows = int64_t{UINT32_MAX} / 256;

// Number of row-kernel workgroups needed for M rows at LPR lanes per row.
inline int64_t row_blocks(int64_t M, int lpr) {
  const int64_t rows_per_block = 256 / lpr;
  return (M + rows_per_block - 1) / rows_per_block;
}

// Row shapes. A row of N elements is split into 16-byte chunks of kVec
// elements; LPR lanes share a row and each lane holds CH chunks. The
// dispatcher picks the smallest shape that covers N and calls
// fn(std::integral_constant<int, LPR>, std::integral_constant<int, CH>).
// Returns false when N exceeds the largest shape (the caller then uses its
// generic kernel). WIDE adds a 128-lane shape for 257..384 chunks (two waves
// per row, three chunks per lane), which the residual + LayerNorm kernel
// prefers at hidden 3072 (10530 rows: 47.5 -> 45.8 us on MI355X).
// FEW (128 or 256) spreads rows of 385..512 chunks over FEW lanes when there
// are fewer rows M than the GPU has wave slots (kFewRows): one wave per row
// would leave one partly filled round of waves whose reads all go out before
// any write. Measured at [3120, 4096]: LayerNorm + modulation 20.0 -> 18.3 us
// with four waves per row (two: 18.4-19.3), per-token quant 8.5 -> 8.1 us
// with two (four: 8.8).
constexpr int64_t kFewRows = 8192;  // 256 CUs x 4 SIMDs x 8 waves

template <int V, bool WIDE = false, int FEW = 0, class Fn>
bool dispatch_row_shape(int64_t N, Fn&& fn, int64_t M = kFewRows) {
  using std::integral_constant;
  const int64_t chunks = (N + V - 1) / V;
  if (chunks <= 8) { fn(integral_constant<int, 8>{}, integral_constant<int, 1>{}); return true; }
  if (chunks <= 16) { fn(integral_constant<int, 16>{}, integral_constant<int, 1>{}); return true; }
  if (chunks <= 32) { fn(integral_constant<int, 32>{}, integral_constant<int, 1>{}); return true; }
  if (chunks <= 64 * 1) { fn(integral_constant<int, 64>{}, integral_constant<int, 1>{}); return true; }
  if (chunks <= 64 * 2) { fn(integral_constant<int, 64>{}, integral_constant<int, 2>{}); return true; }
  if (chunks <= 64 * 3) { fn(integral_constant<int, 64>{}, integral_constant<int, 3>{}); return true; }
  if (chunks <= 64 * 4) { fn(integral_constant<int, 64>{}, integral_constant<int, 4>{}); return true; }
  if constexpr (WIDE)
    if (chunks <= 128 * 3) { fn(integral_constant<int, 128>{}, integral_constant<int, 3>{}); return true; }
  if (chunks <= 64 * 6) { fn(integral_constant<int, 64>{}, integral_constant<int, 6>{}); return true; }
  static_assert(FEW == 0 || FEW == 128 || FEW == 256, "lanes per row for few rows");
  if constexpr (FEW != 0)
    if (M < kFewRows && chunks <= 64 * 8) {
      fn(integral_constant<int, FEW>{}, integral_constant<int, 64 * 8 / FEW>{});
      return true;
    }
  if (chunks <= 64 * 8) { fn(integral_constant<int, 64>{}, integral_constant<int, 8>{}); return true; }
  if (chunks <= 64 * 12) { fn(integral_constant<int, 64>{}, integral_constant<int, 12>{}); return true; }
  if (chunks <= 64 * 16) { fn(integral_constant<int, 64>{}, integral_constant<int, 16>{}); return true; }
  if (chunks <= 256 * 8) { fn(integral_constant<int, 256>{}, integral_constant<int, 8>{}); return true; }
  if (chunks <= 256 * 12) { fn(integral_constant<int, 256>{}, integral_constant<int, 12>{}); return true; }
  if (chunks <= 256 * 16) { fn(integral_constant<int, 256>{}, integral_constant<int, 16>{}); return true; }
  return false;
}

inline int dtype_bytes(int dtype) { return dtype == JO_DTYPE_F32 ? 4 : 2; }

inline bool valid_dtype(int dtype) {
  return dtype == JO_DTYPE_F32 || dtype == JO_DTYPE_F16 || dtype == JO_DTYPE_BF16;
}

}  // namespace jo
