// Per-token FP8 e4m3 quantization (drop-in for the reference's
// sgl_per_token_quant_fp8) and the fused RMSNorm -> FP8 epilogue.
//
// Kernel shape: a row is split into 16-byte chunks; LPR lanes share a row and
// each lane keeps its CH chunks in registers, so HBM is read exactly once and
// written exactly once. The row maximum is reduced with DPP / swizzle /
// readlane (and LDS only when a row spans several waves).
#include "jo_device.hpp"
#include "jo_host.hpp"

namespace jo {
namespace {

// ---------------------------------------------------------------------------
// Per-token quantization: follows per_token_quant_fp8.cu:56-82.
//   amax = max |x| (NaN ignored: fmaxf), scale = amax / 448 (IEEE division),
//   inv = (scale == 0) ? 0 : 1 / scale, q = e4m3fn(clamp(x * inv, +-448)).
// The row maximum is first taken NaN-propagating; when it is finite (no NaN,
// no inf in the row) it is the reference's amax and, with a finite inv, the
// clamp cannot change a code, so it is skipped. Any wave (workgroup, for
// rows wider than a wave) holding a non-finite row recomputes the
// NaN-skipping maximum and clamps that row.
// ---------------------------------------------------------------------------
template <class Tag, int LPR, int CH>
__global__ __launch_bounds__(kBlock) void quant_rows_kernel(const void* __restrict__ x, int64_t xs,
                                                            uint8_t* __restrict__ q, int64_t qs,
                                                            float* __restrict__ s, int64_t M, int N) {
  static_assert(Tag::kVec == 8, "fp8 rows are built from 8-element chunks");
  constexpr int RPB = kBlock / LPR;
  __shared__ float red[kBlock / kWave];
  __shared__ float red2[kBlock / kWave];
  const int lane = threadIdx.x % LPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / LPR;
  const bool row_ok = row < M;
  const void* xr = byte_off(x, row * xs * Tag::kBytes);

  u32x4 c[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int e = (i * LPR + lane) * 8;
    c[i] = (row_ok && e < N) ? ld16_nt(byte_off(xr, static_cast<int64_t>(e) * Tag::kBytes))
                             : u32x4{0u, 0u, 0u, 0u};
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = nan_max_abs(amax, elem<Tag>(c[i], j));
  }
  amax = row_reduce<LPR, OpAmax>(amax, red);
  const bool finite_row = finite_bits(amax);
  if (rows_any<LPR>(!finite_row)) {
    // Reference amax: NaNs skipped (fmaxf from 0).
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
#pragma unroll
      for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(elem<Tag>(c[i], j)));
    }
    amax = row_reduce<LPR, OpAmax>(m, red2);
  }
  const float scale = amax / kFp8Max;
  if (row_ok && lane == 0) s[row] = scale;
  const float inv = (scale == 0.f) ? 0.f : 1.0f / scale;
  const bool fast = finite_row && finite_bits(inv);

  uint8_t* qr = q + row * qs;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int e = (i * LPR + lane) * 8;
    if (row_ok && e < N) {
      float v[8];
      unpack<Tag>(c[i], v);
      st8_nt(qr + e, fast ? quant8<false>(v, inv) : quant8<true>(v, inv));
    }
  }
}

// One row per workgroup, element-wise accesses: any hidden size and any
// alignment (rows whose size is not a multiple of 8, or unaligned views).
template <class Tag>
__global__ __launch_bounds__(kBlock) void quant_generic_kernel(const void* __restrict__ x,
                                                               int64_t xs, uint8_t* __restrict__ q,
                                                               int64_t qs, float* __restrict__ s,
                                                               int N) {
  __shared__ float red[kBlock / kWave];
  const int64_t row = blockIdx.x;
  const int64_t xo = row * xs;
  float amax = 0.f;
  for (int i = threadIdx.x; i < N; i += kBlock) amax = fmaxf(amax, fabsf(load_elem<Tag>(x, xo + i)));
  amax = block_reduce<OpAmax>(amax, red);
  const float scale = amax / kFp8Max;
  if (threadIdx.x == 0) s[row] = scale;
  const float inv = (scale == 0.f) ? 0.f : 1.0f / scale;
  uint8_t* qr = q + row * qs;
  for (int i = threadIdx.x; i < N; i += kBlock) qr[i] = fp8_byte(load_elem<Tag>(x, xo + i) * inv);
}

template <class Tag>
int launch_quant(const void* x, int64_t M, int64_t N, int64_t xs, void* q, int64_t qs, float* s,
                 hipStream_t stream) {
  const bool vec_ok = (N % 8 == 0) && aligned(x, 16) && ((xs * Tag::kBytes) % 16 == 0) &&
                      aligned(q, 8) && (qs % 8 == 0);
  bool launched = false;
  if (vec_ok) {
    launched = dispatch_row_shape<8, false, 128>(N, [&](auto lpr, auto ch) {
      constexpr int LPR = decltype(lpr)::value;
      constexpr int CH = decltype(ch)::value;
      hipLaunchKernelGGL((quant_rows_kernel<Tag, LPR, CH>), dim3(row_blocks(M, LPR)), dim3(kBlock),
                         0, stream, x, xs, static_cast<uint8_t*>(q), qs, s, M,
                         static_cast<int>(N));
    }, M);
  }
  if (!launched) {
    hipLaunchKernelGGL((quant_generic_kernel<Tag>), dim3(M), dim3(kBlock), 0, stream, x, xs,
                       static_cast<uint8_t*>(q), qs, s, static_cast<int>(N));
  }
  return launch_status("sgl_per_token_quant_fp8");
}

// ---------------------------------------------------------------------------
// RMSNorm -> FP8. v = (x * r) * w in fp32 (rmsnorm.cu:41-60 without the
// rounding to the input type), r = 1/sqrt(mean(x^2) + eps) with the mean
// square rounded once from its exact value and IEEE sqrt and division; then
// the per_token_quant_fp8.cu:56-82 rule over the row (GROUP == 0) or over
// each 1x128 block (GROUP == 128, 16 lanes x 8 values).
// ---------------------------------------------------------------------------
template <class Tag, int LPR, int CH, int GROUP, bool WAVE_VOTE = false>
__global__ __launch_bounds__(kBlock) void rmsnorm_quant_kernel(
    const void* __restrict__ x, int64_t xs, const void* __restrict__ w, uint8_t* __restrict__ q,
    int64_t qs, float* __restrict__ s, int64_t M, int N, float eps) {
  static_assert(Tag::kVec == 8, "fp8 rows are built from 8-element chunks");
  static_assert(GROUP == 0 || (GROUP == 128 && LPR >= 16), "group layout");
  constexpr int RPB = kBlock / LPR;
  __shared__ double red_ss[kBlock / kWave];
  __shared__ float red_max[kBlock / kWave];
  __shared__ float red_max2[kBlock / kWave];
  const int lane = threadIdx.x % LPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / LPR;
  const bool row_ok = row < M;
  const void* xr = byte_off(x, row * xs * Tag::kBytes);

  u32x4 c[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int e = (i * LPR + lane) * 8;
    c[i] = (row_ok && e < N) ? ld16_nt(byte_off(xr, static_cast<int64_t>(e) * Tag::kBytes))
                             : u32x4{0u, 0u, 0u, 0u};
  }
  // Weight chunks are issued with the row loads so their (cached) latency
  // overlaps the HBM latency instead of following the row reduction.
  u32x4 wc[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int e = (i * LPR + lane) * 8;
    wc[i] = (e < N) ? ld16(byte_off(w, static_cast<int64_t>(e) * Tag::kBytes))
                    : u32x4{0u, 0u, 0u, 0u};
  }
  // The squares of bf16/fp16 values are exact in fp32; summing them in fp64
  // makes the mean square the correctly rounded fp32 value of the exact
  // mean, independent of the summation order. r then follows with two IEEE
  // fp32 operations, so r, v and the scales do not depend on the launch shape.
  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const double v = static_cast<double>(elem<Tag>(c[i], j));
      ss = __builtin_fma(v, v, ss);  // v*v is exact: one rounding per step, as a sum of squares
    }
  }
  ss = row_reduce_sum64<LPR>(ss, red_ss);
  const float ms = static_cast<float>(ss / static_cast<double>(N));
  const float r = 1.0f / sqrtf(ms + eps);

  // v = (x * r) * w, kept in registers for the quantization pass. The
  // per-chunk maxima are NaN-propagating (see quant_rows_kernel): a finite
  // maximum is the reference's and lets the clamp be skipped.
  float v[CH][8];
  float gmax[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    gmax[i] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v[i][j] = (elem<Tag>(c[i], j) * r) * elem<Tag>(wc[i], j);
      gmax[i] = nan_max_abs(gmax[i], v[i][j]);
    }
  }
  // NaN-skipping maximum of chunk i's part of this lane (the reference's
  // fmaxf rule), for workgroups that hold a non-finite value. The decision
  // is workgroup-wide except with WAVE_VOTE (per token, at least as many
  // rows as the GPU has wave slots): a wave-level vote measured faster only
  // there (T = 10530 per token 20.1 -> 19.5 us) and slower in the other three
  // C4 cases (T = 4725: 10.0 -> 10.3 / 10.4 -> 10.9 us; per block at 10530:
  // 20.4 -> 20.6 us).
  auto skip_nan_max = [&](int i) {
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(v[i][j]));
    return m;
  };
  if constexpr (GROUP == 128) {
    // Each 16-lane DPP row of a chunk holds one 1x128 block.
    bool all_finite = true;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      gmax[i] = allreduce_amax<16>(gmax[i]);
      all_finite = all_finite && finite_bits(gmax[i]);
    }
    bool fast[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) fast[i] = finite_bits(gmax[i]);
    if (__syncthreads_or(!all_finite)) {
#pragma unroll
      for (int i = 0; i < CH; ++i) gmax[i] = allreduce_amax<16>(skip_nan_max(i));
    }
    float ginv[CH];
    if constexpr (LPR >= kWave) {
      // A wave holds 4*CH blocks: gather their maxima into lanes 0..4*CH-1
      // so the two IEEE divisions run once per block, then hand each chunk
      // its inverse scale back.
      const int wl = threadIdx.x % kWave;
      const int wave_in_row = lane / kWave;
      float mine = 0.f;
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        const float t = __builtin_bit_cast(
            float, __builtin_amdgcn_ds_bpermute((wl & 3) * 16 * 4, __builtin_bit_cast(int, gmax[i])));
        if ((wl >> 2) == i) mine = t;
      }
      const float gs = mine / kFp8Max;
      const float gi = (gs == 0.f) ? 0.f : 1.0f / gs;
      const int gc = wl >> 2;  // chunk of the block this lane owns
      const int ge = (gc * LPR + wave_in_row * kWave + (wl & 3) * 16) * 8;  // its first element
      if (row_ok && wl < 4 * CH && ge < N) s[row * (N / 128) + ge / 128] = gs;
#pragma unroll
      for (int i = 0; i < CH; ++i)
        ginv[i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(
                                                (i * 4 + (wl >> 4)) * 4, __builtin_bit_cast(int, gi)));
    } else {
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        const int e = (i * LPR + lane) * 8;
        const float gs = gmax[i] / kFp8Max;
        ginv[i] = (gs == 0.f) ? 0.f : 1.0f / gs;
        if (row_ok && e < N && (lane & 15) == 0) s[row * (N / 128) + e / 128] = gs;
      }
    }
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int e = (i * LPR + lane) * 8;
      if (row_ok && e < N)
        st8_nt(q + row * qs + e, (fast[i] && finite_bits(ginv[i])) ? quant8<false>(v[i], ginv[i])
                                                                   : quant8<true>(v[i], ginv[i]));
    }
  }
  if constexpr (GROUP == 0) {
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < CH; ++i) amax = __builtin_elementwise_maximum(amax, gmax[i]);
    amax = row_reduce<LPR, OpAmax>(amax, red_max);
    const bool finite_row = finite_bits(amax);
    const bool any_nonfinite =
        WAVE_VOTE ? rows_any<LPR>(!finite_row) : __syncthreads_or(!finite_row);
    if (any_nonfinite) {
      float m = 0.f;
#pragma unroll
      for (int i = 0; i < CH; ++i) m = fmaxf(m, skip_nan_max(i));
      amax = row_reduce<LPR, OpAmax>(m, red_max2);
    }
    const float scale = amax / kFp8Max;
    if (row_ok && lane == 0) s[row] = scale;
    const float inv = (scale == 0.f) ? 0.f : 1.0f / scale;
    const bool fast = finite_row && finite_bits(inv);
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int e = (i * LPR + lane) * 8;
      if (row_ok && e < N)
        st8_nt(q + row * qs + e, fast ? quant8<false>(v[i], inv) : quant8<true>(v[i], inv));
    }
  }
}

template <class Tag>
int launch_rmsnorm_quant(const void* x, int64_t xs, const void* w, void* q, int64_t qs, float* s,
                         int64_t M, int64_t N, float eps, int64_t group, hipStream_t stream) {
  bool launched = false;
  if (group == 0) {
    launched = dispatch_row_shape<8>(N, [&](auto lpr, auto ch) {
      constexpr int LPR = decltype(lpr)::value;
      constexpr int CH = decltype(ch)::value;
      if (M >= kFewRows)
        hipLaunchKernelGGL((rmsnorm_quant_kernel<Tag, LPR, CH, 0, true>), dim3(row_blocks(M, LPR)),
                           dim3(kBlock), 0, stream, x, xs, w, static_cast<uint8_t*>(q), qs, s, M,
                           static_cast<int>(N), eps);
      else
        hipLaunchKernelGGL((rmsnorm_quant_kernel<Tag, LPR, CH, 0>), dim3(row_blocks(M, LPR)),
                           dim3(kBlock), 0, stream, x, xs, w, static_cast<uint8_t*>(q), qs, s, M,
                           static_cast<int>(N), eps);
    });
  } else {
    launched = dispatch_row_shape<8>(N, [&](auto lpr, auto ch) {
      constexpr int LPR = decltype(lpr)::value < 16 ? 16 : decltype(lpr)::value;
      constexpr int CH = decltype(ch)::value;
      hipLaunchKernelGGL((rmsnorm_quant_kernel<Tag, LPR, CH, 128>), dim3(row_blocks(M, LPR)),
                         dim3(kBlock), 0, stream, x, xs, w, static_cast<uint8_t*>(q), qs, s, M,
                         static_cast<int>(N), eps);
    });
  }
  if (!launched) {
    set_error("rmsnorm_quant_fp8: hidden size %lld exceeds the largest row shape (32768)",
              static_cast<long long>(N));
    return JO_ERR_UNSUPPORTED;
  }
  return launch_status("rmsnorm_quant_fp8");
}

}  // namespace
}  // namespace jo

using namespace jo;

extern "C" int jo_sgl_per_token_quant_fp8(const void* input, int dtype, int64_t num_tokens,
                                          int64_t hidden_dim, int64_t in_stride, void* output_q,
                                          int64_t q_stride, float* output_s, void* stream) {
  // Checks of per_token_quant_fp8.cu:149-156 and :168-175, plus the output
  // checks the reference leaves out.
  JO_REQUIRE(dtype == JO_DTYPE_BF16 || dtype == JO_DTYPE_F16,
             "per_token_quant_fp8: input must be bf16 or fp16");
  JO_REQUIRE(num_tokens >= 0 && hidden_dim >= 0, "per_token_quant_fp8: negative size");
  JO_REQUIRE(hidden_dim % 4 == 0, "hidden_dim must be divisible by 4, got %lld",
             static_cast<long long>(hidden_dim));
  JO_REQUIRE(hidden_dim <= INT32_MAX, "per_token_quant_fp8: hidden_dim too large");
  JO_REQUIRE(in_stride >= hidden_dim && q_stride >= hidden_dim,
             "per_token_quant_fp8: row stride smaller than hidden_dim");
  if (num_tokens == 0) return JO_OK;
  JO_REQUIRE(input && output_q && output_s, "per_token_quant_fp8: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == JO_DTYPE_BF16)
    return launch_quant<BF16>(input, num_tokens, hidden_dim, in_stride, output_q, q_stride,
                              output_s, st);
  return launch_quant<F16>(input, num_tokens, hidden_dim, in_stride, output_q, q_stride, output_s,
                           st);
}

extern "C" int jo_rmsnorm_quant_fp8(const void* x, int64_t x_stride, const void* weight,
                                    void* out_q, int64_t q_stride, float* out_s, int64_t M,
                                    int64_t N, int dtype, float eps, int64_t group_size,
                                    void* stream) {
  JO_REQUIRE(dtype == JO_DTYPE_BF16 || dtype == JO_DTYPE_F16,
             "rmsnorm_quant_fp8: x must be bf16 or fp16");
  JO_REQUIRE(group_size == 0 || group_size == 128,
             "rmsnorm_quant_fp8: group_size must be 0 (per token) or 128, got %lld",
             static_cast<long long>(group_size));
  JO_REQUIRE(M >= 0 && N > 0, "rmsnorm_quant_fp8: bad shape [%lld, %lld]",
             static_cast<long long>(M), static_cast<long long>(N));
  JO_REQUIRE(N % 8 == 0, "rmsnorm_quant_fp8: N must be divisible by 8, got %lld",
             static_cast<long long>(N));
  JO_REQUIRE(group_size == 0 || N % 128 == 0,
             "rmsnorm_quant_fp8: N must be divisible by 128 for 1x128 blocks, got %lld",
             static_cast<long long>(N));
  JO_REQUIRE(x_stride >= N && q_stride >= N, "rmsnorm_quant_fp8: row stride smaller than N");
  if (M == 0) return JO_OK;
  JO_REQUIRE(x && weight && out_q && out_s, "rmsnorm_quant_fp8: null pointer");
  JO_REQUIRE(aligned(x, 16) && (x_stride * 2) % 16 == 0 && aligned(weight, 16),
             "rmsnorm_quant_fp8: x rows and weight must be 16-byte aligned");
  JO_REQUIRE(aligned(out_q, 8) && q_stride % 8 == 0,
             "rmsnorm_quant_fp8: output rows must be 8-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == JO_DTYPE_BF16)
    return launch_rmsnorm_quant<BF16>(x, x_stride, weight, out_q, q_stride, out_s, M, N, eps,
                                      group_size, st);
  return launch_rmsnorm_quant<F16>(x, x_stride, weight, out_q, q_stride, out_s, M, N, eps,
                                   group_size, st);
}
