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

// GELU with the tanh approximation, the activation torch applies between the
// MLP's two Fp8Linears (dit.py:91-92, 433):
//   gelu(x) = 0.5 * x * (1 + tanh(u)),  u = sqrt(2/pi) * (x + 0.044715 * x^3),
// in fp32 with the rounding structure of that formula where it matters: tanh(u)
// is rounded to fp32 before 1 is added, so where 1 + tanh(u) cancels (x below
// about -3) the result moves in steps of 2^-24 * 0.5|x| as the formula's own
// evaluation does. u is formed as x (b + b k x^2) (one fma, 3 operations
// instead of 5), tanh(|u|) = 1 - 2 / (exp(2|u|) + 1) from the hardware exp2 and
// reciprocal (each within 1 ulp): exp overflows to inf for large |u|, giving
// tanh = +-1. gelu(+inf) = inf, gelu(-inf) = NaN (0 * inf), NaN propagates;
// the caller rounds the result to the row's dtype.
__device__ __forceinline__ float gelu_tanh(float x) {
#pragma clang fp contract(off)
  constexpr float kBeta = 0.7978845608028654f;         // sqrt(2 / pi)
  constexpr float kBetaKappa = 0.035677408136300125f;  // sqrt(2 / pi) * 0.044715
  constexpr float kTwoLog2e = 2.8853900817779268f;     // 2 / ln 2
  const float u = x * __builtin_fmaf(kBetaKappa, x * x, kBeta);
  const float t = __builtin_amdgcn_exp2f(fabsf(u) * kTwoLog2e);  // exp(2|u|)
  // 1 - tanh(|u|) = 2 / (t + 1) = 1 / (0.5 t + 0.5), the fma exact up to its one rounding
  const float r = __builtin_amdgcn_rcpf(__builtin_fmaf(t, 0.5f, 0.5f));
  const float th = copysignf(1.0f - r, u);                        // tanh(u)
  return x * __builtin_fmaf(0.5f, th, 0.5f);  // 0.5 x (1 + tanh(u)), 0.5 (1 + th) exact
}

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
// ACT: the row is first replaced by gelu_tanh of it, rounded to the row's
// dtype (the bf16 / fp16 tensor torch's activation would return), and that
// row is quantized; when act is not null it is also stored there (row
// stride as elements).
template <class Tag, int LPR, int CH, bool ACT = false>
__global__ __launch_bounds__(kBlock) void quant_rows_kernel(const void* __restrict__ x, int64_t xs,
                                                            uint8_t* __restrict__ q, int64_t qs,
                                                            float* __restrict__ s, int64_t M, int N,
                                                            void* __restrict__ act = nullptr,
                                                            int64_t as = 0) {
  static_assert(Tag::kVec == 8, "fp8 rows are built from 8-element chunks");
  constexpr int RPB = kBlock / LPR;
  __shared__ float red[kBlock / kWave];
  __shared__ float red2[kBlock / kWave];
  const int lane = threadIdx.x % LPR;
  // One-wave rows: whole lines of scales per XCD (see xcd_row_block).
  const int64_t blk = LPR == kWave ? xcd_row_block<RPB>(blockIdx.x, gridDim.x) : blockIdx.x;
  const int64_t row = blk * RPB + wave_uniform_row<LPR>();
  const bool row_ok = row < M;
  const void* xr = byte_off(x, row * xs * Tag::kBytes);

  u32x4 c[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int e = (i * LPR + lane) * 8;
    c[i] = (row_ok && e < N) ? ld16_nt(byte_off(xr, static_cast<int64_t>(e) * Tag::kBytes))
                             : u32x4{0u, 0u, 0u, 0u};
  }
  if constexpr (ACT) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      float v[8];
      unpack<Tag>(c[i], v);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = gelu_tanh(v[j]);
      c[i] = pack<Tag>(v);  // gelu(0) = 0 keeps the lanes past N at zero
    }
    if (act != nullptr && row_ok) {
      char* ar = static_cast<char*>(act) + row * as * Tag::kBytes;
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        const int e = (i * LPR + lane) * 8;
        if (e < N) st16_nt(ar + static_cast<int64_t>(e) * Tag::kBytes, c[i]);
      }
    }
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = nan_max_abs(amax, elem<Tag>(c[i], j));
  }
  bool any_nonfinite;
  amax = row_amax_vote<LPR>(amax, red, any_nonfinite);
  const bool finite_row = finite_bits(amax);
  if (any_nonfinite) {
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
template <class Tag, bool ACT>
__device__ __forceinline__ float generic_value(const void* x, int64_t i) {
  const float v = load_elem<Tag>(x, i);
  if constexpr (ACT)
    return round_to<Tag>(gelu_tanh(v));
  else
    return v;
}

template <class Tag, bool ACT = false>
__global__ __launch_bounds__(kBlock) void quant_generic_kernel(const void* __restrict__ x,
                                                               int64_t xs, uint8_t* __restrict__ q,
                                                               int64_t qs, float* __restrict__ s,
                                                               int N, void* __restrict__ act = nullptr,
                                                               int64_t as = 0) {
  __shared__ float red[kBlock / kWave];
  const int64_t row = blockIdx.x;
  const int64_t xo = row * xs;
  float amax = 0.f;
  for (int i = threadIdx.x; i < N; i += kBlock) {
    const float v = generic_value<Tag, ACT>(x, xo + i);
    amax = fmaxf(amax, fabsf(v));
    if (ACT && act != nullptr) store_elem<Tag>(act, row * as + i, v);
  }
  amax = block_reduce<OpAmax>(amax, red);
  const float scale = amax / kFp8Max;
  if (threadIdx.x == 0) s[row] = scale;
  const float inv = (scale == 0.f) ? 0.f : 1.0f / scale;
  uint8_t* qr = q + row * qs;
  for (int i = threadIdx.x; i < N; i += kBlock)
    qr[i] = fp8_byte(generic_value<Tag, ACT>(x, xo + i) * inv);
}

template <class Tag, bool ACT = false>
int launch_quant(const void* x, int64_t M, int64_t N, int64_t xs, void* q, int64_t qs, float* s,
                 hipStream_t stream, void* act = nullptr, int64_t as = 0,
                 const char* op = "sgl_per_token_quant_fp8") {
  const bool vec_ok = (N % 8 == 0) && aligned(x, 16) && ((xs * Tag::kBytes) % 16 == 0) &&
                      aligned(q, 8) && (qs % 8 == 0) &&
                      (act == nullptr || (aligned(act, 16) && (as * Tag::kBytes) % 16 == 0));
  bool launched = false;
  if (vec_ok) {
    launched = dispatch_row_shape<8, false, 128>(N, [&](auto lpr, auto ch) {
      constexpr int LPR = decltype(lpr)::value;
      constexpr int CH = decltype(ch)::value;
      hipLaunchKernelGGL((quant_rows_kernel<Tag, LPR, CH, ACT>), dim3(row_blocks(M, LPR)),
                         dim3(kBlock), 0, stream, x, xs, static_cast<uint8_t*>(q), qs, s, M,
                         static_cast<int>(N), act, as);
    }, M);
  }
  if (!launched) {
    hipLaunchKernelGGL((quant_generic_kernel<Tag, ACT>), dim3(M), dim3(kBlock), 0, stream, x, xs,
                       static_cast<uint8_t*>(q), qs, s, static_cast<int>(N), act, as);
  }
  return launch_status(op);
}

// ---------------------------------------------------------------------------
// RMSNorm -> FP8. v = (x * r) * w in fp32 (rmsnorm.cu:41-60 without the
// rounding to the input type), r = 1/sqrt(mean(x^2) + eps) with IEEE
// division and sqrt, the sum of squares in fp32 in a fixed order (below, as
// the reference sums in fp32 in its own order, rmsnorm.cu:47-53); then the
// per_token_quant_fp8.cu:56-82 rule over the row (per token) or over each
// 1x128 block (16 lanes x 8 values of one chunk).
//
// These kernels are bound by VALU issue as much as by HBM: a wave holds a
// whole 3072-wide row (48 values per lane) and runs ~10 instructions per value
// (4 cycles each on a 16-lane SIMD), most of them only once its last chunk
// has arrived. So the loads are not predicated (a predicated load's join
// makes the compiler wait for every load before the first use), the sum of
// squares advances chunk by chunk as the chunks arrive, and the register
// budget is kept low enough that every row of a one-round grid is resident.
// ---------------------------------------------------------------------------

// At least 5 resident waves per SIMD (at most 96 registers): with one wave
// per row, 5120 slots hold a [4725, 3072] grid in one round. The compiler
// otherwise spends registers on unpacking the next phase's operands early
// (104 for the per-token kernel, 4 waves per SIMD).
constexpr int kC4WavesPerSimd = 5;

// Weight chunks first (cached: they arrive before the row), then the row's.
// A row past M reads row M - 1 and a lane past N reads chunk 0 of its row;
// their values are cleared (EXACT == false) and never stored.
//
// SHARED (one row per wave): the workgroup's four waves share one copy of
// the weight row through LDS, each loading a quarter of its chunks, which cuts
// the weight traffic through L2 fourfold ([4725, 3072] per 1x128 block:
// 10.2 -> 9.9 us on MI355X). The meeting point is a bare s_barrier behind an
// LDS-only wait: a fenced barrier would also wait for the row loads in flight.
template <class Tag, int LPR, int CH, bool EXACT, bool SHARED>
__device__ __forceinline__ void load_row_weight(const void* x, int64_t xs, const void* w,
                                                int64_t row, int lane, int N, u32x4 (&c)[CH],
                                                u32x4 (&wc)[CH]) {
  const void* xr = byte_off(x, row * xs * Tag::kBytes);
  if constexpr (SHARED) {
    static_assert(LPR == kWave, "one row per wave");
    constexpr int kWaves = kBlock / kWave;
    constexpr int kMine = (CH + kWaves - 1) / kWaves;
    __shared__ u32x4 wl[CH * LPR];
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
    u32x4 wt[kMine];
#pragma unroll
    for (int k = 0; k < kMine; ++k) {
      const int i = wave + kWaves * k;
      const int e = (i * LPR + lane) * 8;
      if (i < CH)
        wt[k] = ld16(byte_off(w, static_cast<int64_t>((EXACT || e < N) ? e : 0) * Tag::kBytes));
    }
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int e = (i * LPR + lane) * 8;
      c[i] = ld16_nt(byte_off(xr, static_cast<int64_t>((EXACT || e < N) ? e : 0) * Tag::kBytes));
    }
#pragma unroll
    for (int k = 0; k < kMine; ++k) {
      const int i = wave + kWaves * k;
      if (i < CH) wl[i * LPR + lane] = wt[k];
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are done
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < CH; ++i) wc[i] = wl[i * LPR + lane];
  } else {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int e = (i * LPR + lane) * 8;
      wc[i] = ld16(byte_off(w, static_cast<int64_t>((EXACT || e < N) ? e : 0) * Tag::kBytes));
    }
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int e = (i * LPR + lane) * 8;
      c[i] = ld16_nt(byte_off(xr, static_cast<int64_t>((EXACT || e < N) ? e : 0) * Tag::kBytes));
    }
  }
  if constexpr (!EXACT) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const bool in = (i * LPR + lane) * 8 < N;
      c[i] = u32x4{in ? c[i].x : 0u, in ? c[i].y : 0u, in ? c[i].z : 0u, in ? c[i].w : 0u};
      wc[i] = u32x4{in ? wc[i].x : 0u, in ? wc[i].y : 0u, in ? wc[i].z : 0u, in ? wc[i].w : 0u};
    }
  }
}

// This lane's sum of squares, in fp32 in a fixed order: two accumulators,
// element j of each chunk (chunks in order, j = 0..7) into accumulator j % 2
// with one fused multiply-add (x^2 of a bf16/fp16 value is exact in fp32, so
// each step is the correctly rounded acc + x^2), then acc[0] + acc[1]. The
// row's lanes are then added by allreduce's fixed butterfly (and, for rows
// wider than a wave, the waves' sums in order), so the mean square is a
// function of the row and its launch shape (LPR, CH), which the CPU oracle
// restates step by step. (An fp64 exact sum instead measured 1-3% slower on
// [10530, 3072] and [4725, 3072]: one more conversion per value and 64-bit
// cross-lane steps.) Each chunk's part is issued before the next chunk is
// waited for. KEEPX keeps the fp32 values of x for the product that follows
// (48 more registers, 48 fewer instructions per row); otherwise the unpacked
// values die here and are unpacked again.
template <class Tag, int CH, bool KEEPX>
__device__ __forceinline__ float lane_sum_squares(u32x4 (&c)[CH], float (&xf)[KEEPX ? CH : 1][8]) {
  float acc[2] = {0.f, 0.f};
#pragma unroll
  for (int i = 0; i < CH; ++i) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float f = elem<Tag>(c[i], j);
      if constexpr (KEEPX) xf[i][j] = f;
      acc[j & 1] = __builtin_fmaf(f, f, acc[j & 1]);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  const float ss = acc[0] + acc[1];
  if constexpr (!KEEPX) {
#pragma unroll
    for (int i = 0; i < CH; ++i) asm volatile("" : "+v"(c[i]));
  }
  return ss;
}

template <class Tag, int CH, bool KEEPX>
__device__ __forceinline__ float x_at(const u32x4 (&c)[CH], const float (&xf)[KEEPX ? CH : 1][8],
                                      int i, int j) {
  if constexpr (KEEPX)
    return xf[i][j];
  else
    return elem<Tag>(c[i], j);
}

// r = 1 / sqrt(ss / N + eps), each step an IEEE fp32 operation.
__device__ __forceinline__ float rms_rstd(float ss, int N, float eps) {
  const float ms = ss / static_cast<float>(N);
  return 1.0f / sqrtf(ms + eps);
}

// Per token. The row maximum is taken NaN-propagating: when it is finite (no
// NaN, no inf) it is the reference's amax and, with a finite inverse scale,
// the clamp cannot change a code, so it is skipped; rows of a wave
// (workgroup, for rows wider than a wave) holding a non-finite value take the
// NaN-skipping maximum and the clamp.
template <class Tag, int LPR, int CH, bool EXACT, bool KEEPX>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(kC4WavesPerSimd)))
void rmsnorm_quant_tok_kernel(
    const void* __restrict__ x, int64_t xs, const void* __restrict__ w, uint8_t* __restrict__ q,
    int64_t qs, float* __restrict__ s, int64_t M, int N, float eps) {
  static_assert(Tag::kVec == 8, "fp8 rows are built from 8-element chunks");
  constexpr int RPB = kBlock / LPR;
  __shared__ float red_ss[kBlock / kWave];
  __shared__ float red_max[kBlock / kWave];
  __shared__ float red_max2[kBlock / kWave];
  const int lane = threadIdx.x % LPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / LPR;
  const bool row_ok = row < M;
  u32x4 c[CH], wc[CH];
  load_row_weight<Tag, LPR, CH, EXACT, false>(x, xs, w, row_ok ? row : M - 1, lane, N, c, wc);
  float xf[KEEPX ? CH : 1][8];
  const float r =
      rms_rstd(row_reduce<LPR, OpSum>(lane_sum_squares<Tag, CH, KEEPX>(c, xf), red_ss), N, eps);

  float v[CH][8];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v[i][j] = (x_at<Tag, CH, KEEPX>(c, xf, i, j) * r) * elem<Tag>(wc[i], j);
      amax = nan_max_abs(amax, v[i][j]);
    }
  }
  bool any_nonfinite;
  amax = row_amax_vote<LPR>(amax, red_max, any_nonfinite);
  const bool finite_row = finite_bits(amax);
  if (any_nonfinite) {
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < CH; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(v[i][j]));
    amax = row_reduce<LPR, OpAmax>(m, red_max2);
  }
  const float scale = amax / kFp8Max;
  if (row_ok && lane == 0) s[row] = scale;
  const float inv = (scale == 0.f) ? 0.f : 1.0f / scale;
  const bool fast = finite_row && finite_bits(inv);
  if (!row_ok) return;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int e = (i * LPR + lane) * 8;
    if (EXACT || e < N)
      st8_nt(q + row * qs + e, fast ? quant8<false>(v[i], inv) : quant8<true>(v[i], inv));
  }
}

// Per 1x128 block: each 16-lane DPP row of a chunk holds one block. Same
// fast / exact paths as per token, decided per block; the vote for the
// NaN-skipping maxima is wave-wide (workgroup-wide for rows wider than a wave).
template <class Tag, int LPR, int CH, bool EXACT, bool KEEPX, bool SHARED>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(kC4WavesPerSimd)))
void rmsnorm_quant_blk_kernel(
    const void* __restrict__ x, int64_t xs, const void* __restrict__ w, uint8_t* __restrict__ q,
    int64_t qs, float* __restrict__ s, int64_t M, int N, float eps) {
  static_assert(Tag::kVec == 8 && LPR >= 16, "block layout");
  constexpr int RPB = kBlock / LPR;
  __shared__ float red_ss[kBlock / kWave];
  const int lane = threadIdx.x % LPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / LPR;
  const bool row_ok = row < M;
  u32x4 c[CH], wc[CH];
  load_row_weight<Tag, LPR, CH, EXACT, SHARED>(x, xs, w, row_ok ? row : M - 1, lane, N, c, wc);
  float xf[KEEPX ? CH : 1][8];
  const float r =
      rms_rstd(row_reduce<LPR, OpSum>(lane_sum_squares<Tag, CH, KEEPX>(c, xf), red_ss), N, eps);

  float v[CH][8];
  float gmax[CH];
  bool all_finite = true;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v[i][j] = (x_at<Tag, CH, KEEPX>(c, xf, i, j) * r) * elem<Tag>(wc[i], j);
      m = nan_max_abs(m, v[i][j]);
    }
    if constexpr (KEEPX) {
      gmax[i] = m;
    } else {
      gmax[i] = allreduce_amax<16>(m);
      all_finite = all_finite && finite_bits(gmax[i]);
    }
    __builtin_amdgcn_sched_barrier(0);  // chunk by chunk: c[i], wc[i] die here
  }
  if constexpr (KEEPX) {
    // The chunks' 16-lane maxima as CH independent DPP chains, which the
    // scheduler interleaves instead of padding each step with wait states
    // ([10530, 3072]: 18.5-18.7 -> 18.2-18.4 us; in the register-capped
    // one-round kernel below 8192 rows it measured slower, 9.6 -> 9.8-10.0 us).
#pragma unroll
    for (int i = 0; i < CH; ++i) gmax[i] = allreduce_amax<16>(gmax[i]);
#pragma unroll
    for (int i = 0; i < CH; ++i) all_finite = all_finite && finite_bits(gmax[i]);
  }
  bool fast[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) fast[i] = finite_bits(gmax[i]);
  if (rows_any<LPR>(!all_finite)) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      float m = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(v[i][j]));
      gmax[i] = allreduce_amax<16>(m);
    }
  }
  const int nblk = N / 128;
  float ginv[CH];
  if constexpr (LPR >= kWave) {
    // A wave holds 4*CH blocks: lane b < 4*CH takes block b's maximum, runs
    // the two IEEE divisions once, and hands each chunk its inverse back.
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
    const int ge = ((wl >> 2) * LPR + wave_in_row * kWave + (wl & 3) * 16) * 8;  // block's first element
    if (row_ok && wl < 4 * CH && ge < N) s[row * nblk + ge / 128] = gs;
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
      if (row_ok && e < N && (lane & 15) == 0) s[row * nblk + e / 128] = gs;
    }
  }
  if (!row_ok) return;
  // One wave-uniform branch when every block of the wave takes the clamp-free
  // path (a per-block select would run both conversions).
  bool lane_fast = true;
#pragma unroll
  for (int i = 0; i < CH; ++i) lane_fast = lane_fast && fast[i] && finite_bits(ginv[i]);
  if (__builtin_amdgcn_ballot_w64(!lane_fast) == 0) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int e = (i * LPR + lane) * 8;
      if (EXACT || e < N) st8_nt(q + row * qs + e, quant8<false>(v[i], ginv[i]));
    }
  } else {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int e = (i * LPR + lane) * 8;
      if (EXACT || e < N)
        st8_nt(q + row * qs + e, (fast[i] && finite_bits(ginv[i])) ? quant8<false>(v[i], ginv[i])
                                                                  : quant8<true>(v[i], ginv[i]));
    }
  }
}

// Launch shapes (MI355X, [T, 3072] bf16, interleaved A/B against the previous
// kernels): per token, fewer rows than wave slots keeps 74 registers so all
// rows are resident in one round (T = 4725: 10.3 -> 9.7 us), more rows keeps
// x in fp32 (T = 10530: 18.5 -> 17.8 us); per block (T = 10530: 19.7 -> 18.6
// us), and with fewer rows than wave slots the weight row is shared through
// LDS (T = 4725: 10.2 -> 9.9 us; per token and with more rows it measured no
// gain). Two or three rows per wave, each row's arithmetic overlapping the
// next row's arrival, measured slower (T = 4725 per token 9.6 -> 10.4 us).
template <class Tag>
int launch_rmsnorm_quant(const void* x, int64_t xs, const void* w, void* q, int64_t qs, float* s,
                         int64_t M, int64_t N, float eps, int64_t group, hipStream_t stream) {
  uint8_t* q8 = static_cast<uint8_t*>(q);
  const int n = static_cast<int>(N);
  bool launched = false;
  if (group == 0) {
    launched = dispatch_row_shape<8>(N, [&](auto lpr, auto ch) {
      constexpr int LPR = decltype(lpr)::value;
      constexpr int CH = decltype(ch)::value;
      const dim3 grid(static_cast<unsigned>(row_blocks(M, LPR)));
      const bool exact = int64_t{LPR} * CH * 8 == N;
      if (M >= kFewRows) {
        if (exact)
          hipLaunchKernelGGL((rmsnorm_quant_tok_kernel<Tag, LPR, CH, true, true>), grid,
                             dim3(kBlock), 0, stream, x, xs, w, q8, qs, s, M, n, eps);
        else
          hipLaunchKernelGGL((rmsnorm_quant_tok_kernel<Tag, LPR, CH, false, true>), grid,
                             dim3(kBlock), 0, stream, x, xs, w, q8, qs, s, M, n, eps);
      } else {
        if (exact)
          hipLaunchKernelGGL((rmsnorm_quant_tok_kernel<Tag, LPR, CH, true, false>), grid,
                             dim3(kBlock), 0, stream, x, xs, w, q8, qs, s, M, n, eps);
        else
          hipLaunchKernelGGL((rmsnorm_quant_tok_kernel<Tag, LPR, CH, false, false>), grid,
                             dim3(kBlock), 0, stream, x, xs, w, q8, qs, s, M, n, eps);
      }
    });
  } else {
    launched = dispatch_row_shape<8>(N, [&](auto lpr, auto ch) {
      constexpr int LPR = decltype(lpr)::value < 16 ? 16 : decltype(lpr)::value;
      constexpr int CH = decltype(ch)::value;
      const dim3 grid(static_cast<unsigned>(row_blocks(M, LPR)));
      const bool exact = int64_t{LPR} * CH * 8 == N;
      if (M >= kFewRows) {
        if (exact)
          hipLaunchKernelGGL((rmsnorm_quant_blk_kernel<Tag, LPR, CH, true, true, false>), grid,
                             dim3(kBlock), 0, stream, x, xs, w, q8, qs, s, M, n, eps);
        else
          hipLaunchKernelGGL((rmsnorm_quant_blk_kernel<Tag, LPR, CH, false, true, false>), grid,
                             dim3(kBlock), 0, stream, x, xs, w, q8, qs, s, M, n, eps);
      } else {
        if (exact)
          hipLaunchKernelGGL((rmsnorm_quant_blk_kernel<Tag, LPR, CH, true, false, LPR == kWave>), grid,
                             dim3(kBlock), 0, stream, x, xs, w, q8, qs, s, M, n, eps);
        else
          hipLaunchKernelGGL((rmsnorm_quant_blk_kernel<Tag, LPR, CH, false, false, LPR == kWave>), grid,
                             dim3(kBlock), 0, stream, x, xs, w, q8, qs, s, M, n, eps);
      }
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
  JO_REQUIRE(num_tokens <= kMaxRows, "per_token_quant_fp8: shape too large (more than %lld rows)",
             static_cast<long long>(kMaxRows));
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

extern "C" int jo_gelu_tanh_quant_fp8(const void* input, int dtype, int64_t num_tokens,
                                     int64_t hidden_dim, int64_t in_stride, void* output_q,
                                     int64_t q_stride, float* output_s, void* output_act,
                                     int64_t act_stride, void* stream) {
  JO_REQUIRE(dtype == JO_DTYPE_BF16 || dtype == JO_DTYPE_F16,
             "gelu_tanh_quant_fp8: input must be bf16 or fp16");
  JO_REQUIRE(num_tokens >= 0 && hidden_dim >= 0, "gelu_tanh_quant_fp8: negative size");
  JO_REQUIRE(hidden_dim % 4 == 0, "hidden_dim must be divisible by 4, got %lld",
             static_cast<long long>(hidden_dim));
  JO_REQUIRE(hidden_dim <= INT32_MAX, "gelu_tanh_quant_fp8: hidden_dim too large");
  JO_REQUIRE(num_tokens <= kMaxRows, "gelu_tanh_quant_fp8: shape too large (more than %lld rows)",
             static_cast<long long>(kMaxRows));
  JO_REQUIRE(in_stride >= hidden_dim && q_stride >= hidden_dim,
             "gelu_tanh_quant_fp8: row stride smaller than hidden_dim");
  JO_REQUIRE(output_act == nullptr || act_stride >= hidden_dim,
             "gelu_tanh_quant_fp8: activation row stride smaller than hidden_dim");
  if (num_tokens == 0) return JO_OK;
  JO_REQUIRE(input && output_q && output_s, "gelu_tanh_quant_fp8: null pointer");
  if (output_act != nullptr && hidden_dim > 0) {
    // The element-wise path stores the activation of a row before it reads
    // the row again to quantize it, so the activation must not overlap the
    // input (the byte ranges the two row-strided views span).
    const auto lo_in = reinterpret_cast<uintptr_t>(input);
    const auto lo_act = reinterpret_cast<uintptr_t>(output_act);
    const uintptr_t hi_in = lo_in + static_cast<uintptr_t>((num_tokens - 1) * in_stride + hidden_dim) * 2;
    const uintptr_t hi_act = lo_act + static_cast<uintptr_t>((num_tokens - 1) * act_stride + hidden_dim) * 2;
    JO_REQUIRE(hi_in <= lo_act || hi_act <= lo_in,
               "gelu_tanh_quant_fp8: output_act must not overlap input");
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == JO_DTYPE_BF16)
    return launch_quant<BF16, true>(input, num_tokens, hidden_dim, in_stride, output_q, q_stride,
                                    output_s, st, output_act, act_stride, "gelu_tanh_quant_fp8");
  return launch_quant<F16, true>(input, num_tokens, hidden_dim, in_stride, output_q, q_stride,
                                 output_s, st, output_act, act_stride, "gelu_tanh_quant_fp8");
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
  JO_REQUIRE(M >= 0 && N > 0 && N <= INT32_MAX && M <= kMaxRows,
             "rmsnorm_quant_fp8: bad shape [%lld, %lld]", static_cast<long long>(M),
             static_cast<long long>(N));
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
