// Device-side building blocks shared by the joyomni gfx950 kernels.
//
// Everything here is written for CDNA4 wave64: 16-byte global accesses,
// cross-lane reductions with DPP row operations (within 16-lane rows),
// ds_swizzle (across the two rows of a 32-lane half) and readlane (across
// the two halves), and the gfx950 conversion instructions for bf16
// (v_cvt_pk_bf16_f32, round-to-nearest-even) and OCP fp8 e4m3fn
// (v_cvt_pk_fp8_f32, round-to-nearest-even).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace jo {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr int kBlock = 256;  // threads per workgroup for every row kernel
constexpr float kFp8Max = 448.0f;

// x / n for a row length n > 0, rounded as the IEEE division: when n is a
// power of two the quotient is x scaled by an exact 2^-k, one rounding either
// way (the branch is uniform: n is a kernel argument).
__device__ __forceinline__ float div_by_len(float x, int n) {
  if (n > 0 && (n & (n - 1)) == 0)
    return x * __builtin_bit_cast(float, static_cast<uint32_t>(127 - __builtin_ctz(n)) << 23);
  return x / static_cast<float>(n);
}

// ---------------------------------------------------------------------------
// Element types. kVec = elements carried by one 16-byte chunk.
// ---------------------------------------------------------------------------
struct BF16 {
  static constexpr int kVec = 8;
  static constexpr int kBytes = 2;
};
struct F16 {
  static constexpr int kVec = 8;
  static constexpr int kBytes = 2;
};
struct F32 {
  static constexpr int kVec = 4;
  static constexpr int kBytes = 4;
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) {
  return __builtin_bit_cast(float, w & 0xffff0000u);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
__device__ __forceinline__ f32x2 unpack_f16x2(uint32_t w) {
  return __builtin_convertvector(__builtin_bit_cast(f16x2, w), f32x2);
}
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}

// One element of a 16-byte chunk as fp32.
template <class Tag>
__device__ __forceinline__ float elem(const u32x4& c, int j);

template <>
__device__ __forceinline__ float elem<BF16>(const u32x4& c, int j) {
  const uint32_t w = c[j >> 1];
  return (j & 1) ? bf16_hi(w) : bf16_lo(w);
}
template <>
__device__ __forceinline__ float elem<F16>(const u32x4& c, int j) {
  const f32x2 v = unpack_f16x2(c[j >> 1]);
  return (j & 1) ? v.y : v.x;
}
template <>
__device__ __forceinline__ float elem<F32>(const u32x4& c, int j) {
  // Copy the element out first: __builtin_bit_cast applied directly to an
  // ext-vector element expression reads element 0 with this compiler.
  const uint32_t w = c[j];
  return __builtin_bit_cast(float, w);
}

// All kVec elements of a chunk as fp32.
template <class Tag>
__device__ __forceinline__ void unpack(const u32x4& c, float (&f)[Tag::kVec]) {
#pragma unroll
  for (int j = 0; j < Tag::kVec; ++j) f[j] = elem<Tag>(c, j);
}

// kVec fp32 values rounded (nearest-even) into one 16-byte chunk.
template <class Tag>
__device__ __forceinline__ u32x4 pack(const float (&f)[Tag::kVec]);

template <>
__device__ __forceinline__ u32x4 pack<BF16>(const float (&f)[8]) {
  return u32x4{pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
               pack_bf16x2(f[6], f[7])};
}
template <>
__device__ __forceinline__ u32x4 pack<F16>(const float (&f)[8]) {
  return u32x4{pack_f16x2(f[0], f[1]), pack_f16x2(f[2], f[3]), pack_f16x2(f[4], f[5]),
               pack_f16x2(f[6], f[7])};
}
template <>
__device__ __forceinline__ u32x4 pack<F32>(const float (&f)[4]) {
  return u32x4{__builtin_bit_cast(uint32_t, f[0]), __builtin_bit_cast(uint32_t, f[1]),
               __builtin_bit_cast(uint32_t, f[2]), __builtin_bit_cast(uint32_t, f[3])};
}

// v rounded (nearest-even) to the element type and widened back to fp32:
// the value a store of v followed by a load would give.
template <class Tag>
__device__ __forceinline__ float round_to(float v);
template <>
__device__ __forceinline__ float round_to<BF16>(float v) {
  return float(__bf16(v));
}
template <>
__device__ __forceinline__ float round_to<F16>(float v) {
  return float(_Float16(v));
}
template <>
__device__ __forceinline__ float round_to<F32>(float v) {
  return v;
}

// Scalar element load / store (generic fallback kernels).
template <class Tag>
__device__ __forceinline__ float load_elem(const void* p, int64_t i);
template <>
__device__ __forceinline__ float load_elem<BF16>(const void* p, int64_t i) {
  return __builtin_bit_cast(float, uint32_t(static_cast<const uint16_t*>(p)[i]) << 16);
}
template <>
__device__ __forceinline__ float load_elem<F16>(const void* p, int64_t i) {
  return float(static_cast<const _Float16*>(p)[i]);
}
template <>
__device__ __forceinline__ float load_elem<F32>(const void* p, int64_t i) {
  return static_cast<const float*>(p)[i];
}
template <class Tag>
__device__ __forceinline__ void store_elem(void* p, int64_t i, float v);
template <>
__device__ __forceinline__ void store_elem<BF16>(void* p, int64_t i, float v) {
  static_cast<__bf16*>(p)[i] = __bf16(v);
}
template <>
__device__ __forceinline__ void store_elem<F16>(void* p, int64_t i, float v) {
  static_cast<_Float16*>(p)[i] = _Float16(v);
}
template <>
__device__ __forceinline__ void store_elem<F32>(void* p, int64_t i, float v) {
  static_cast<float*>(p)[i] = v;
}

// ---------------------------------------------------------------------------
// 16-byte global accesses.
// ---------------------------------------------------------------------------
// ld16/st16/st8: cached accesses, for data that is reused (weights, one
// broadcast modulation row, rotation tables). The *_nt forms are the
// streaming accesses for row data that is touched exactly once: they carry
// the nontemporal hint so the stream does not churn L2 and the Infinity Cache
// (measured on MI355X: read-16B/write-8B rows at the C1 shape go from 5.1 to
// 5.8 TB/s).
__device__ __forceinline__ u32x4 ld16(const void* p) { return *static_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, const u32x4& v) { *static_cast<u32x4*>(p) = v; }
__device__ __forceinline__ void st8(void* p, const u32x2& v) { *static_cast<u32x2*>(p) = v; }
__device__ __forceinline__ u32x4 ld16_nt(const void* p) {
  return __builtin_nontemporal_load(static_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16_nt(void* p, const u32x4& v) {
  __builtin_nontemporal_store(v, static_cast<u32x4*>(p));
}
__device__ __forceinline__ void st8_nt(void* p, const u32x2& v) {
  __builtin_nontemporal_store(v, static_cast<u32x2*>(p));
}

// Division of a 32-bit unsigned n by a divisor fixed for a launch, as a
// multiply-high, a subtraction, an add and two shifts instead of the ~15
// instructions of an integer division by a run-time value (Granlund and
// Montgomery, "Division by invariant integers using multiplication", PLDI
// 1994, the round-up method of their section 4 with the N+1-bit multiplier
// 2^32 + m): with l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1,
// t = mulhi(m, n), n / d = (t + ((n - t) >> min(l, 1))) >> max(l - 1, 0).
// Exact for every n < 2^32 and 1 <= d < 2^32. make_fastdiv runs on the host;
// fdiv on either side (the 64-bit product's high half is v_mul_hi_u32 on the
// device).
struct FastDiv {
  uint32_t d, m;
  int s1, s2;
};

inline FastDiv make_fastdiv(uint32_t d) {
  if (d == 0) return FastDiv{0, 0, 0, 0};  // callers pass d >= 1; no division by zero here
  int l = 0;
  while ((uint64_t{1} << l) < d) ++l;
  const uint64_t m = ((uint64_t{1} << 32) * ((uint64_t{1} << l) - d)) / d + 1;
  return FastDiv{d, static_cast<uint32_t>(m), l < 1 ? l : 1, l > 1 ? l - 1 : 0};
}

__host__ __device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
  const uint32_t t = static_cast<uint32_t>((uint64_t{n} * f.m) >> 32);
  return (t + ((n - t) >> f.s1)) >> f.s2;
}

// 16-byte store with the system-scope nontemporal policy (sc0 sc1 nt: the
// line is written through rather than left dirty in L2), through a raw
// buffer resource. `base` must be wave-uniform (a row base computed from the
// wave index), so that the resource lives in scalar registers; `off` is the
// lane's byte offset from it, below 2^31. Measured on MI355X for the QK
// kernels' in-place row stores: [1, 1560, 32, 128] with tables 10.26-10.52 ->
// 10.01 us, [1, 3120, 32, 128] 17.65 -> 17.43-17.55 us, [1, 3510, 24, 128]
// grid 15.83 -> 15.60-15.78 us; the ring-cache mode, whose k rows go to
// another buffer, measured 0.8% slower with it and keeps st16_nt, as do the
// other row kernels (bare streams of their shapes showed no gain).
__device__ __forceinline__ void st16_sys_nt(const void* base, int off, const u32x4& v) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(base), static_cast<short>(0), 0x7fffffff, 0x00020000);
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 19);  // 19 = sc0 | nt | sc1
}

__device__ __forceinline__ const void* byte_off(const void* p, int64_t bytes) {
  return static_cast<const char*>(p) + bytes;
}
__device__ __forceinline__ void* byte_off(void* p, int64_t bytes) {
  return static_cast<char*>(p) + bytes;
}

// ---------------------------------------------------------------------------
// FP8 e4m3fn.
// The clamp reproduces fmaxf(fminf(v, 448), -448): a NaN becomes +448.
// v_cvt_pk_fp8_f32 rounds to nearest-even; the clamp keeps every input in the
// finite range, so the result equals a saturating conversion.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float fp8_clamp(float v) { return fmaxf(fminf(v, kFp8Max), -kFp8Max); }

// Four values -> four e4m3fn bytes (element 0 in the lowest byte).
// CLAMP = true applies the clamp first (any input, NaN -> +448).
// CLAMP = false is for finite inputs with |v| <= 464: v_cvt_pk_fp8_f32 then
// rounds to nearest-even onto the finite codes (measured on MI355X: values in
// (448, 464] give 448, above 464 NaN), which equals clamping first. The
// quantizers use it for rows whose values and inverse scale are finite, where
// |x * inv| <= amax * inv <= 448 * (1 + 3 * 2^-24).
template <bool CLAMP = true>
__device__ __forceinline__ uint32_t fp8x4(float a, float b, float c, float d) {
  if constexpr (CLAMP) {
    a = fp8_clamp(a);
    b = fp8_clamp(b);
    c = fp8_clamp(c);
    d = fp8_clamp(d);
  }
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return static_cast<uint32_t>(w);
}

// Quantizes 8 fp32 values with the reference's rule and returns 8 bytes.
// CLAMP = false only where the inputs are finite and inv is finite (see fp8x4).
template <bool CLAMP = true>
__device__ __forceinline__ u32x2 quant8(const float (&v)[8], float inv) {
  return u32x2{fp8x4<CLAMP>(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv),
               fp8x4<CLAMP>(v[4] * inv, v[5] * inv, v[6] * inv, v[7] * inv)};
}

// One value -> its e4m3fn byte, with the clamp (any input).
__device__ __forceinline__ uint8_t fp8_byte(float v) {
  return static_cast<uint8_t>(__builtin_amdgcn_cvt_pk_fp8_f32(fp8_clamp(v), 0.f, 0, false) & 0xff);
}

// max(m, |v|) propagating NaN (IEEE maximum; v_maximum3_f32 on gfx950).
// Starting from 0, a row maximum built with it is +0..+inf, or a NaN whose
// bit pattern sorts above +inf; allreduce_amax's unsigned compare keeps that
// order, so "row maximum is finite" means "no NaN and no inf in the row".
__device__ __forceinline__ float nan_max_abs(float m, float v) {
  return __builtin_elementwise_maximum(m, __builtin_fabsf(v));
}
__device__ __forceinline__ bool finite_bits(float v) {
  return (__builtin_bit_cast(uint32_t, v) & 0x7fffffffu) < 0x7f800000u;
}

// ---------------------------------------------------------------------------
// Cross-lane reductions.
// allreduce<W>(v) combines v over aligned groups of W consecutive lanes
// (W in {8, 16, 32, 64}) and returns the result in every lane of the group.
// Every lane of a group ends with bit-identical values: each step combines a
// lane with a partner holding the mirror partial, and + / max commute.
// ---------------------------------------------------------------------------
struct OpSum {
  __device__ __forceinline__ static float apply(float a, float b) { return a + b; }
};
struct OpMax {
  __device__ __forceinline__ static float apply(float a, float b) { return fmaxf(a, b); }
};
// Max of non-negative values (|x| maxima from 0, possibly a positive NaN
// pattern): compares bit patterns as unsigned integers at every step, so a
// NaN (which sorts above +inf) survives the cross-wave combine as well.
struct OpAmax {
  __device__ __forceinline__ static float apply(float a, float b) {
    return __builtin_bit_cast(
        float, max(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b)));
  }
};

template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                               kCtrl, 0xf, 0xf, false));
}
// DPP controls (gfx9 encoding).
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppRor4 = 0x124;       // row_ror:4
constexpr int kDppRor8 = 0x128;       // row_ror:8
constexpr int kDppHalfMirror = 0x141; // row_half_mirror

__device__ __forceinline__ float swizzle_xor16(float v) {
  // ds_swizzle bit mode: and_mask 0x1f, or_mask 0, xor_mask 0x10.
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401f));
}
__device__ __forceinline__ float readlane(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

template <int W, class Op>
__device__ __forceinline__ float allreduce(float v) {
  static_assert(W == 8 || W == 16 || W == 32 || W == 64, "group width");
  if constexpr (W == 8) {
    v = Op::apply(v, dpp<kDppHalfMirror>(v));
  } else {
    v = Op::apply(v, dpp<kDppRor8>(v));
    v = Op::apply(v, dpp<kDppRor4>(v));
  }
  v = Op::apply(v, dpp<kDppXor2>(v));
  v = Op::apply(v, dpp<kDppXor1>(v));
  if constexpr (W >= 32) v = Op::apply(v, swizzle_xor16(v));
  if constexpr (W == 64) v = Op::apply(readlane(v, 0), readlane(v, 32));
  return v;
}

// Maximum of non-negative, non-NaN floats over aligned groups of W lanes.
// For such values the IEEE order equals the unsigned order of the bit
// patterns, so the reduction runs on integers (no NaN canonicalization
// between DPP steps). Used for amax values built with fmaxf from 0, which
// skips NaNs and is never negative.
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(v), kCtrl, 0xf, 0xf, false));
}
template <int W>
__device__ __forceinline__ float allreduce_amax(float x) {
  static_assert(W == 8 || W == 16 || W == 32 || W == 64, "group width");
  uint32_t v = __builtin_bit_cast(uint32_t, x);
  if constexpr (W == 8) {
    v = max(v, dpp_u32<kDppHalfMirror>(v));
  } else {
    v = max(v, dpp_u32<kDppRor8>(v));
    v = max(v, dpp_u32<kDppRor4>(v));
  }
  v = max(v, dpp_u32<kDppXor2>(v));
  v = max(v, dpp_u32<kDppXor1>(v));
  if constexpr (W >= 32)
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(v), 0x401f)));
  if constexpr (W == 64)
    v = max(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 0)),
            static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 32)));
  return __builtin_bit_cast(float, v);
}

// float64 sum over aligned groups of W lanes (W in {8, 16, 32, 64}); DPP and
// swizzle move the two 32-bit halves separately. Every lane of a group ends
// with bit-identical values (same argument as allreduce).
template <int kCtrl>
__device__ __forceinline__ double dpp64(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(u & 0xffffffffu), kCtrl, 0xf, 0xf, false);
  const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(u >> 32), kCtrl, 0xf, 0xf, false);
  return __builtin_bit_cast(double, (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                                        static_cast<uint32_t>(lo));
}
__device__ __forceinline__ double swizzle_xor16_f64(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const int lo = __builtin_amdgcn_ds_swizzle(static_cast<int>(u & 0xffffffffu), 0x401f);
  const int hi = __builtin_amdgcn_ds_swizzle(static_cast<int>(u >> 32), 0x401f);
  return __builtin_bit_cast(double, (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                                        static_cast<uint32_t>(lo));
}
__device__ __forceinline__ double readlane64(double v, int lane) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(u & 0xffffffffu), lane);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(u >> 32), lane);
  return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

template <int W>
__device__ __forceinline__ double allreduce_sum64(double v) {
  static_assert(W == 8 || W == 16 || W == 32 || W == 64, "group width");
  if constexpr (W == 8) {
    v += dpp64<kDppHalfMirror>(v);
  } else {
    v += dpp64<kDppRor8>(v);
    v += dpp64<kDppRor4>(v);
  }
  v += dpp64<kDppXor2>(v);
  v += dpp64<kDppXor1>(v);
  if constexpr (W >= 32) v += swizzle_xor16_f64(v);
  if constexpr (W == 64) v = readlane64(v, 0) + readlane64(v, 32);
  return v;
}

// float64 sum over LPR lanes of a 256-thread block; `slot` is __shared__ double[4].
template <int LPR>
__device__ __forceinline__ double row_reduce_sum64(double v, double* slot) {
  if constexpr (LPR <= kWave) {
    return allreduce_sum64<LPR>(v);
  } else {
    static_assert(LPR == 128 || LPR == 256, "lanes per row");
    v = allreduce_sum64<kWave>(v);
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) slot[wave] = v;
    __syncthreads();
    constexpr int kWavesPerRow = LPR / kWave;
    const int first = (wave / kWavesPerRow) * kWavesPerRow;
    double r = slot[first];
#pragma unroll
    for (int i = 1; i < kWavesPerRow; ++i) r += slot[first + i];
    return r;
  }
}

// Reduction over LPR lanes of a 256-thread block (LPR in {8..256}). Groups
// wider than a wave exchange per-wave partials through LDS; `slot` is a
// __shared__ float[4] scratch owned by the caller (one per reduction in
// flight). All threads of the block must call it (it may hit a barrier).
template <int W, class Op>
__device__ __forceinline__ float wave_reduce(float v) {
  if constexpr (std::is_same_v<Op, OpAmax>)
    return allreduce_amax<W>(v);
  else
    return allreduce<W, Op>(v);
}

template <int LPR, class Op>
__device__ __forceinline__ float row_reduce(float v, float* slot) {
  if constexpr (LPR <= kWave) {
    return wave_reduce<LPR, Op>(v);
  } else {
    static_assert(LPR == 128 || LPR == 256, "lanes per row");
    v = wave_reduce<kWave, Op>(v);
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) slot[wave] = v;
    __syncthreads();
    constexpr int kWavesPerRow = LPR / kWave;
    const int first = (wave / kWavesPerRow) * kWavesPerRow;
    float r = slot[first];
#pragma unroll
    for (int i = 1; i < kWavesPerRow; ++i) r = Op::apply(r, slot[first + i]);
    return r;
  }
}

// True on every lane of the rows that share this thread's reduction group
// when `pred` holds on any of their lanes: a wave-wide vote when a row fits in
// a wave (no barrier; the rows of one wave then take the same branch), else a
// block-wide one. (Measured on the per-token quantizer at [10530, 3072]:
// 17.7 -> 17.4 us against a block-wide vote; the norm kernels measured the
// same or slower with it and keep theirs.)
template <int LPR>
__device__ __forceinline__ bool rows_any(bool pred) {
  if constexpr (LPR <= kWave)
    return __builtin_amdgcn_ballot_w64(pred) != 0;
  else
    return __syncthreads_or(pred);
}

// Row maximum of non-negative values (OpAmax order: a NaN pattern sorts above
// +inf) over LPR lanes, and in any_nonfinite whether a row of the wave (rows
// that fit in a wave) or of the workgroup (wider rows) has a NaN or inf
// maximum — the same answer as row_reduce<LPR, OpAmax> followed by
// rows_any<LPR>(!finite), but for rows wider than a wave from one exchange
// through `slot` (__shared__ float[4]) and one barrier instead of two.
// Measured on MI355X: per-token quant [3120, 4096] (two waves per row)
// 8.00 -> 7.70 us, [3120, 16384] (four) 26.0 -> 25.7 us.
template <int LPR>
__device__ __forceinline__ float row_amax_vote(float v, float* slot, bool& any_nonfinite) {
  if constexpr (LPR <= kWave) {
    const float m = allreduce_amax<LPR>(v);
    any_nonfinite = __builtin_amdgcn_ballot_w64(!finite_bits(m)) != 0;
    return m;
  } else {
    static_assert(LPR == 128 || LPR == 256, "lanes per row");
    const float wm = allreduce_amax<kWave>(v);
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) slot[wave] = wm;
    __syncthreads();
    constexpr int kWavesPerRow = LPR / kWave;
    const int first = (wave / kWavesPerRow) * kWavesPerRow;
    float rm = slot[first];
#pragma unroll
    for (int i = 1; i < kWavesPerRow; ++i) rm = OpAmax::apply(rm, slot[first + i]);
    float all = slot[0];
#pragma unroll
    for (int i = 1; i < kBlock / kWave; ++i) all = OpAmax::apply(all, slot[i]);
    any_nonfinite = !finite_bits(all);
    return rm;
  }
}

// threadIdx.x / LPR, the row of the calling thread within its workgroup. For
// one-wave rows it goes through readfirstlane, so that the row's index and
// address arithmetic is scalar (the compiler cannot tell on its own that
// threadIdx.x / 64 is wave-uniform). Measured on MI355X with the per-token
// quantizer: [3120, 16384] (256 lanes) 26.6 -> 25.9 us, [10530, 3072] level;
// the two-wave rows of [3120, 4096] (128 lanes) measured 8% slower with it,
// so they keep the vector form.
template <int LPR>
__device__ __forceinline__ int wave_uniform_row() {
  if constexpr (LPR == kWave || LPR == 4 * kWave)
    return __builtin_amdgcn_readfirstlane(threadIdx.x / LPR);
  else
    return threadIdx.x / LPR;
}

// Row block of workgroup b (of nb) for kernels that also write a few fp32
// scales per row. Workgroups are dispatched round-robin over the 8 XCDs
// (workgroup b runs on XCD b % 8), so in launch order the scales of 32
// consecutive rows (one 128-byte line) would come from 8 XCDs, and each
// XCD's L2 would write its part of the line back on its own. Within every
// block of 8*G workgroups the index is transposed so that each XCD runs G
// consecutive workgroups, i.e. 32 consecutive rows and whole lines of
// scales; workgroups after the last whole block keep their order. The rows
// and outputs stream as before (the 8 XCDs still work on one window of
// 8*G*RPB consecutive rows). Measured on MI355X with bare streams of the
// shape [10530, 3072] bf16 -> fp8 + 4-byte scales: 17.05 -> 16.89 us (the
// scale stores' cost drops from ~0.2 us to ~0.05 us; without scales the
// order changes nothing), and with the per-token quantizer on it
// 17.27 -> 17.10 us. Used there only: the same order measured level for the
// RMSNorm -> FP8 kernels and the FP8 epilogue of the residual + LayerNorm
// kernel, slower for the RMSNorm -> FP8 per-block kernel at [4725, 3072]
// (9.6-9.9 -> 10.1 us) and for two-wave rows ([3120, 4096]: 7.7 -> 9.4 us).
template <int RPB>
__device__ __forceinline__ int64_t xcd_row_block(int64_t b, int64_t nb) {
  static_assert(RPB >= 1 && RPB <= 32 && (RPB & (RPB - 1)) == 0, "rows per workgroup");
  constexpr int64_t G = 32 / RPB;
  constexpr int64_t kSpan = 8 * G;
  if (b >= (nb / kSpan) * kSpan) return b;
  const int64_t l = b % kSpan;
  return (b - l) + (l % 8) * G + l / 8;
}

// Block-wide reduction for the generic (one row per block) kernels.
template <class Op>
__device__ __forceinline__ float block_reduce(float v, float* slot) {
  v = wave_reduce<kWave, Op>(v);
  const int wave = threadIdx.x / kWave;
  __syncthreads();  // slot may still be read by a previous reduction
  if ((threadIdx.x & (kWave - 1)) == 0) slot[wave] = v;
  __syncthreads();
  float r = slot[0];
#pragma unroll
  for (int i = 1; i < kBlock / kWave; ++i) r = Op::apply(r, slot[i]);
  return r;
}

}  // namespace jo
