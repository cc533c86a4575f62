/*
 * Independent C restatement of the FP8 path — TEST INFRASTRUCTURE ONLY.
 *
 * fp8ref_encode() finds the OCP e4m3fn code nearest to a float by brute
 * force over all finite codes (ties to the code with an even mantissa, the
 * sign kept), i.e. IEEE round-to-nearest-even into e4m3fn. It shares no code
 * with torch's cast, so it pins the torch restatement in oracle/ops.py.
 *
 * fp8ref_per_token_quant() restates the reference kernel rule
 * (deploy/joyomni_ops/csrc/per_token_quant_fp8.cu:56-82):
 *   amax = fmaxf over |x| from 0 (NaN ignored), scale = amax / 448,
 *   inv = (scale == 0) ? 0 : 1 / scale, q = e4m3fn(fmaxf(fminf(x*inv, 448), -448)).
 * fp8ref_group_quant() applies the same rule to consecutive groups of a row.
 *
 * Built with -ffp-contract=off so every product and quotient is one IEEE
 * binary32 operation.
 */
#include <math.h>
#include <stdint.h>

/* Exact value of an e4m3fn code (bias 7, no infinities, 0x7f/0xff are NaN). */
double fp8ref_decode(uint8_t c) {
  const int sign = c >> 7;
  const int exp = (c >> 3) & 0xf;
  const int man = c & 0x7;
  double v;
  if (exp == 0xf && man == 0x7) return NAN;
  if (exp == 0)
    v = ldexp((double)man, -9); /* subnormal: man/8 * 2^-6 */
  else
    v = ldexp(1.0 + man / 8.0, exp - 7);
  return sign ? -v : v;
}

/* Nearest finite e4m3fn code to v with the sign of v; ties to even mantissa.
 * |v| beyond the largest finite value (448) saturates to +-448; NaN -> 0x7f. */
uint8_t fp8ref_encode(float v) {
  if (isnan(v)) return 0x7f;
  const int neg = signbit(v) ? 1 : 0;
  const double a = fabs((double)v);
  uint8_t best = 0;
  double best_d = INFINITY;
  for (int m = 0; m < 0x7f; ++m) { /* magnitudes 0x00..0x7e */
    const double d = fabs(fp8ref_decode((uint8_t)m) - a);
    if (d < best_d || (d == best_d && (m & 1) == 0)) {
      best_d = d;
      best = (uint8_t)m;
    }
  }
  return (uint8_t)(best | (neg << 7));
}

static float clamp448(float v) { return fmaxf(fminf(v, 448.0f), -448.0f); }

static void quant_span(const float* x, int64_t n, uint8_t* q, float* s) {
  float amax = 0.0f;
  for (int64_t j = 0; j < n; ++j) amax = fmaxf(amax, fabsf(x[j]));
  const float scale = amax / 448.0f;
  const float inv = (scale == 0.0f) ? 0.0f : 1.0f / scale;
  *s = scale;
  for (int64_t j = 0; j < n; ++j) q[j] = fp8ref_encode(clamp448(x[j] * inv));
}

/* x: fp32 [M, K] row-major (bf16/fp16 inputs widened exactly by the caller). */
void fp8ref_per_token_quant(const float* x, int64_t M, int64_t K, uint8_t* q, float* s) {
  for (int64_t r = 0; r < M; ++r) quant_span(x + r * K, K, q + r * K, s + r);
}

/* Per-group scales: s is [M, K/group] row-major. K % group == 0. */
void fp8ref_group_quant(const float* x, int64_t M, int64_t K, int64_t group, uint8_t* q,
                        float* s) {
  const int64_t G = K / group;
  for (int64_t r = 0; r < M; ++r)
    for (int64_t g = 0; g < G; ++g)
      quant_span(x + r * K + g * group, group, q + r * K + g * group, s + r * G + g);
}

/* Encode an array of already-clamped floats (used to pin torch's cast). */
void fp8ref_encode_array(const float* v, int64_t n, uint8_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = fp8ref_encode(v[i]);
}
