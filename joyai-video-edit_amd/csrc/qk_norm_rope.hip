// Fused per-head QK RMSNorm + interleaved-pair RoPE.
//
// One wave64 owns one (batch, token): it loads all heads of q and of k for
// that token with 16-byte accesses (a head of D bf16 is D/8 lanes; a wave
// load covers 512 contiguous elements = 512/D heads), so one token's
// rotation coefficients are fetched or computed once and reused for every
// head of q and k. Each head's sum of squares reduces over its D/8 lanes with
// DPP row operations. Three modes share the kernel:
//   TABLE  coefficients read from bf16 cos/sin [seq_len, D/2] tables
//          (drop-in for fused_qk_norm_rope_3d_paired);
//   GRID   coefficients computed in registers from the token's (t, h, w)
//          grid position: each lane evaluates sincos for D/128 (min 1) pairs
//          and the wave redistributes them with ds_bpermute;
//   KVC    GRID, with the rotated k written to a frame ring buffer instead
//          of in place.
#include <stdlib.h>

#include "jo_device.hpp"
#include "jo_host.hpp"

namespace jo {
namespace {

constexpr int kTable = 0;
constexpr int kGrid = 1;
constexpr int kKvCache = 2;

struct QKArgs {
  void* q;
  const void* k;
  void* kout;  // == k for the in-place modes
  int64_t q_bs, q_ts, k_bs, k_ts, o_bs, o_ts;
  int64_t tokens;  // batch * seq_len
  int seq_len;
  int row_elems;  // num_heads * head_dim
  float eps;
  const void* qw;
  const void* kw;
  const void* cos;  // TABLE
  const void* sin;
  const float* freqs;  // GRID / KVC: [2, D/2]
  int pairs_t, pairs_h;
  int grid_h, grid_w;
  int t0;
  float source_id;
  int cache_slots, slot_start;  // KVC
};

// Rotation coefficients of pair p of a token at grid position (t, h, w),
// following the table builders rope.py:46-51 (angle = pos * freq in fp32)
// and the source-id composition dit.py:931-932.
__device__ __forceinline__ void grid_pair_cs(const QKArgs& a, int P, int p, float t, float h,
                                             float w, float& c, float& s) {
  const float pos = p < a.pairs_t ? t : (p < a.pairs_t + a.pairs_h ? h : w);
  const float ang = pos * a.freqs[p];
  sincosf(ang, &s, &c);
  if (a.source_id != 0.f) {
    float sr, cr;
    sincosf(a.source_id * a.freqs[P + p], &sr, &cr);
    const float c2 = c * cr - s * sr;
    const float s2 = s * cr + c * sr;
    c = c2;
    s = s2;
  }
}

// SPLIT = 1: one wave does q and k of its token. SPLIT = 2: two waves per
// token, the even one q and the odd one k (twice the waves, for sequences
// too short to fill the chip; the rotation coefficients are then evaluated
// by both waves).
template <int HD, int G, int MODE, int SPLIT>
__global__ __launch_bounds__(kBlock) void qk_norm_rope_kernel(const QKArgs a) {
  constexpr int LPH = HD / 8;      // lanes per head
  constexpr int P = HD / 2;        // rotation pairs per head
  constexpr int K = P > 64 ? P / 64 : 1;  // pairs evaluated per lane in grid modes
  const int lane = threadIdx.x % kWave;
  const int64_t wid = static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) + threadIdx.x / kWave;
  const int64_t tok = wid / SPLIT;
  const bool do_q = SPLIT == 1 || (wid % SPLIT) == 0;
  const bool do_k = SPLIT == 1 || (wid % SPLIT) == 1;
  if (tok >= a.tokens) return;
  const int64_t b = tok / a.seq_len;
  const int n = static_cast<int>(tok - b * a.seq_len);
  const int pl = lane % LPH;  // this lane holds elements 8*pl .. 8*pl+7 of its head

  char* qrow = static_cast<char*>(a.q) + (b * a.q_bs + n * a.q_ts) * 2;
  const char* krow = static_cast<const char*>(a.k) + (b * a.k_bs + n * a.k_ts) * 2;

  const int groups = (a.row_elems + 511) / 512;
  // Rotation coefficients for pairs 4*pl .. 4*pl+3.
  float c[4], s[4];
  int64_t kdst_tok;  // destination token of the rotated k
  if constexpr (MODE == kTable) {
    const u32x2 cw = *reinterpret_cast<const u32x2*>(static_cast<const char*>(a.cos) +
                                                     (static_cast<int64_t>(n) * P + 4 * pl) * 2);
    const u32x2 sw = *reinterpret_cast<const u32x2*>(static_cast<const char*>(a.sin) +
                                                     (static_cast<int64_t>(n) * P + 4 * pl) * 2);
    c[0] = bf16_lo(cw.x); c[1] = bf16_hi(cw.x); c[2] = bf16_lo(cw.y); c[3] = bf16_hi(cw.y);
    s[0] = bf16_lo(sw.x); s[1] = bf16_hi(sw.x); s[2] = bf16_lo(sw.y); s[3] = bf16_hi(sw.y);
    kdst_tok = n;
  } else {
    const int frame_tokens = a.grid_h * a.grid_w;
    const int f = n / frame_tokens;
    const int rr = n - f * frame_tokens;
    const int hh = rr / a.grid_w;
    const int ww = rr - hh * a.grid_w;
    const float t = static_cast<float>(a.t0 + f);
    float mc[K], ms[K];
#pragma unroll
    for (int k = 0; k < K; ++k) grid_pair_cs(a, P, (lane * K + k) % P, t, hh, ww, mc[k], ms[k]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = 4 * pl + i;
      const int src = (p / K) << 2;  // ds_bpermute byte address of the owning lane
      c[i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, mc[i % K])));
      s[i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, ms[i % K])));
    }
    if constexpr (MODE == kKvCache)
      kdst_tok = static_cast<int64_t>((a.slot_start + f) % a.cache_slots) * frame_tokens + rr;
    else
      kdst_tok = n;
  }
  char* kdst = static_cast<char*>(a.kout) + (b * a.o_bs + kdst_tok * a.o_ts) * 2;

  const u32x4 wq = ld16(static_cast<const char*>(a.qw) + pl * 16);
  const u32x4 wk = ld16(static_cast<const char*>(a.kw) + pl * 16);

  for (int g0 = 0; g0 < groups; g0 += G) {
    u32x4 xq[G], xk[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int e = (g0 + g) * 512 + lane * 8;
      const bool ok = e < a.row_elems;
      xq[g] = (ok && do_q) ? ld16_nt(qrow + e * 2) : u32x4{0u, 0u, 0u, 0u};
      xk[g] = (ok && do_k) ? ld16_nt(krow + e * 2) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      if ((half == 0 && !do_q) || (half == 1 && !do_k)) continue;  // wave-uniform
      const u32x4& wv = half == 0 ? wq : wk;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int e = (g0 + g) * 512 + lane * 8;
        const u32x4& xv = half == 0 ? xq[g] : xk[g];
        float x[8];
        unpack<BF16>(xv, x);
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
        ss = allreduce<LPH, OpSum>(ss);
        const float r = rsqrtf(ss * (1.0f / HD) + a.eps);
        float o[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // e = x * (r * w) as fused_qknorm_rope_3d_kernel.cu:117, then the
          // pair rotation of :128-131.
          const float e0 = x[2 * i] * (r * elem<BF16>(wv, 2 * i));
          const float e1 = x[2 * i + 1] * (r * elem<BF16>(wv, 2 * i + 1));
          o[2 * i] = e0 * c[i] - e1 * s[i];
          o[2 * i + 1] = e0 * s[i] + e1 * c[i];
        }
        if (e < a.row_elems) {
          if (half == 0)
            st16_nt(qrow + e * 2, pack<BF16>(o));
          else
            st16_nt(kdst + e * 2, pack<BF16>(o));
        }
      }
    }
  }
}

// Waves per token. Two (q and k on separate waves) measured faster on MI355X
// at every BASELINE shape (3510 tokens: 19.0 -> 17.5 us; 10530 tokens:
// 46.4 -> 45.2 us): the extra waves hide HBM latency better than the saved
// rotation-coefficient work. JO_QK_SPLIT=1|2 overrides the choice (launch
// shape only; results are identical).
int qk_split(int64_t /*tokens*/) {
  const char* e = getenv("JO_QK_SPLIT");
  const int forced = e ? atoi(e) : 0;
  if (forced == 1 || forced == 2) return forced;
  return 2;
}

template <int MODE>
int launch_qk(const QKArgs& a, int head_dim, hipStream_t stream, const char* op) {
  const int groups = (a.row_elems + 511) / 512;
  const int split = qk_split(a.tokens);
  const dim3 grid(static_cast<unsigned>((a.tokens * split + 3) / 4));
  auto go = [&](auto hd, auto sp) {
    constexpr int HD = decltype(hd)::value;
    constexpr int S = decltype(sp)::value;
    if (groups <= 1)
      hipLaunchKernelGGL((qk_norm_rope_kernel<HD, 1, MODE, S>), grid, dim3(kBlock), 0, stream, a);
    else if (groups <= 2)
      hipLaunchKernelGGL((qk_norm_rope_kernel<HD, 2, MODE, S>), grid, dim3(kBlock), 0, stream, a);
    else if (groups <= 4)
      hipLaunchKernelGGL((qk_norm_rope_kernel<HD, 4, MODE, S>), grid, dim3(kBlock), 0, stream, a);
    else if (groups <= 6)
      hipLaunchKernelGGL((qk_norm_rope_kernel<HD, 6, MODE, S>), grid, dim3(kBlock), 0, stream, a);
    else
      hipLaunchKernelGGL((qk_norm_rope_kernel<HD, 8, MODE, S>), grid, dim3(kBlock), 0, stream, a);
  };
  auto go_hd = [&](auto hd) {
    if (split == 2)
      go(hd, std::integral_constant<int, 2>{});
    else
      go(hd, std::integral_constant<int, 1>{});
  };
  switch (head_dim) {
    case 64: go_hd(std::integral_constant<int, 64>{}); break;
    case 128: go_hd(std::integral_constant<int, 128>{}); break;
    default: go_hd(std::integral_constant<int, 256>{}); break;
  }
  return launch_status(op);
}

// Shared validation of the q/k geometry. Strides are in elements.
int check_qk(const char* op, const void* q, const void* k, int64_t batch, int64_t seq_len,
             int64_t num_heads, int64_t head_dim, int64_t q_bs, int64_t q_ts, int64_t k_bs,
             int64_t k_ts, const void* qw, const void* kw) {
  JO_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256,
             "Unsupported head_dim for %s: %lld", op, static_cast<long long>(head_dim));
  JO_REQUIRE(batch >= 0 && seq_len >= 0 && num_heads > 0, "%s: bad shape", op);
  JO_REQUIRE(seq_len <= INT32_MAX && num_heads * head_dim <= INT32_MAX, "%s: shape too large", op);
  JO_REQUIRE(q_ts >= num_heads * head_dim && k_ts >= num_heads * head_dim,
             "%s: token stride smaller than num_heads*head_dim", op);
  JO_REQUIRE(q_bs >= 0 && k_bs >= 0, "%s: negative batch stride", op);
  JO_REQUIRE(q_ts % 8 == 0 && k_ts % 8 == 0 && q_bs % 8 == 0 && k_bs % 8 == 0,
             "%s: strides must be multiples of 8 elements (16-byte rows)", op);
  if (batch * seq_len == 0) return JO_OK;
  JO_REQUIRE(q && k && qw && kw, "%s: null pointer", op);
  JO_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(qw, 16) && aligned(kw, 16),
             "%s: q, k and weights must be 16-byte aligned", op);
  return JO_OK;
}

int check_grid(const char* op, int64_t seq_len, int64_t head_dim, const float* freqs,
               int32_t pairs_t, int32_t pairs_h, int32_t grid_h, int32_t grid_w) {
  JO_REQUIRE(freqs != nullptr, "%s: null freqs", op);
  JO_REQUIRE(grid_h > 0 && grid_w > 0, "%s: grid_h and grid_w must be positive", op);
  JO_REQUIRE(seq_len % (static_cast<int64_t>(grid_h) * grid_w) == 0,
             "%s: seq_len %lld is not a whole number of %dx%d frames", op,
             static_cast<long long>(seq_len), grid_h, grid_w);
  JO_REQUIRE(pairs_t >= 0 && pairs_h >= 0 && pairs_t + pairs_h <= head_dim / 2,
             "%s: pairs_t + pairs_h must not exceed head_dim/2", op);
  return JO_OK;
}

}  // namespace
}  // namespace jo

using namespace jo;

extern "C" int jo_fused_qk_norm_rope_3d_paired(void* q, void* k, int64_t batch, int64_t seq_len,
                                               int64_t num_heads, int64_t head_dim,
                                               int64_t q_batch_stride, int64_t q_token_stride,
                                               int64_t k_batch_stride, int64_t k_token_stride,
                                               float eps, const void* q_weight,
                                               const void* k_weight, const void* cos,
                                               const void* sin, void* stream) {
  const char* op = "fused_qk_norm_rope_3d_paired";
  int st = check_qk(op, q, k, batch, seq_len, num_heads, head_dim, q_batch_stride,
                    q_token_stride, k_batch_stride, k_token_stride, q_weight, k_weight);
  if (st != JO_OK || batch * seq_len == 0) return st;
  JO_REQUIRE(cos && sin, "%s: null cos/sin", op);
  JO_REQUIRE(aligned(cos, 8) && aligned(sin, 8), "%s: cos/sin must be 8-byte aligned", op);
  QKArgs a{};
  a.q = q; a.k = k; a.kout = k;
  a.q_bs = q_batch_stride; a.q_ts = q_token_stride;
  a.k_bs = a.o_bs = k_batch_stride; a.k_ts = a.o_ts = k_token_stride;
  a.tokens = batch * seq_len; a.seq_len = static_cast<int>(seq_len);
  a.row_elems = static_cast<int>(num_heads * head_dim); a.eps = eps;
  a.qw = q_weight; a.kw = k_weight; a.cos = cos; a.sin = sin;
  return launch_qk<kTable>(a, static_cast<int>(head_dim), static_cast<hipStream_t>(stream), op);
}

extern "C" int jo_fused_qk_norm_rope_3d_grid(void* q, void* k, int64_t batch, int64_t seq_len,
                                             int64_t num_heads, int64_t head_dim,
                                             int64_t q_batch_stride, int64_t q_token_stride,
                                             int64_t k_batch_stride, int64_t k_token_stride,
                                             float eps, const void* q_weight,
                                             const void* k_weight, const float* freqs,
                                             int32_t pairs_t, int32_t pairs_h, int32_t grid_h,
                                             int32_t grid_w, int32_t t0, float source_id,
                                             void* stream) {
  const char* op = "fused_qk_norm_rope_3d_grid";
  int st = check_qk(op, q, k, batch, seq_len, num_heads, head_dim, q_batch_stride,
                    q_token_stride, k_batch_stride, k_token_stride, q_weight, k_weight);
  if (st != JO_OK) return st;
  st = check_grid(op, seq_len, head_dim, freqs, pairs_t, pairs_h, grid_h, grid_w);
  if (st != JO_OK || batch * seq_len == 0) return st;
  QKArgs a{};
  a.q = q; a.k = k; a.kout = k;
  a.q_bs = q_batch_stride; a.q_ts = q_token_stride;
  a.k_bs = a.o_bs = k_batch_stride; a.k_ts = a.o_ts = k_token_stride;
  a.tokens = batch * seq_len; a.seq_len = static_cast<int>(seq_len);
  a.row_elems = static_cast<int>(num_heads * head_dim); a.eps = eps;
  a.qw = q_weight; a.kw = k_weight;
  a.freqs = freqs; a.pairs_t = pairs_t; a.pairs_h = pairs_h;
  a.grid_h = grid_h; a.grid_w = grid_w; a.t0 = t0; a.source_id = source_id;
  return launch_qk<kGrid>(a, static_cast<int>(head_dim), static_cast<hipStream_t>(stream), op);
}

extern "C" int jo_fused_qk_norm_rope_3d_kvcache(
    void* q, const void* k, void* k_cache, int64_t batch, int64_t seq_len, int64_t num_heads,
    int64_t head_dim, int64_t q_batch_stride, int64_t q_token_stride, int64_t k_batch_stride,
    int64_t k_token_stride, int64_t cache_batch_stride, int64_t cache_token_stride,
    int64_t cache_slots, int64_t slot_start, float eps, const void* q_weight,
    const void* k_weight, const float* freqs, int32_t pairs_t, int32_t pairs_h, int32_t grid_h,
    int32_t grid_w, int32_t t0, float source_id, void* stream) {
  const char* op = "fused_qk_norm_rope_3d_kvcache";
  int st = check_qk(op, q, k, batch, seq_len, num_heads, head_dim, q_batch_stride,
                    q_token_stride, k_batch_stride, k_token_stride, q_weight, k_weight);
  if (st != JO_OK) return st;
  st = check_grid(op, seq_len, head_dim, freqs, pairs_t, pairs_h, grid_h, grid_w);
  if (st != JO_OK) return st;
  JO_REQUIRE(cache_slots > 0 && cache_slots <= INT32_MAX, "%s: cache_slots must be positive", op);
  JO_REQUIRE(slot_start >= 0 && slot_start < cache_slots, "%s: slot_start out of range", op);
  JO_REQUIRE(seq_len / (static_cast<int64_t>(grid_h) * grid_w) <= cache_slots,
             "%s: chunk has more frames than the cache has slots", op);
  JO_REQUIRE(cache_token_stride >= num_heads * head_dim && cache_token_stride % 8 == 0 &&
                 cache_batch_stride >= 0 && cache_batch_stride % 8 == 0,
             "%s: bad cache strides", op);
  if (batch * seq_len == 0) return JO_OK;
  JO_REQUIRE(k_cache && aligned(k_cache, 16), "%s: k_cache must be a 16-byte aligned pointer", op);
  QKArgs a{};
  a.q = q; a.k = k; a.kout = k_cache;
  a.q_bs = q_batch_stride; a.q_ts = q_token_stride;
  a.k_bs = k_batch_stride; a.k_ts = k_token_stride;
  a.o_bs = cache_batch_stride; a.o_ts = cache_token_stride;
  a.tokens = batch * seq_len; a.seq_len = static_cast<int>(seq_len);
  a.row_elems = static_cast<int>(num_heads * head_dim); a.eps = eps;
  a.qw = q_weight; a.kw = k_weight;
  a.freqs = freqs; a.pairs_t = pairs_t; a.pairs_h = pairs_h;
  a.grid_h = grid_h; a.grid_w = grid_w; a.t0 = t0; a.source_id = source_id;
  a.cache_slots = static_cast<int>(cache_slots); a.slot_start = static_cast<int>(slot_start);
  return launch_qk<kKvCache>(a, static_cast<int>(head_dim), static_cast<hipStream_t>(stream), op);
}
