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
#include <string.h>

#include "jo_device.hpp"
#include "jo_host.hpp"

namespace jo {
namespace {

constexpr int kMaxPairs = 128;  // head_dim 256
constexpr int kTable = 0;
constexpr int kGrid = 1;
constexpr int kKvCache = 2;

struct QKArgs {
  void* q;
  const void* k;
  void* kout;  // == k for the in-place modes
  int64_t q_bs, q_ts, k_bs, k_ts, o_bs, o_ts;
  void* kstage;  // STAGE: the pre-RoPE normalized k, [batch, seq_len, H*D] rows
  int64_t s_bs, s_ts;
  int64_t tokens;  // batch * seq_len
  int seq_len;
  int row_elems;  // num_heads * head_dim
  float eps;
  const void* qw;
  const void* kw;
  const void* cos;  // TABLE
  const void* sin;
  int pairs_t, pairs_h;
  int grid_h, grid_w;
  int t0;
  float source_id;
  int cache_slots, slot_start;  // KVC
  // The run-time divisors of the kernel's index arithmetic (set by launch_qk).
  FastDiv fd_seq, fd_row, fd_gw, fd_frame, fd_slots;
  // GRID / KVC: [2, D/2] axis and source-id frequencies, carried by value in
  // the kernel arguments (lanes index them with their own pair numbers, which
  // compiles to loads from the kernel-argument segment). No device copy, so a
  // grid launch needs no setup and captures into a HIP graph as it is.
  float freqs[2 * kMaxPairs];
};

// sin and cos of an fp32 angle a. For |a| <= 65536: Cody-Waite reduction by
// pi/2 with pi/2 split into three fp32 parts (the first FMA step is exact for
// |a| >= 1 because k*P1 and a are multiples of 2^-23 there), then the Taylor
// series of sin (to r^9) and cos (to r^10) on [-pi/4, pi/4], whose truncation
// is below 2e-9. The absolute error is a few 2^-25, far inside the bf16 output
// rounding. Larger or non-finite angles take sincosf.
__device__ __forceinline__ void sincos_reduced(float a, float& s, float& c) {
  if (__builtin_expect(!(fabsf(a) <= 65536.f), 0)) {
    sincosf(a, &s, &c);
    return;
  }
  constexpr float kTwoOverPi = 0x1.45f306p-1f;
  constexpr float kP1 = 0x1.921fb6p+0f;   // fp32(pi/2)
  constexpr float kP2 = -0x1.777a5cp-25f;  // fp32(pi/2 - P1)
  constexpr float kP3 = -0x1.ee59dap-50f;  // fp32(pi/2 - P1 - P2)
  const float k = __builtin_rintf(a * kTwoOverPi);
  float r = __builtin_fmaf(-k, kP1, a);
  r = __builtin_fmaf(-k, kP2, r);
  r = __builtin_fmaf(-k, kP3, r);
  const float z = r * r;
  float ps = __builtin_fmaf(z, 1.f / 362880.f, -1.f / 5040.f);
  ps = __builtin_fmaf(z, ps, 1.f / 120.f);
  ps = __builtin_fmaf(z, ps, -1.f / 6.f);
  const float sr = __builtin_fmaf(r * z, ps, r);
  float pc = __builtin_fmaf(z, -1.f / 3628800.f, 1.f / 40320.f);
  pc = __builtin_fmaf(z, pc, -1.f / 720.f);
  pc = __builtin_fmaf(z, pc, 1.f / 24.f);
  pc = __builtin_fmaf(z, pc, -0.5f);
  const float cr = __builtin_fmaf(z, pc, 1.f);
  // Quadrant q = k mod 4: (sin, cos) = (S, C), (C, -S), (-S, -C), (-C, S).
  const int q = static_cast<int>(k) & 3;
  const float sv = (q & 1) ? cr : sr;
  const float cv = (q & 1) ? sr : cr;
  s = (q & 2) ? -sv : sv;
  c = ((q + 1) & 2) ? -cv : cv;
}

// Rotation coefficients of a pair at grid position pos on its axis, from its
// axis frequency f and source-id frequency fr, following the table builders
// rope.py:46-51 (angle = pos * freq in fp32) and the source-id composition
// dit.py:931-932 (angle addition, skipped when the source id is 0).
__device__ __forceinline__ void grid_pair_cs(float pos, float f, float source_id, float fr,
                                             float& c, float& s) {
  const float ang = pos * f;
  sincos_reduced(ang, s, c);
  if (source_id != 0.f) {
    float sr, cr;
    sincos_reduced(source_id * fr, sr, cr);
    const float c2 = c * cr - s * sr;
    const float s2 = s * cr + c * sr;
    c = c2;
    s = s2;
  }
}

// SPLIT = 1: one wave does q and k of its token. SPLIT = 2: two waves per
// token, one for q and one for k. SPLIT = 4, 6, 8: that many waves per token,
// q and k each split into SPLIT / 2 parts of their head groups. The rotation
// coefficients are evaluated by every wave.
//
// Issue order matters: the memory counter retires loads in order, so the
// small parameter loads (rotation table or frequencies, weights) go out
// first, then the row loads, and only then is anything waited on — the
// sincos then overlaps the row loads instead of delaying their issue.
// The pre-RoPE K row of rmsnorm_qk_bf16 (rmsnorm.cu:53-60 as the rmsnorm op
// evaluates it: ms = ss / D and r = 1 / sqrt(ms + eps) as separate IEEE
// operations, then (x * r) * w): the same per-lane sum and DPP reduction as
// the QK normalization, so the row is bit-identical to that op's.
__device__ __forceinline__ float kernel_rms_rstd(float ss, float n, float eps) {
#pragma clang fp contract(off)
  const float ms = ss / n;
  return 1.0f / sqrtf(ms + eps);
}

// STAGE: k waves also write the pre-RoPE normalized k to a.kstage, so that a
// forward that caches K before RoPE (dit.py:360-370) reads K once.
template <int HD, int G, int MODE, int SPLIT, bool STAGE = false>
__global__ __launch_bounds__(kBlock) void qk_norm_rope_kernel(const QKArgs a) {
  constexpr int LPH = HD / 8;      // lanes per head
  constexpr int P = HD / 2;        // rotation pairs per head
  constexpr int K = P > 64 ? P / 64 : 1;  // pairs evaluated per lane in grid modes
  constexpr int NS = SPLIT == 1 ? 2 : 1;  // tensor streams per wave (q and k, or one)
  const int lane = threadIdx.x % kWave;
  // The wave index through readfirstlane: the token and part arithmetic below
  // (divisions included) is then scalar instead of repeated in every lane
  // (858 instead of 1048 vector instructions; C0 16.0 -> 15.85 us, every QK
  // shape 0.6-1.5% faster).
  const int64_t wid = static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) +
                      __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  // Waves of q come first, then waves of k (SPLIT >= 2): a workgroup streams
  // consecutive rows of one tensor (measured against interleaving q and k
  // waves per token: [1, 3510, 24, 128] 16.38 -> 16.15 us, C3 43.9 -> 43.4 us,
  // table mode at [1, 3120, 32, 128] 19.0 -> 18.7 us). part: bit 0 = k, bit 1
  // and up = the part of the head groups (SPLIT >= 4).
  // Token and wave indices fit 32 bits (the launch check bounds the tokens),
  // so the index arithmetic is 32-bit, with the run-time divisions by
  // multiply-high (FastDiv): [1, 3510, 24, 128] grid 15.3-15.5 -> 15.1 us.
  int64_t tok;
  int part;
  if constexpr (SPLIT == 1) {
    tok = wid;
    part = 0;
  } else {
    const int64_t per_tensor = a.tokens * (SPLIT / 2);
    const bool on_k = wid >= per_tensor;
    const uint32_t w = static_cast<uint32_t>(on_k ? wid - per_tensor : wid);
    tok = w / (SPLIT / 2);
    part = (on_k ? 1 : 0) | (static_cast<int>(w % (SPLIT / 2)) << 1);
  }
  if (tok >= a.tokens) return;
  const uint32_t b32 = fdiv(static_cast<uint32_t>(tok), a.fd_seq);
  const int64_t b = b32;
  const int n = static_cast<int>(static_cast<uint32_t>(tok) - b32 * static_cast<uint32_t>(a.seq_len));
  const int pl = lane % LPH;  // this lane holds elements 8*pl .. 8*pl+7 of its head

  // Destination token of the rotated k (grid modes: frame ring slot).
  int64_t kdst_tok = n;
  int f = 0, rr = 0;
  if constexpr (MODE != kTable) {
    const int frame_tokens = a.grid_h * a.grid_w;
    f = static_cast<int>(fdiv(static_cast<uint32_t>(n), a.fd_frame));
    rr = n - f * frame_tokens;
    if constexpr (MODE == kKvCache) {
      const uint32_t slot = static_cast<uint32_t>(a.slot_start + f);
      const uint32_t ring = slot - fdiv(slot, a.fd_slots) * static_cast<uint32_t>(a.cache_slots);
      kdst_tok = static_cast<int64_t>(ring) * frame_tokens + rr;
    }
  }
  char* qrow = static_cast<char*>(a.q) + (b * a.q_bs + n * a.q_ts) * 2;
  const char* krow = static_cast<const char*>(a.k) + (b * a.k_bs + n * a.k_ts) * 2;
  char* kdst = static_cast<char*>(a.kout) + (b * a.o_bs + kdst_tok * a.o_ts) * 2;
  char* kstg = STAGE ? static_cast<char*>(a.kstage) + (b * a.s_bs + n * a.s_ts) * 2 : nullptr;
  const char* src[NS];
  char* dst[NS];
  const char* wsrc[NS];
  if constexpr (NS == 2) {
    src[0] = qrow; dst[0] = qrow; wsrc[0] = static_cast<const char*>(a.qw);
    src[1] = krow; dst[1] = kdst; wsrc[1] = static_cast<const char*>(a.kw);
  } else {
    const bool is_k = (part & 1) != 0;  // wave-uniform
    src[0] = is_k ? krow : qrow;
    dst[0] = is_k ? kdst : qrow;
    wsrc[0] = static_cast<const char*>(is_k ? a.kw : a.qw);
  }
  // Head groups (512 elements each) this wave handles: all of its tensor's,
  // or one of SPLIT / 2 equal parts of them.
  constexpr int kParts = SPLIT >= 4 ? SPLIT / 2 : 1;
  const int all_groups = (a.row_elems + 511) / 512;
  const int part_groups = (all_groups + kParts - 1) / kParts;
  const int gbeg = (part >> 1) * part_groups;
  const int groups = min(all_groups, gbeg + part_groups);

  // 1. Parameter loads: rotation table row or frequencies, weights.
  u32x2 cw, sw;
  float fq[K], fr[K];
  if constexpr (MODE == kTable) {
    const int64_t off = (static_cast<int64_t>(n) * P + 4 * pl) * 2;
    cw = *reinterpret_cast<const u32x2*>(static_cast<const char*>(a.cos) + off);
    sw = *reinterpret_cast<const u32x2*>(static_cast<const char*>(a.sin) + off);
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int p = (lane * K + k) % P;
      fq[k] = a.freqs[p];
      fr[k] = a.source_id != 0.f ? a.freqs[P + p] : 0.f;
    }
  }
  u32x4 wv[NS];
#pragma unroll
  for (int t = 0; t < NS; ++t) wv[t] = ld16(wsrc[t] + pl * 16);

  // 2. Row loads of the first batch of head groups. Loads are never
  // predicated (a predicated load's join forces an early wait): a chunk
  // outside this wave's range reads a valid chunk of the same row instead.
  // Its lanes form whole heads (a chunk holds 512/HD complete heads), so
  // their values stay within heads that are never stored.
  const uint32_t l8 = static_cast<uint32_t>(lane * 8);
  const int e_safe = static_cast<int>(l8 - fdiv(l8, a.fd_row) * static_cast<uint32_t>(a.row_elems));
  u32x4 x[NS][G];
  auto load_batch = [&](int g0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int e = (g0 + g) * 512 + lane * 8;
      const bool ok = (g0 + g) < groups && e < a.row_elems;  // own range, inside the row
      const int el = ok ? e : e_safe;
#pragma unroll
      for (int t = 0; t < NS; ++t) x[t][g] = ld16_nt(src[t] + el * 2);
    }
  };
  load_batch(gbeg);
  // Keep every row load of the first batch ahead of the angle math below,
  // which waits for the parameter loads.
  __builtin_amdgcn_sched_barrier(0);

  // 3. Rotation coefficients for pairs 4*pl .. 4*pl+3 (overlaps the row loads).
  float c[4], s[4];
  if constexpr (MODE == kTable) {
    c[0] = bf16_lo(cw.x); c[1] = bf16_hi(cw.x); c[2] = bf16_lo(cw.y); c[3] = bf16_hi(cw.y);
    s[0] = bf16_lo(sw.x); s[1] = bf16_hi(sw.x); s[2] = bf16_lo(sw.y); s[3] = bf16_hi(sw.y);
  } else {
    const int hh = static_cast<int>(fdiv(static_cast<uint32_t>(rr), a.fd_gw));
    const int ww = rr - hh * a.grid_w;
    const float tpos = static_cast<float>(a.t0 + f);
    float mc[K], ms[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int p = (lane * K + k) % P;
      const float pos = p < a.pairs_t ? tpos
                      : (p < a.pairs_t + a.pairs_h ? static_cast<float>(hh) : static_cast<float>(ww));
      grid_pair_cs(pos, fq[k], a.source_id, fr[k], mc[k], ms[k]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = 4 * pl + i;
      const int owner = (p / K) << 2;  // ds_bpermute byte address of the owning lane
      c[i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(owner, __builtin_bit_cast(int, mc[i % K])));
      s[i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(owner, __builtin_bit_cast(int, ms[i % K])));
    }
  }

  // 4. Normalize, rotate, store; further batches only when H*D > G*512.
  // Waves do not meet: a workgroup barrier here (so that a workgroup's row
  // stores leave together) measured slower with the current loads
  // ([1, 1560, 32, 128] tables 10.20 -> 10.32 us, [1, 3120, 32, 128] 17.57 ->
  // 17.67 us, C3 41.30 -> 41.43 us).
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  for (int g0 = gbeg; g0 < groups; g0 += G) {
    if (g0 != gbeg) load_batch(g0);
#pragma unroll
    for (int t = 0; t < NS; ++t) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int e = (g0 + g) * 512 + lane * 8;
        float xv[8];
        unpack<BF16>(x[t][g], xv);
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) ss += xv[j] * xv[j];
        ss = allreduce<LPH, OpSum>(ss);
        const float r = rsqrtf(ss * (1.0f / HD) + a.eps);
        if constexpr (STAGE) {
          const bool on_k = NS == 2 ? t == 1 : (part & 1) != 0;  // wave-uniform
          if (on_k && (g0 + g) < groups && e < a.row_elems) {
            const float rs = kernel_rms_rstd(ss, static_cast<float>(HD), a.eps);
            float so[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) so[j] = (xv[j] * rs) * elem<BF16>(wv[t], j);
            if constexpr (MODE == kKvCache)
              st16_nt(kstg + e * 2, pack<BF16>(so));
            else
              st16_sys_nt(kstg, e * 2, pack<BF16>(so));
          }
        }
        float o[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // e = x * (r * w) as fused_qknorm_rope_3d_kernel.cu:117, then the
          // pair rotation of :128-131.
          const float e0 = xv[2 * i] * (r * elem<BF16>(wv[t], 2 * i));
          const float e1 = xv[2 * i + 1] * (r * elem<BF16>(wv[t], 2 * i + 1));
          o[2 * i] = e0 * c[i] - e1 * s[i];
          o[2 * i + 1] = e0 * s[i] + e1 * c[i];
        }
        if ((g0 + g) < groups && e < a.row_elems) {
          // dst[t] is the wave's row base (wave-uniform: from the wave index).
          if constexpr (MODE == kKvCache)
            st16_nt(dst[t] + e * 2, pack<BF16>(o));
          else
            st16_sys_nt(dst[t], e * 2, pack<BF16>(o));
        }
      }
    }
  }
}

// Waves per token. Two (q and k on separate waves) measured faster on MI355X
// than one at every benchmark shape (3510 tokens: 19.0 -> 17.5 us; 10530
// tokens: 46.4 -> 45.2 us): the extra waves hide HBM latency better than the
// saved rotation-coefficient work. Four (each of q and k split into halves of
// its head groups) is faster again, at 3510 tokens (17.3 -> 17.0 us) and, once
// the waves of q precede those of k, at 10530 (C3 42.8 -> 41.7 us). Eight
// (quarters) helps further on small grids whose groups divide evenly into
// quarters of two or more ([1, 3120, 32, 128] tables 18.6 -> 18.0 us,
// [1, 1560, 32, 128] 11.3 -> 10.4 us); with 24 heads (six groups) a quarter
// would be 1.5 groups and it costs ([1, 3510, 24, 128] 16.1 -> 18.5 us); six
// (thirds of two groups each) is faster there once the in-place rows are
// stored through ([1, 3510, 24, 128] grid 15.63 -> 15.35 us; with the plain
// nontemporal stores it measured level with four) but not at 10530 tokens
// (C3 41.65 -> 41.84 us); twelve (one head group per wave) measured no better
// than four ([1, 3510, 24, 128] 16.4 -> 16.3 us, C3 42.6 -> 43.0 us), sixteen
// at 32 heads level with eight. The JO_KNOB_QK_SPLIT override (1, 2, 4, 6, 8)
// forces the choice (launch shape only; results are identical).
int qk_split(int64_t tokens, int all_groups) {
  const int forced = launch_knob(JO_KNOB_QK_SPLIT);
  if (forced == 1 || forced == 2) return forced;
  if (forced == 8 && all_groups >= 4) return 8;
  if (forced == 6 && all_groups >= 3) return 6;
  if (forced == 4 || forced == 6 || forced == 8) return all_groups >= 2 ? 4 : 2;
  if (all_groups < 2) return 2;
  if (tokens < 8192 && all_groups >= 8 && all_groups % 4 == 0) return 8;
  if (tokens < 8192 && all_groups >= 6 && all_groups % 3 == 0) return 6;
  return 4;
}

template <int MODE, bool STAGE = false>
int launch_qk(const QKArgs& args, int head_dim, hipStream_t stream, const char* op) {
  QKArgs a = args;
  a.fd_seq = make_fastdiv(static_cast<uint32_t>(a.seq_len));
  a.fd_row = make_fastdiv(static_cast<uint32_t>(a.row_elems));
  if (MODE != kTable) {
    a.fd_gw = make_fastdiv(static_cast<uint32_t>(a.grid_w));
    a.fd_frame = make_fastdiv(static_cast<uint32_t>(a.grid_h) * static_cast<uint32_t>(a.grid_w));
  }
  if (MODE == kKvCache) a.fd_slots = make_fastdiv(static_cast<uint32_t>(a.cache_slots));
  const int all_groups = (a.row_elems + 511) / 512;
  const int split = qk_split(a.tokens, all_groups);
  const int parts = split >= 4 ? split / 2 : 1;
  const int groups = (all_groups + parts - 1) / parts;  // per wave
  const dim3 grid(static_cast<unsigned>((a.tokens * split + 3) / 4));
  auto go = [&](auto hd, auto sp) {
    constexpr int HD = decltype(hd)::value;
    constexpr int S = decltype(sp)::value;
    if (groups <= 1)
      hipLaunchKernelGGL((qk_norm_rope_kernel<HD, 1, MODE, S, STAGE>), grid, dim3(kBlock), 0, stream, a);
    else if (groups <= 2)
      hipLaunchKernelGGL((qk_norm_rope_kernel<HD, 2, MODE, S, STAGE>), grid, dim3(kBlock), 0, stream, a);
    else if (groups <= 3)
      hipLaunchKernelGGL((qk_norm_rope_kernel<HD, 3, MODE, S, STAGE>), grid, dim3(kBlock), 0, stream, a);
    else if (groups <= 4)
      hipLaunchKernelGGL((qk_norm_rope_kernel<HD, 4, MODE, S, STAGE>), grid, dim3(kBlock), 0, stream, a);
    else if (groups <= 6)
      hipLaunchKernelGGL((qk_norm_rope_kernel<HD, 6, MODE, S, STAGE>), grid, dim3(kBlock), 0, stream, a);
    else
      hipLaunchKernelGGL((qk_norm_rope_kernel<HD, 8, MODE, S, STAGE>), grid, dim3(kBlock), 0, stream, a);
  };
  auto go_hd = [&](auto hd) {
    if (split == 8)
      go(hd, std::integral_constant<int, 8>{});
    else if (split == 6)
      go(hd, std::integral_constant<int, 6>{});
    else if (split == 4)
      go(hd, std::integral_constant<int, 4>{});
    else if (split == 2)
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
  // Up to 8 waves of 64 lanes per token: the launch's work-item count must
  // stay below 2^32.
  JO_REQUIRE(seq_len <= INT32_MAX && num_heads * head_dim <= INT32_MAX &&
                 batch * seq_len <= int64_t{UINT32_MAX} / (8 * kWave),
             "%s: shape too large (batch * seq_len must not exceed %lld tokens)", op,
             static_cast<long long>(int64_t{UINT32_MAX} / (8 * kWave)));
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
  JO_REQUIRE(head_dim / 2 <= kMaxPairs, "%s: head_dim too large for the frequency table", op);
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

namespace jo {
namespace {

// The pre-RoPE K stage of the *_kstage entry points: [batch, seq_len, H*D]
// rows with the given strides (elements), 16-byte aligned.
int check_stage(const char* op, const void* k_stage, int64_t s_bs, int64_t s_ts,
                int64_t num_heads, int64_t head_dim) {
  JO_REQUIRE(s_ts >= num_heads * head_dim && s_bs >= 0 && s_ts % 8 == 0 && s_bs % 8 == 0,
             "%s: bad k_stage strides", op);
  JO_REQUIRE(k_stage && aligned(k_stage, 16), "%s: k_stage must be a 16-byte aligned pointer",
             op);
  return JO_OK;
}

int qk_paired(const char* op, void* q, void* k, void* k_stage, int64_t batch, int64_t seq_len,
              int64_t num_heads, int64_t head_dim, int64_t q_bs, int64_t q_ts, int64_t k_bs,
              int64_t k_ts, int64_t s_bs, int64_t s_ts, float eps, const void* q_weight,
              const void* k_weight, const void* cos, const void* sin, void* stream,
              bool stage) {
  int st = check_qk(op, q, k, batch, seq_len, num_heads, head_dim, q_bs, q_ts, k_bs, k_ts,
                    q_weight, k_weight);
  if (st != JO_OK || batch * seq_len == 0) return st;
  JO_REQUIRE(cos && sin, "%s: null cos/sin", op);
  JO_REQUIRE(aligned(cos, 8) && aligned(sin, 8), "%s: cos/sin must be 8-byte aligned", op);
  if (stage && (st = check_stage(op, k_stage, s_bs, s_ts, num_heads, head_dim)) != JO_OK)
    return st;
  QKArgs a{};
  a.q = q; a.k = k; a.kout = k;
  a.q_bs = q_bs; a.q_ts = q_ts;
  a.k_bs = a.o_bs = k_bs; a.k_ts = a.o_ts = k_ts;
  a.kstage = k_stage; a.s_bs = s_bs; a.s_ts = s_ts;
  a.tokens = batch * seq_len; a.seq_len = static_cast<int>(seq_len);
  a.row_elems = static_cast<int>(num_heads * head_dim); a.eps = eps;
  a.qw = q_weight; a.kw = k_weight; a.cos = cos; a.sin = sin;
  hipStream_t hs = static_cast<hipStream_t>(stream);
  return stage ? launch_qk<kTable, true>(a, static_cast<int>(head_dim), hs, op)
               : launch_qk<kTable>(a, static_cast<int>(head_dim), hs, op);
}

int qk_grid(const char* op, void* q, void* k, void* k_stage, int64_t batch, int64_t seq_len,
            int64_t num_heads, int64_t head_dim, int64_t q_bs, int64_t q_ts, int64_t k_bs,
            int64_t k_ts, int64_t s_bs, int64_t s_ts, float eps, const void* q_weight,
            const void* k_weight, const float* freqs, int32_t pairs_t, int32_t pairs_h,
            int32_t grid_h, int32_t grid_w, int32_t t0, float source_id, void* stream,
            bool stage) {
  int st = check_qk(op, q, k, batch, seq_len, num_heads, head_dim, q_bs, q_ts, k_bs, k_ts,
                    q_weight, k_weight);
  if (st != JO_OK) return st;
  st = check_grid(op, seq_len, head_dim, freqs, pairs_t, pairs_h, grid_h, grid_w);
  if (st != JO_OK || batch * seq_len == 0) return st;
  if (stage && (st = check_stage(op, k_stage, s_bs, s_ts, num_heads, head_dim)) != JO_OK)
    return st;
  QKArgs a{};
  a.q = q; a.k = k; a.kout = k;
  a.q_bs = q_bs; a.q_ts = q_ts;
  a.k_bs = a.o_bs = k_bs; a.k_ts = a.o_ts = k_ts;
  a.kstage = k_stage; a.s_bs = s_bs; a.s_ts = s_ts;
  a.tokens = batch * seq_len; a.seq_len = static_cast<int>(seq_len);
  a.row_elems = static_cast<int>(num_heads * head_dim); a.eps = eps;
  a.qw = q_weight; a.kw = k_weight;
  memcpy(a.freqs, freqs, sizeof(float) * head_dim);
  a.pairs_t = pairs_t; a.pairs_h = pairs_h;
  a.grid_h = grid_h; a.grid_w = grid_w; a.t0 = t0; a.source_id = source_id;
  hipStream_t hs = static_cast<hipStream_t>(stream);
  return stage ? launch_qk<kGrid, true>(a, static_cast<int>(head_dim), hs, op)
               : launch_qk<kGrid>(a, static_cast<int>(head_dim), hs, op);
}

}  // namespace
}  // namespace jo

extern "C" int jo_fused_qk_norm_rope_3d_paired(void* q, void* k, int64_t batch, int64_t seq_len,
                                               int64_t num_heads, int64_t head_dim,
                                               int64_t q_batch_stride, int64_t q_token_stride,
                                               int64_t k_batch_stride, int64_t k_token_stride,
                                               float eps, const void* q_weight,
                                               const void* k_weight, const void* cos,
                                               const void* sin, void* stream) {
  return qk_paired("fused_qk_norm_rope_3d_paired", q, k, nullptr, batch, seq_len, num_heads,
                   head_dim, q_batch_stride, q_token_stride, k_batch_stride, k_token_stride, 0, 0,
                   eps, q_weight, k_weight, cos, sin, stream, false);
}

extern "C" int jo_fused_qk_norm_rope_3d_paired_kstage(
    void* q, void* k, void* k_stage, int64_t batch, int64_t seq_len, int64_t num_heads,
    int64_t head_dim, int64_t q_batch_stride, int64_t q_token_stride, int64_t k_batch_stride,
    int64_t k_token_stride, int64_t stage_batch_stride, int64_t stage_token_stride, float eps,
    const void* q_weight, const void* k_weight, const void* cos, const void* sin, void* stream) {
  return qk_paired("fused_qk_norm_rope_3d_paired_kstage", q, k, k_stage, batch, seq_len,
                   num_heads, head_dim, q_batch_stride, q_token_stride, k_batch_stride,
                   k_token_stride, stage_batch_stride, stage_token_stride, eps, q_weight,
                   k_weight, cos, sin, stream, true);
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
  return qk_grid("fused_qk_norm_rope_3d_grid", q, k, nullptr, batch, seq_len, num_heads,
                 head_dim, q_batch_stride, q_token_stride, k_batch_stride, k_token_stride, 0, 0,
                 eps, q_weight, k_weight, freqs, pairs_t, pairs_h, grid_h, grid_w, t0, source_id,
                 stream, false);
}

extern "C" int jo_fused_qk_norm_rope_3d_grid_kstage(
    void* q, void* k, void* k_stage, int64_t batch, int64_t seq_len, int64_t num_heads,
    int64_t head_dim, int64_t q_batch_stride, int64_t q_token_stride, int64_t k_batch_stride,
    int64_t k_token_stride, int64_t stage_batch_stride, int64_t stage_token_stride, float eps,
    const void* q_weight, const void* k_weight, const float* freqs, int32_t pairs_t,
    int32_t pairs_h, int32_t grid_h, int32_t grid_w, int32_t t0, float source_id, void* stream) {
  return qk_grid("fused_qk_norm_rope_3d_grid_kstage", q, k, k_stage, batch, seq_len, num_heads,
                 head_dim, q_batch_stride, q_token_stride, k_batch_stride, k_token_stride,
                 stage_batch_stride, stage_token_stride, eps, q_weight, k_weight, freqs, pairs_t,
                 pairs_h, grid_h, grid_w, t0, source_id, stream, true);
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
  memcpy(a.freqs, freqs, sizeof(float) * head_dim);
  a.pairs_t = pairs_t; a.pairs_h = pairs_h;
  a.grid_h = grid_h; a.grid_w = grid_w; a.t0 = t0; a.source_id = source_id;
  a.cache_slots = static_cast<int>(cache_slots); a.slot_start = static_cast<int>(slot_start);
  return launch_qk<kKvCache>(a, static_cast<int>(head_dim), static_cast<hipStream_t>(stream), op);
}
