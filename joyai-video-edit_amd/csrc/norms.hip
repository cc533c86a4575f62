// LayerNorm / RMSNorm with AdaLN modulation, standalone RMSNorm, the fused
// (gated) residual add + LayerNorm + AdaLN, and both with a per-token FP8
// epilogue in place of the bf16/fp16 output.
//
// Row kernels: LPR lanes per row, CH 16-byte chunks per lane held in
// registers, so x (and the residual) are read from HBM once and y (and the
// residual) written once. LayerNorm statistics are two-pass from registers
// (mean, then the sum of squared deviations), like the reference. Row sums
// reduce with DPP / swizzle / readlane, through LDS only across waves.
#include "jo_device.hpp"
#include "jo_host.hpp"

namespace jo {
namespace {

struct NormArgs {
  const void* x;
  int64_t xs;
  void* res;  // residual (add kernel only), updated in place
  int64_t rs;
  const void* gate;  // optional gate of the residual update
  int64_t gs;
  const void* gamma;  // optional, [N]
  const void* beta;   // optional, [N]; applied only with gamma
  const void* scale;
  int64_t scs;  // 0 = one row for all rows
  const void* shift;
  int64_t shs;
  void* y;
  int64_t ys;
  int64_t M;
  int N;
  float eps;
  uint8_t* q = nullptr;  // FP8 epilogue: e4m3fn rows (stride qs) and fp32 scales [M]
  int64_t qs = 0;
  float* s = nullptr;
  uint32_t mod_rows = 1;  // rows that share one gate / scale / shift row
};

// Row of the gate / scale / shift tensors that serves row `row` of x: the
// same row, or one row per mod_rows consecutive rows (one per sample of a
// [B, L, N] batch). M < 2^32 (checked on the host), so 32-bit division.
__device__ __forceinline__ int64_t mod_row(const NormArgs& a, int64_t row) {
  return a.mod_rows == 1 ? row
                         : static_cast<int64_t>(static_cast<uint32_t>(row) / a.mod_rows);
}

constexpr int kLayer = JO_NORM_LAYER;
constexpr int kRms = JO_NORM_RMS;

// A chunk of 1.0 values of the element type.
template <class Tag>
__device__ __forceinline__ u32x4 ones_chunk() {
  constexpr uint32_t w = Tag::kBytes == 4 ? 0x3F800000u
                         : std::is_same_v<Tag, BF16> ? 0x3F803F80u : 0x3C003C00u;
  return u32x4{w, w, w, w};
}

// residual + x * gate as torch.addcmul evaluates it: the product and the sum
// are two separately rounded fp32 operations (no fused multiply-add).
__device__ __forceinline__ float residual_update(float res, float x, float gate, bool gated) {
#pragma clang fp contract(off)
  return gated ? res + x * gate : res + x;
}

// Chunk e of the row that starts row_elems elements into base. ld_chunk is
// cached (reused data: gamma, beta, a broadcast row); ld_row / st_row stream
// row data that is touched once.
template <class Tag>
__device__ __forceinline__ u32x4 ld_chunk(const void* base, int64_t row_elems, int e) {
  return ld16(byte_off(base, (row_elems + e) * Tag::kBytes));
}
template <class Tag>
__device__ __forceinline__ u32x4 ld_row(const void* base, int64_t row_elems, int e) {
  return ld16_nt(byte_off(base, (row_elems + e) * Tag::kBytes));
}
template <class Tag>
__device__ __forceinline__ void st_row(void* base, int64_t row_elems, int e, const u32x4& v) {
  st16_nt(byte_off(base, (row_elems + e) * Tag::kBytes), v);
}
// A modulation row: streamed when every row has its own (stride != 0),
// cached when one row is broadcast to all rows (stride == 0).
template <class Tag>
__device__ __forceinline__ u32x4 ld_mod(const void* base, int64_t stride, int64_t row, int e) {
  return stride ? ld_row<Tag>(base, row * stride, e) : ld_chunk<Tag>(base, 0, e);
}

// ---------------------------------------------------------------------------
// y = Norm(v)(gamma, beta) * (1 + scale) + shift, follows
// fused_norm_scale_shift.cu:88-142. With ADD, v is first formed as
// round(res + x * gate) and written back to res (sgl_fused_ops.py:114-117).
// With QNT, y is rounded to the row dtype as the unfused op would store it,
// and that row is quantized per token by the rule of per_token_quant_fp8.cu:
// 56-82 (the input Fp8Linear.forward quantizes, fp8_linear.py:138-169)
// instead of being written.
// ---------------------------------------------------------------------------
//
// EXACT (N == LPR * CH * V, taken with BCAST): every lane's chunks lie inside
// the row, so the per-lane bounds tests go; a row past M (in the last
// workgroup) reads row M - 1 and stores nothing. With rows of one or more
// whole waves the row index is made wave-uniform, so each row's base address
// is scalar and the lanes add 32-bit offsets to it.
template <class Tag, int LPR, int CH, int NT, bool ADD, bool QNT, bool BCAST = false,
          bool EARLY = false, bool EXACT = false>
__global__ __launch_bounds__(kBlock) void norm_mod_kernel(const NormArgs a) {
  constexpr int V = Tag::kVec;
  constexpr int RPB = kBlock / LPR;
  static_assert(!QNT || V == 8, "the FP8 epilogue takes 16-bit rows");
  __shared__ float red_a[kBlock / kWave];
  __shared__ float red_b[kBlock / kWave];
  __shared__ float red_c[kBlock / kWave];
  __shared__ float red_d[kBlock / kWave];
  const int lane = threadIdx.x % LPR;
  const int rib = (EXACT && LPR >= kWave)
                      ? __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / LPR))
                      : static_cast<int>(threadIdx.x / LPR);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + rib;
  const bool row_ok = row < a.M;
  const int64_t lrow = (EXACT && !row_ok) ? a.M - 1 : row;  // the row this thread reads
  const int64_t mrow = mod_row(a, lrow);
  const int N = a.N;
  // EXACT: the rows' base addresses, and chunk e of a row at base + e * bytes.
  const void* xrow = byte_off(a.x, lrow * a.xs * Tag::kBytes);
  void* rrow = ADD ? byte_off(a.res, lrow * a.rs * Tag::kBytes) : nullptr;
  auto ld_x = [&](int e) {
    return EXACT ? ld16_nt(byte_off(xrow, e * Tag::kBytes)) : ld_row<Tag>(a.x, row * a.xs, e);
  };
  auto ld_res = [&](int e) {
    return EXACT ? ld16_nt(byte_off(rrow, e * Tag::kBytes)) : ld_row<Tag>(a.res, row * a.rs, e);
  };
  auto st_res = [&](int e, const u32x4& v) {
    if constexpr (EXACT)
      st16_nt(byte_off(rrow, e * Tag::kBytes), v);
    else
      st_row<Tag>(a.res, row * a.rs, e, v);
  };

  // BCAST: one scale row and one shift row for all rows (stride 0, no
  // gamma), fetched before the row itself so that their (cached) latency is
  // spent while the row is in flight rather than after the reductions
  // (residual + LN + AdaLN at [10530, 3072]: 45.5 -> 45.4 us, with the FP8
  // epilogue 42.2 -> 41.8 us).
  u32x4 bsc[BCAST ? CH : 1], bsh[BCAST ? CH : 1];
  if constexpr (BCAST) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int e = (i * LPR + lane) * V;
      const int el = (EXACT || e < N) ? e : 0;
      bsc[i] = ld_chunk<Tag>(a.scale, 0, el);
      bsh[i] = ld_chunk<Tag>(a.shift, 0, el);
    }
  }
  u32x4 c[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int e = (i * LPR + lane) * V;
    c[i] = (EXACT || (row_ok && e < N)) ? ld_x(e) : u32x4{0u, 0u, 0u, 0u};
  }
  // BCAST: 1 + scale and shift unpacked to fp32 once, while the row is in
  // flight, so the output loop is one fused multiply-add per element (the
  // same fp32 operations; [10530, 3072] with residual 44.1 -> 43.8 us, with
  // the FP8 epilogue 41.2 -> 41.0 us, at 5 waves per SIMD instead of 7).
  float sc1[BCAST ? CH : 1][V], shf[BCAST ? CH : 1][V];
  if constexpr (BCAST) {
#pragma unroll
    for (int i = 0; i < CH; ++i)
#pragma unroll
      for (int j = 0; j < V; ++j) {
        sc1[i][j] = 1.f + elem<Tag>(bsc[i], j);
        shf[i][j] = elem<Tag>(bsh[i], j);
      }
  }
  if constexpr (ADD) {
    u32x4 rc[CH];
    u32x4 gc[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int e = (i * LPR + lane) * V;
      const bool ok = EXACT || (row_ok && e < N);
      rc[i] = ok ? ld_res(e) : u32x4{0u, 0u, 0u, 0u};
      // No gate is a gate of ones: x * 1 is x exactly, so res + x * 1 is
      // res + x with its one rounding, and no per-element select is needed.
      gc[i] = !a.gate ? ones_chunk<Tag>()
                      : (ok ? ld_mod<Tag>(a.gate, a.gs, mrow, e) : u32x4{0u, 0u, 0u, 0u});
    }
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int e = (i * LPR + lane) * V;
      float u[V];
#pragma unroll
      for (int j = 0; j < V; ++j)
        u[j] = residual_update(elem<Tag>(rc[i], j), elem<Tag>(c[i], j), elem<Tag>(gc[i], j),
                               true);
      c[i] = pack<Tag>(u);  // the rounded residual is what gets normalized
      if (row_ok && (EXACT || e < N)) st_res(e, c[i]);
    }
  }

  // Statistics.
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const float v = elem<Tag>(c[i], j);
      if constexpr (NT == kLayer)
        sum += v;
      else
        sum += v * v;
    }
  }
  sum = row_reduce<LPR, OpSum>(sum, red_a);
  float mean = 0.f;
  float r;
  // EARLY: per-row scale and shift issued once the mean is known, so that
  // their latency overlaps the variance reduction; the launcher takes it only
  // when the grid holds two or more full rounds of waves (below).
  u32x4 esc[EARLY ? CH : 1], esh[EARLY ? CH : 1];
  if constexpr (NT == kLayer) {
    mean = div_by_len(sum, N);
    if constexpr (EARLY) {
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        const int e = (i * LPR + lane) * V;
        const bool ok = EXACT || (row_ok && e < N);
        esc[i] = ok ? ld_mod<Tag>(a.scale, a.scs, mrow, e) : u32x4{0u, 0u, 0u, 0u};
        esh[i] = ok ? ld_mod<Tag>(a.shift, a.shs, mrow, e) : u32x4{0u, 0u, 0u, 0u};
      }
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int e = (i * LPR + lane) * V;
      if (EXACT || e < N) {
#pragma unroll
        for (int j = 0; j < V; ++j) {
          const float t = elem<Tag>(c[i], j) - mean;
          ss += t * t;
        }
      }
    }
    ss = row_reduce<LPR, OpSum>(ss, red_b);
    r = 1.0f / sqrtf(div_by_len(ss, N) + a.eps);
  } else {
    r = 1.0f / sqrtf(div_by_len(sum, N) + a.eps);
  }

  // Output.
  // BCAST is taken only without gamma: no weight loads in the output loop
  // (a load on a branch there costs a wait for every memory operation in
  // flight, the row's stores included, before each chunk).
  const bool affine = !BCAST && a.gamma != nullptr;
  const bool has_beta = affine && a.beta != nullptr && NT == kLayer;
  float yq[QNT ? CH : 1][8];  // FP8 epilogue: the rounded y of this lane
  float ymax = 0.f;           // and its NaN-propagating maximum |y|
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int e = (i * LPR + lane) * V;
    if constexpr (QNT && !EXACT) {
#pragma unroll
      for (int j = 0; j < 8; ++j) yq[i][j] = 0.f;
    }
    if (!EXACT && !(row_ok && e < N)) continue;
    // Per-row scale and shift are loaded here rather than with the row:
    // issuing them with x measured slower at [3120, 4096] (20.0 -> 22.7 us).
    // (BCAST uses the fp32 rows sc1 / shf unpacked above.)
    u32x4 sc{0u, 0u, 0u, 0u}, sh{0u, 0u, 0u, 0u};
    if constexpr (EARLY) {
      sc = esc[i];
      sh = esh[i];
    } else if constexpr (!BCAST) {
      sc = ld_mod<Tag>(a.scale, a.scs, mrow, e);
      sh = ld_mod<Tag>(a.shift, a.shs, mrow, e);
    }
    u32x4 gm = u32x4{0u, 0u, 0u, 0u}, bt = u32x4{0u, 0u, 0u, 0u};
    if (affine) gm = ld_chunk<Tag>(a.gamma, 0, e);
    if (has_beta) bt = ld_chunk<Tag>(a.beta, 0, e);
    float o[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      float t = (NT == kLayer) ? (elem<Tag>(c[i], j) - mean) * r : elem<Tag>(c[i], j) * r;
      if (affine) t = t * elem<Tag>(gm, j);
      if (has_beta) t = t + elem<Tag>(bt, j);
      if constexpr (BCAST)
        o[j] = t * sc1[i][j] + shf[i][j];
      else
        o[j] = t * (1.f + elem<Tag>(sc, j)) + elem<Tag>(sh, j);
    }
    if constexpr (QNT) {
      const u32x4 yr = pack<Tag>(o);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        yq[i][j] = elem<Tag>(yr, j);
        ymax = nan_max_abs(ymax, yq[i][j]);
      }
    } else if constexpr (EXACT) {
      if (row_ok) st16_nt(byte_off(a.y, (row * a.ys) * Tag::kBytes + e * Tag::kBytes), pack<Tag>(o));
    } else {
      st_row<Tag>(a.y, row * a.ys, e, pack<Tag>(o));
    }
  }
  if constexpr (QNT) {
    // As quant_rows_kernel: a finite NaN-propagating maximum is the
    // reference's amax and lets the clamp go; waves (workgroups, for rows
    // wider than a wave) with a non-finite row take the NaN-skipping maximum
    // and clamp.
    bool any_nonfinite;
    float amax = row_amax_vote<LPR>(ymax, red_c, any_nonfinite);
    const bool finite_row = finite_bits(amax);
    if (any_nonfinite) {
      float m = 0.f;
#pragma unroll
      for (int i = 0; i < CH; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(yq[i][j]));
      amax = row_reduce<LPR, OpAmax>(m, red_d);
    }
    const float scale = amax / kFp8Max;
    if (row_ok && lane == 0) a.s[row] = scale;
    const float inv = (scale == 0.f) ? 0.f : 1.0f / scale;
    const bool fast = finite_row && finite_bits(inv);
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int e = (i * LPR + lane) * V;
      if (row_ok && (EXACT || e < N))
        st8_nt((a.q + row * a.qs) + e, fast ? quant8<false>(yq[i], inv) : quant8<true>(yq[i], inv));
    }
  }
}

// One row per workgroup with element-wise accesses (any N, any alignment).
// With QNT, y is evaluated twice (for the row maximum, then to quantize):
// both evaluations are the same operations on the same values.
template <class Tag, int NT, bool ADD, bool QNT>
__global__ __launch_bounds__(kBlock) void norm_mod_generic_kernel(const NormArgs a) {
  __shared__ float red[kBlock / kWave];
  const int64_t row = blockIdx.x;
  const int N = a.N;
  const int64_t mrow = mod_row(a, row);
  const int64_t xo = row * a.xs, ro = row * a.rs, go = mrow * a.gs;
  const int64_t so = mrow * a.scs, ho = mrow * a.shs, yo = row * a.ys;
  if constexpr (ADD) {
    // Each thread later reads back exactly the elements it writes here.
    for (int i = threadIdx.x; i < N; i += kBlock) {
      const float xv = load_elem<Tag>(a.x, xo + i);
      store_elem<Tag>(a.res, ro + i, residual_update(load_elem<Tag>(a.res, ro + i), xv,
                                                     a.gate ? load_elem<Tag>(a.gate, go + i) : 1.f,
                                                     a.gate != nullptr));
    }
  }
  const void* src = ADD ? a.res : a.x;
  const int64_t so_src = ADD ? ro : xo;
  float sum = 0.f;
  for (int i = threadIdx.x; i < N; i += kBlock) {
    const float v = load_elem<Tag>(src, so_src + i);
    sum += (NT == kLayer) ? v : v * v;
  }
  sum = block_reduce<OpSum>(sum, red);
  float mean = 0.f, r;
  if constexpr (NT == kLayer) {
    mean = div_by_len(sum, N);
    float ss = 0.f;
    for (int i = threadIdx.x; i < N; i += kBlock) {
      const float t = load_elem<Tag>(src, so_src + i) - mean;
      ss += t * t;
    }
    ss = block_reduce<OpSum>(ss, red);
    r = 1.0f / sqrtf(div_by_len(ss, N) + a.eps);
  } else {
    r = 1.0f / sqrtf(div_by_len(sum, N) + a.eps);
  }
  const bool affine = a.gamma != nullptr;
  const bool has_beta = affine && a.beta != nullptr && NT == kLayer;
  auto y_at = [&](int i) {
    const float v = load_elem<Tag>(src, so_src + i);
    float t = (NT == kLayer) ? (v - mean) * r : v * r;
    if (affine) t = t * load_elem<Tag>(a.gamma, i);
    if (has_beta) t = t + load_elem<Tag>(a.beta, i);
    return t * (1.f + load_elem<Tag>(a.scale, so + i)) + load_elem<Tag>(a.shift, ho + i);
  };
  if constexpr (QNT) {
    float amax = 0.f;
    for (int i = threadIdx.x; i < N; i += kBlock) amax = fmaxf(amax, fabsf(round_to<Tag>(y_at(i))));
    amax = block_reduce<OpAmax>(amax, red);
    const float scale = amax / kFp8Max;
    if (threadIdx.x == 0) a.s[row] = scale;
    const float inv = (scale == 0.f) ? 0.f : 1.0f / scale;
    for (int i = threadIdx.x; i < N; i += kBlock)
      a.q[row * a.qs + i] = fp8_byte(round_to<Tag>(y_at(i)) * inv);
  } else {
    for (int i = threadIdx.x; i < N; i += kBlock) store_elem<Tag>(a.y, yo + i, y_at(i));
  }
}

template <class Tag, int NT, bool ADD, bool QNT>
int launch_norm_mod(const NormArgs& a, hipStream_t stream, const char* op) {
  const int b = Tag::kBytes;
  const bool out_ok = QNT ? (aligned(a.q, 8) && a.qs % 8 == 0)
                          : (aligned(a.y, 16) && (a.ys * b) % 16 == 0);
  bool vec_ok = (a.N % Tag::kVec == 0) && aligned(a.x, 16) && (a.xs * b) % 16 == 0 && out_ok &&
                aligned(a.scale, 16) && (a.scs * b) % 16 == 0 && aligned(a.shift, 16) &&
                (a.shs * b) % 16 == 0 && aligned(a.gamma, 16) && aligned(a.beta, 16);
  if (ADD)
    vec_ok = vec_ok && aligned(a.res, 16) && (a.rs * b) % 16 == 0 && aligned(a.gate, 16) &&
             (a.gs * b) % 16 == 0;
  bool launched = false;
  if (vec_ok) {
    launched = dispatch_row_shape<Tag::kVec, true, 256>(a.N, [&](auto lpr, auto ch) {
      constexpr int LPR = decltype(lpr)::value;
      constexpr int CH = decltype(ch)::value;
      // Per-row scale and shift issued early (EARLY) pay when waves wait on
      // others' completion: with four waves per row at [4096, 4096] (two full
      // rounds of 8192 wave slots) 23.9 -> 23.4 us, while at [3120, 4096]
      // (1.5 rounds) the same kernel lost, 18.2 -> 18.7 us.
      constexpr bool kEarlyShape = LPR == 256 && CH == 2 && NT == kLayer && !ADD && !QNT;
      const dim3 grid(static_cast<unsigned>(row_blocks(a.M, LPR)));
      // Rows that fill the lanes exactly (N == LPR * CH * V, 16-bit types)
      // with broadcast modulation drop the per-lane bounds tests ([10530,
      // 3072] residual + LayerNorm + AdaLN 45.4 -> 43.9 us, with the FP8
      // epilogue 41.6 -> 41.2 us; with per-row scale / shift, [3120, 4096] and
      // [4096, 4096], the same change measured 1% slower, so those keep the
      // tested form).
      const bool exact = Tag::kVec == 8 && int64_t{LPR} * CH * Tag::kVec == a.N;
      if (a.scs == 0 && a.shs == 0 && !a.gamma) {
        if (exact)
          hipLaunchKernelGGL((norm_mod_kernel<Tag, LPR, CH, NT, ADD, QNT, true, false,
                                              Tag::kVec == 8>),
                             grid, dim3(kBlock), 0, stream, a);
        else
          hipLaunchKernelGGL((norm_mod_kernel<Tag, LPR, CH, NT, ADD, QNT, true>), grid,
                             dim3(kBlock), 0, stream, a);
      } else if (kEarlyShape && a.M * (LPR / kWave) >= 2 * kFewRows) {
        hipLaunchKernelGGL((norm_mod_kernel<Tag, LPR, CH, NT, ADD, QNT, false, kEarlyShape>),
                           grid, dim3(kBlock), 0, stream, a);
      } else {
        hipLaunchKernelGGL((norm_mod_kernel<Tag, LPR, CH, NT, ADD, QNT>), grid, dim3(kBlock), 0,
                           stream, a);
      }
    }, a.M);
  }
  if (!launched)
    hipLaunchKernelGGL((norm_mod_generic_kernel<Tag, NT, ADD, QNT>), dim3(a.M), dim3(kBlock), 0,
                       stream, a);
  return launch_status(op);
}

template <int NT, bool ADD>
int launch_norm_mod_dt(int dtype, const NormArgs& a, hipStream_t stream, const char* op) {
  switch (dtype) {
    case JO_DTYPE_BF16: return launch_norm_mod<BF16, NT, ADD, false>(a, stream, op);
    case JO_DTYPE_F16: return launch_norm_mod<F16, NT, ADD, false>(a, stream, op);
    default: return launch_norm_mod<F32, NT, ADD, false>(a, stream, op);
  }
}

template <int NT, bool ADD>
int launch_norm_mod_quant_dt(int dtype, const NormArgs& a, hipStream_t stream, const char* op) {
  if (dtype == JO_DTYPE_BF16) return launch_norm_mod<BF16, NT, ADD, true>(a, stream, op);
  return launch_norm_mod<F16, NT, ADD, true>(a, stream, op);
}

// ---------------------------------------------------------------------------
// RMSNorm rows.
//   MODE kKernelRms: out = (x * r) * w, one rounding (rmsnorm.cu:41-60);
//     the sum of squares in fp32 like the reference kernel.
//   MODE kModuleRms: out = round(round(x * r) * w), the torch RMSNorm module
//     (dit.py:244-249: the normalized row is cast back to the input type
//     before the weight multiply). Its mean square is an fp64 sum of the
//     (exact) squares rounded once to fp32; two summation orders give fp64
//     sums within ~2^-52 of each other, so the fp32 value, and with it the
//     intermediate rounding, depends on the order only for sums that fall on
//     an fp32 rounding boundary to that precision.
//   r = 1 / sqrt(mean(x^2) + eps) with IEEE sqrt and division.
// HEADS: row m is head m % heads of token m / heads, read at
// x + token * xs + head * xhs (a per-head norm straight from a packed qkv
// view); otherwise row m starts at x + m * xs. Output rows are out + m * os.
// ---------------------------------------------------------------------------
constexpr int kKernelRms = 0;
constexpr int kModuleRms = 1;

// An fp32 product rounded on to the element type: two roundings, as
// x.float() * rsqrt(...) followed by .type_as(x) does. The empty asm keeps the
// product an fp32 value; without it the compiler folds multiply and
// conversion into v_fma_mixlo_f16, which rounds the exact product once.
template <class Tag>
__device__ __forceinline__ float round_fp32_product(float v) {
  asm volatile("" : "+v"(v));
  return round_to<Tag>(v);
}

struct RmsArgs {
  const void* x;
  int64_t xs, xhs;
  int heads;
  const void* w;
  void* out;
  int64_t os;
  int64_t M;
  int N;
  float eps;
  FastDiv fd_heads;  // HEADS: the row index's divisor (set by launch_rmsnorm)
};

template <bool HEADS>
__device__ __forceinline__ int64_t rms_row_offset(const RmsArgs& a, int64_t row) {
  if constexpr (HEADS) {
    // M < 2^32 (checked on the host), so the division can be 32-bit, by
    // multiply-high ([1, 3120, 32, 128] K slice: R_kn).
    const uint32_t t = fdiv(static_cast<uint32_t>(row), a.fd_heads);
    return static_cast<int64_t>(t) * a.xs + (row - static_cast<int64_t>(t) * a.heads) * a.xhs;
  } else {
    return row * a.xs;
  }
}

template <class Tag, int LPR, int CH, bool HEADS, int MODE>
__global__ __launch_bounds__(kBlock) void rmsnorm_kernel(const RmsArgs a) {
  constexpr int V = Tag::kVec;
  constexpr int RPB = kBlock / LPR;
  __shared__ float red[kBlock / kWave];
  __shared__ double red64[kBlock / kWave];
  const int lane = threadIdx.x % LPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / LPR;
  const bool row_ok = row < a.M;
  const int N = a.N;
  const int64_t xo = row_ok ? rms_row_offset<HEADS>(a, row) : 0;
  u32x4 c[CH], wv[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int e = (i * LPR + lane) * V;
    c[i] = (row_ok && e < N) ? ld_row<Tag>(a.x, xo, e) : u32x4{0u, 0u, 0u, 0u};
  }
  // Weight chunks are issued with the row loads so their (cached) latency
  // overlaps the row's instead of following the reduction ([99840, 128]:
  // 10.8 -> 10.2 us).
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int e = (i * LPR + lane) * V;
    wv[i] = e < N ? ld_chunk<Tag>(a.w, 0, e) : u32x4{0u, 0u, 0u, 0u};
  }
  float ms;
  if constexpr (MODE == kModuleRms) {
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const double v = static_cast<double>(elem<Tag>(c[i], j));
        ss = __builtin_fma(v, v, ss);
      }
    }
    ss = row_reduce_sum64<LPR>(ss, red64);
    ms = static_cast<float>(ss / static_cast<double>(N));
  } else {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const float v = elem<Tag>(c[i], j);
        ss += v * v;
      }
    }
    ss = row_reduce<LPR, OpSum>(ss, red);
    ms = div_by_len(ss, N);
  }
  const float r = 1.0f / sqrtf(ms + a.eps);
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int e = (i * LPR + lane) * V;
    if (!(row_ok && e < N)) continue;
    float o[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      float xr = elem<Tag>(c[i], j) * r;
      if constexpr (MODE == kModuleRms) xr = round_fp32_product<Tag>(xr);
      o[j] = xr * elem<Tag>(wv[i], j);
    }
    st_row<Tag>(a.out, row * a.os, e, pack<Tag>(o));
  }
}

// One row per workgroup, element-wise accesses: any row length and alignment.
template <class Tag, bool HEADS, int MODE>
__global__ __launch_bounds__(kBlock) void rmsnorm_generic_kernel(const RmsArgs a) {
  __shared__ float red[kBlock / kWave];
  __shared__ double red64[kBlock / kWave];
  const int64_t row = blockIdx.x;
  const int64_t xo = rms_row_offset<HEADS>(a, row);
  float ms;
  if constexpr (MODE == kModuleRms) {
    double ss = 0.0;
    for (int i = threadIdx.x; i < a.N; i += kBlock) {
      const double v = static_cast<double>(load_elem<Tag>(a.x, xo + i));
      ss = __builtin_fma(v, v, ss);
    }
    ss = row_reduce_sum64<kBlock>(ss, red64);
    ms = static_cast<float>(ss / static_cast<double>(a.N));
  } else {
    float ss = 0.f;
    for (int i = threadIdx.x; i < a.N; i += kBlock) {
      const float v = load_elem<Tag>(a.x, xo + i);
      ss += v * v;
    }
    ss = block_reduce<OpSum>(ss, red);
    ms = div_by_len(ss, a.N);
  }
  const float r = 1.0f / sqrtf(ms + a.eps);
  for (int i = threadIdx.x; i < a.N; i += kBlock) {
    float xr = load_elem<Tag>(a.x, xo + i) * r;
    if constexpr (MODE == kModuleRms) xr = round_fp32_product<Tag>(xr);
    store_elem<Tag>(a.out, row * a.os + i, xr * load_elem<Tag>(a.w, i));
  }
}

template <class Tag, bool HEADS, int MODE>
int launch_rmsnorm(const RmsArgs& args, hipStream_t stream, const char* op) {
  RmsArgs a = args;
  if (HEADS) a.fd_heads = make_fastdiv(static_cast<uint32_t>(a.heads));
  const int b = Tag::kBytes;
  const bool vec_ok = (a.N % Tag::kVec == 0) && aligned(a.x, 16) && (a.xs * b) % 16 == 0 &&
                      (!HEADS || (a.xhs * b) % 16 == 0) && aligned(a.w, 16) &&
                      aligned(a.out, 16) && (a.os * b) % 16 == 0;
  bool launched = false;
  if (vec_ok) {
    launched = dispatch_row_shape<Tag::kVec>(a.N, [&](auto lpr, auto ch) {
      constexpr int LPR = decltype(lpr)::value;
      constexpr int CH = decltype(ch)::value;
      hipLaunchKernelGGL((rmsnorm_kernel<Tag, LPR, CH, HEADS, MODE>), dim3(row_blocks(a.M, LPR)),
                         dim3(kBlock), 0, stream, a);
    });
  }
  if (!launched)
    hipLaunchKernelGGL((rmsnorm_generic_kernel<Tag, HEADS, MODE>), dim3(a.M), dim3(kBlock), 0,
                       stream, a);
  return launch_status(op);
}

template <bool HEADS, int MODE>
int launch_rmsnorm_dt(int dtype, const RmsArgs& a, hipStream_t stream, const char* op) {
  switch (dtype) {
    case JO_DTYPE_BF16: return launch_rmsnorm<BF16, HEADS, MODE>(a, stream, op);
    case JO_DTYPE_F16: return launch_rmsnorm<F16, HEADS, MODE>(a, stream, op);
    default: return launch_rmsnorm<F32, HEADS, MODE>(a, stream, op);
  }
}

}  // namespace
}  // namespace jo

using namespace jo;

namespace {
int norm_scale_shift_impl(const void* x, int64_t x_stride, const void* gamma, const void* beta,
                          const void* scale, int64_t scale_stride, const void* shift,
                          int64_t shift_stride, int64_t mod_rows, void* y, int64_t y_stride,
                          int64_t M, int64_t N, int dtype, int norm_type, float eps,
                          void* stream) {
  // Checks of fused_norm_scale_shift.cu:176-196.
  JO_REQUIRE(valid_dtype(dtype), "Unsupported dtype; use float32/float16/bfloat16");
  JO_REQUIRE(norm_type == JO_NORM_LAYER || norm_type == JO_NORM_RMS,
             "norm_type must be 0 (layer) or 1 (rms)");
  JO_REQUIRE(M >= 0 && N >= 0 && N <= INT32_MAX && M <= kMaxRows,
             "fused_norm_scale_shift: bad shape");
  JO_REQUIRE(N % 4 == 0, "N must be divisible by 4");
  JO_REQUIRE(x_stride >= N && y_stride >= N && scale_stride >= 0 && shift_stride >= 0,
             "fused_norm_scale_shift: bad row stride");
  JO_REQUIRE(mod_rows >= 1 && mod_rows <= UINT32_MAX,
             "fused_norm_scale_shift: mod_rows must be positive");
  if (M == 0 || N == 0) return JO_OK;
  JO_REQUIRE(x && y && scale && shift, "fused_norm_scale_shift: null pointer");
  NormArgs a{x, x_stride, nullptr, 0, nullptr, 0, gamma, beta, scale, scale_stride, shift,
             shift_stride, y, y_stride, M, static_cast<int>(N), eps};
  a.mod_rows = static_cast<uint32_t>(mod_rows);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (norm_type == JO_NORM_LAYER)
    return launch_norm_mod_dt<kLayer, false>(dtype, a, st, "fused_norm_scale_shift");
  return launch_norm_mod_dt<kRms, false>(dtype, a, st, "fused_norm_scale_shift");
}
}  // namespace

extern "C" int jo_fused_norm_scale_shift(const void* x, int64_t x_stride, const void* gamma,
                                         const void* beta, const void* scale,
                                         int64_t scale_stride, const void* shift,
                                         int64_t shift_stride, void* y, int64_t y_stride,
                                         int64_t M, int64_t N, int dtype, int norm_type,
                                         float eps, void* stream) {
  return norm_scale_shift_impl(x, x_stride, gamma, beta, scale, scale_stride, shift,
                               shift_stride, 1, y, y_stride, M, N, dtype, norm_type, eps, stream);
}

extern "C" int jo_fused_norm_scale_shift_per_sample(
    const void* x, int64_t x_stride, const void* gamma, const void* beta, const void* scale,
    int64_t scale_stride, const void* shift, int64_t shift_stride, int64_t mod_rows, void* y,
    int64_t y_stride, int64_t M, int64_t N, int dtype, int norm_type, float eps, void* stream) {
  return norm_scale_shift_impl(x, x_stride, gamma, beta, scale, scale_stride, shift,
                               shift_stride, mod_rows, y, y_stride, M, N, dtype, norm_type, eps,
                               stream);
}

extern "C" int jo_rmsnorm(const void* x, int64_t x_stride, const void* weight, void* out,
                          int64_t out_stride, int64_t M, int64_t N, int dtype, float eps,
                          void* stream) {
  // Checks of rmsnorm.cu:77-81.
  JO_REQUIRE(valid_dtype(dtype), "Unsupported dtype; use float32/float16/bfloat16");
  JO_REQUIRE(M >= 0 && N >= 0 && N <= INT32_MAX && M <= kMaxRows, "rmsnorm: bad shape");
  JO_REQUIRE(x_stride >= N && out_stride >= N, "rmsnorm: bad row stride");
  if (M == 0 || N == 0) return JO_OK;
  JO_REQUIRE(x && weight && out, "rmsnorm: null pointer");
  const RmsArgs a{x, x_stride, 0, 1, weight, out, out_stride, M, static_cast<int>(N), eps};
  return launch_rmsnorm_dt<false, kKernelRms>(dtype, a, static_cast<hipStream_t>(stream),
                                              "rmsnorm");
}

extern "C" int jo_rmsnorm_heads(const void* x, int64_t x_token_stride, int64_t x_head_stride,
                                const void* weight, void* out, int64_t out_stride,
                                int64_t tokens, int64_t heads, int64_t head_dim, int dtype,
                                float eps, int round_first, void* stream) {
  const char* op = "rmsnorm_heads";
  JO_REQUIRE(valid_dtype(dtype), "Unsupported dtype; use float32/float16/bfloat16");
  JO_REQUIRE(round_first == 0 || round_first == 1, "%s: round_first must be 0 or 1", op);
  JO_REQUIRE(tokens >= 0 && heads > 0 && heads <= INT32_MAX && head_dim > 0 &&
                 head_dim <= INT32_MAX && tokens <= kMaxRows && tokens * heads <= kMaxRows,
             "%s: bad shape [%lld, %lld, %lld]", op, static_cast<long long>(tokens),
             static_cast<long long>(heads), static_cast<long long>(head_dim));
  JO_REQUIRE((heads == 1 || x_head_stride >= head_dim) && x_head_stride >= 0 &&
                 x_token_stride >= 0 && out_stride >= head_dim,
             "%s: bad strides", op);
  if (tokens == 0) return JO_OK;
  JO_REQUIRE(x && weight && out, "%s: null pointer", op);
  const RmsArgs a{x, x_token_stride, x_head_stride, static_cast<int>(heads), weight, out,
                  out_stride, tokens * heads, static_cast<int>(head_dim), eps};
  hipStream_t st = static_cast<hipStream_t>(stream);
  return round_first ? launch_rmsnorm_dt<true, kModuleRms>(dtype, a, st, op)
                     : launch_rmsnorm_dt<true, kKernelRms>(dtype, a, st, op);
}

extern "C" int jo_fused_add_layernorm_scale_shift(
    const void* x, int64_t x_stride, void* residual, int64_t res_stride, const void* gate,
    int64_t gate_stride, const void* gamma, const void* beta, const void* scale,
    int64_t scale_stride, const void* shift, int64_t shift_stride, int64_t mod_rows, void* y,
    int64_t y_stride, int64_t M, int64_t N, int dtype, float eps, void* stream) {
  JO_REQUIRE(valid_dtype(dtype), "Unsupported dtype; use float32/float16/bfloat16");
  JO_REQUIRE(M >= 0 && N >= 0 && N <= INT32_MAX && M <= kMaxRows,
             "fused_add_layernorm_scale_shift: bad shape");
  JO_REQUIRE(N % 4 == 0, "N must be divisible by 4");
  JO_REQUIRE(x_stride >= N && res_stride >= N && y_stride >= N && scale_stride >= 0 &&
                 shift_stride >= 0 && gate_stride >= 0,
             "fused_add_layernorm_scale_shift: bad row stride");
  JO_REQUIRE(mod_rows >= 1 && mod_rows <= UINT32_MAX,
             "fused_add_layernorm_scale_shift: mod_rows must be positive");
  if (M == 0 || N == 0) return JO_OK;
  JO_REQUIRE(x && residual && y && scale && shift,
             "fused_add_layernorm_scale_shift: null pointer");
  NormArgs a{x, x_stride, residual, res_stride, gate, gate_stride, gamma, beta, scale,
             scale_stride, shift, shift_stride, y, y_stride, M, static_cast<int>(N), eps};
  a.mod_rows = static_cast<uint32_t>(mod_rows);
  return launch_norm_mod_dt<kLayer, true>(dtype, a, static_cast<hipStream_t>(stream),
                                          "fused_add_layernorm_scale_shift");
}

extern "C" int jo_norm_scale_shift_quant_fp8(
    const void* x, int64_t x_stride, void* residual, int64_t res_stride, const void* gate,
    int64_t gate_stride, const void* gamma, const void* beta, const void* scale,
    int64_t scale_stride, const void* shift, int64_t shift_stride, int64_t mod_rows, void* out_q,
    int64_t q_stride, float* out_s, int64_t M, int64_t N, int dtype, int norm_type, float eps,
    void* stream) {
  const char* op = "norm_scale_shift_quant_fp8";
  JO_REQUIRE(dtype == JO_DTYPE_BF16 || dtype == JO_DTYPE_F16,
             "%s: input must be bf16 or fp16 (the quantized row is the 16-bit y)", op);
  JO_REQUIRE(norm_type == JO_NORM_LAYER || norm_type == JO_NORM_RMS,
             "norm_type must be 0 (layer) or 1 (rms)");
  // N == 0 is rejected: there would be scales to write but no values to
  // take them from.
  JO_REQUIRE(M >= 0 && N > 0 && N <= INT32_MAX && M <= kMaxRows, "%s: bad shape [%lld, %lld]",
             op, static_cast<long long>(M), static_cast<long long>(N));
  JO_REQUIRE(N % 4 == 0, "N must be divisible by 4");
  JO_REQUIRE(x_stride >= N && q_stride >= N && scale_stride >= 0 && shift_stride >= 0 &&
                 gate_stride >= 0 && (residual == nullptr || res_stride >= N),
             "%s: bad row stride", op);
  JO_REQUIRE(residual != nullptr || gate == nullptr, "%s: a gate needs a residual", op);
  JO_REQUIRE(mod_rows >= 1 && mod_rows <= UINT32_MAX, "%s: mod_rows must be positive", op);
  if (M == 0) return JO_OK;
  JO_REQUIRE(x && out_q && out_s && scale && shift, "%s: null pointer", op);
  NormArgs a{x, x_stride, residual, res_stride, gate, gate_stride, gamma, beta, scale,
             scale_stride, shift, shift_stride, nullptr, 0, M, static_cast<int>(N), eps,
             static_cast<uint8_t*>(out_q), q_stride, out_s, static_cast<uint32_t>(mod_rows)};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (residual) {
    if (norm_type == JO_NORM_LAYER) return launch_norm_mod_quant_dt<kLayer, true>(dtype, a, st, op);
    return launch_norm_mod_quant_dt<kRms, true>(dtype, a, st, op);
  }
  if (norm_type == JO_NORM_LAYER) return launch_norm_mod_quant_dt<kLayer, false>(dtype, a, st, op);
  return launch_norm_mod_quant_dt<kRms, false>(dtype, a, st, op);
}
