// RoPE-and-copy of staged K (and plain copy of V) into the graph runner's KV
// pool: the commit step of deploy/xvideo/serving/graph_runner.py:137-142
// (also its seeding, :204-215, and the pre-RoPE cache reuse of
// deploy/xvideo/models/dit/dit.py:211-217), all layers in one launch.
//
// The rotation is apply_rotary_emb (rope.py:21-28) as torch evaluates it:
//   out = (x.float() * cos + rotate_half(x.float()) * sin).type_as(x)
// i.e. for a pair (x0, x1) at columns (2i, 2i+1):
//   out0 = fl(fl(x0 * cos[2i])   - fl(x1 * sin[2i]))
//   out1 = fl(fl(x1 * cos[2i+1]) + fl(x0 * sin[2i+1]))
// three separately rounded fp32 operations (no fused multiply-add), then one
// round to the element type. The fp32 tables are read as given ([T, D], both
// columns of a pair), so any table the reference's builders produce is
// reproduced bit for bit.
//
// One wave64 per (layer, batch, token) row of H*D elements and tensor: 16-byte
// streaming loads/stores, the row in registers; the V rows are copied by
// waves of their own, after all the K waves. A lane's table columns repeat
// every head (512 elements per pass is a whole number of heads when D divides
// 512), so a lane reads its 8 cos and 8 sin values once per row.

#include <type_traits>

#include "jo_device.hpp"
#include "jo_host.hpp"

namespace jo {
namespace {

struct CommitArgs {
  const void* src_k;
  const void* src_v;  // optional
  void* dst_k;
  void* dst_v;        // optional (with src_v)
  int64_t layers, batch, tokens;
  int row_elems;      // H * D
  int head_dim;
  int64_t s_ls, s_bs, s_ts;  // source strides (elements): layer, batch, token
  int64_t d_ls, d_bs, d_ts;  // destination strides
  int64_t d_off;             // destination token offset
  const float* cos;          // [B?, T, D] fp32: token stride tab_ts, batch stride tab_bs
  const float* sin;          // (tab_bs 0: one table for every batch row)
  int64_t tab_ts, tab_bs;
  FastDiv fd_tokens, fd_batch;  // the row index's divisors (set by launch_commit)
};

// The pair rotation with torch's rounding sequence.
__device__ __forceinline__ void rope_pair(float x0, float x1, float c0, float s0, float c1,
                                          float s1, float& o0, float& o1) {
#pragma clang fp contract(off)
  const float a = x0 * c0;
  const float b = x1 * s0;
  const float c = x1 * c1;
  const float d = x0 * s1;
  o0 = a - b;
  o1 = c + d;
}

// KV2: K rows and V rows on separate waves, all K waves first (each wave
// streams one tensor; a V wave is a plain copy and reads no table).
template <class Tag, int CH, bool KV2>
__global__ __launch_bounds__(kBlock) void rope_commit_kernel(const CommitArgs a) {
  static_assert(Tag::kVec == 8, "16-bit rows");
  const int lane = threadIdx.x % kWave;
  // The wave index through readfirstlane, and 32-bit row arithmetic with
  // multiply-high division (rows < 2^32 by the launch check): the index math
  // is scalar instead of 64-bit divisions in every lane.
  const int64_t wid = static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) +
                      __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int64_t rows = a.layers * a.batch * a.tokens;
  const bool v_wave = KV2 && wid >= rows;  // wave-uniform
  const int64_t row = v_wave ? wid - rows : wid;
  if (row >= rows) return;
  const uint32_t r32 = static_cast<uint32_t>(row);
  const uint32_t lb32 = fdiv(r32, a.fd_tokens);
  const uint32_t l32 = fdiv(lb32, a.fd_batch);
  const int64_t n = r32 - lb32 * static_cast<uint32_t>(a.tokens);
  const int64_t b = lb32 - l32 * static_cast<uint32_t>(a.batch);
  const int64_t l = l32;
  const int64_t so = l * a.s_ls + b * a.s_bs + n * a.s_ts;
  const int64_t dof = l * a.d_ls + b * a.d_bs + (a.d_off + n) * a.d_ts;
  const bool do_k = !v_wave;
  const bool do_v = a.src_v != nullptr && (!KV2 || v_wave);

  // Loads are never predicated per lane (a predicated load's join forces an
  // early wait): a chunk beyond the row reads a chunk inside it instead and
  // is never stored. The branches below are uniform over the wave.
  const int e_safe = (lane * 8) % a.row_elems;
  u32x4 k[CH], v[CH];
  u32x4 c_lo, c_hi, s_lo, s_hi;
  if (do_k) {
    // Table columns of this lane (same in every chunk: 512 % D == 0).
    const int d0 = (lane * 8) % a.head_dim;
    const float* ct = a.cos + b * a.tab_bs + n * a.tab_ts + d0;
    const float* st = a.sin + b * a.tab_bs + n * a.tab_ts + d0;
    c_lo = ld16(ct);
    c_hi = ld16(ct + 4);
    s_lo = ld16(st);
    s_hi = ld16(st + 4);
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int e = i * 512 + lane * 8;
      k[i] = ld16_nt(byte_off(a.src_k, (so + (e < a.row_elems ? e : e_safe)) * Tag::kBytes));
    }
  }
  if (do_v) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int e = i * 512 + lane * 8;
      v[i] = ld16_nt(byte_off(a.src_v, (so + (e < a.row_elems ? e : e_safe)) * Tag::kBytes));
    }
  }
  if (do_k) {
    float cs[8], sn[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      cs[j] = elem<F32>(c_lo, j);
      cs[j + 4] = elem<F32>(c_hi, j);
      sn[j] = elem<F32>(s_lo, j);
      sn[j + 4] = elem<F32>(s_hi, j);
    }
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int e = i * 512 + lane * 8;
      if (e >= a.row_elems) continue;
      float o[8];
#pragma unroll
      for (int p = 0; p < 4; ++p)
        rope_pair(elem<Tag>(k[i], 2 * p), elem<Tag>(k[i], 2 * p + 1), cs[2 * p], sn[2 * p],
                  cs[2 * p + 1], sn[2 * p + 1], o[2 * p], o[2 * p + 1]);
      st16_nt(byte_off(a.dst_k, (dof + e) * Tag::kBytes), pack<Tag>(o));
    }
  }
  if (do_v) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int e = i * 512 + lane * 8;
      if (e < a.row_elems) st16_nt(byte_off(a.dst_v, (dof + e) * Tag::kBytes), v[i]);
    }
  }
}

// One row per workgroup, element pairs (any head_dim, any alignment).
template <class Tag>
__global__ __launch_bounds__(kBlock) void rope_commit_generic_kernel(const CommitArgs a) {
  const int64_t row = blockIdx.x;
  const int64_t n = row % a.tokens;
  const int64_t lb = row / a.tokens;
  const int64_t b = lb % a.batch;
  const int64_t l = lb / a.batch;
  const int64_t so = l * a.s_ls + b * a.s_bs + n * a.s_ts;
  const int64_t dof = l * a.d_ls + b * a.d_bs + (a.d_off + n) * a.d_ts;
  const float* ct = a.cos + b * a.tab_bs + n * a.tab_ts;
  const float* st = a.sin + b * a.tab_bs + n * a.tab_ts;
  for (int p = threadIdx.x; p < a.row_elems / 2; p += kBlock) {
    const int e = 2 * p;
    const int d = e % a.head_dim;
    float o0, o1;
    rope_pair(load_elem<Tag>(a.src_k, so + e), load_elem<Tag>(a.src_k, so + e + 1), ct[d], st[d],
              ct[d + 1], st[d + 1], o0, o1);
    store_elem<Tag>(a.dst_k, dof + e, o0);
    store_elem<Tag>(a.dst_k, dof + e + 1, o1);
    if (a.src_v) {
      store_elem<Tag>(a.dst_v, dof + e, load_elem<Tag>(a.src_v, so + e));
      store_elem<Tag>(a.dst_v, dof + e + 1, load_elem<Tag>(a.src_v, so + e + 1));
    }
  }
}

template <class Tag>
int launch_commit(const CommitArgs& args, hipStream_t stream) {
  CommitArgs a = args;
  a.fd_tokens = make_fastdiv(static_cast<uint32_t>(a.tokens));
  a.fd_batch = make_fastdiv(static_cast<uint32_t>(a.batch));
  const int b = Tag::kBytes;
  const int64_t rows = a.layers * a.batch * a.tokens;
  auto al = [&](const void* p, int64_t stride_elems) {
    return p == nullptr || (aligned(p, 16) && (stride_elems * b) % 16 == 0);
  };
  const bool vec_ok = a.row_elems % 8 == 0 && 512 % a.head_dim == 0 && a.head_dim % 8 == 0 &&
                      al(a.src_k, a.s_ls) && al(a.src_k, a.s_bs) && al(a.src_k, a.s_ts) &&
                      al(a.src_v, a.s_ls) && al(a.src_v, a.s_bs) && al(a.src_v, a.s_ts) &&
                      al(a.dst_k, a.d_ls) && al(a.dst_k, a.d_bs) && al(a.dst_k, a.d_ts) &&
                      al(a.dst_v, a.d_ls) && al(a.dst_v, a.d_bs) && al(a.dst_v, a.d_ts) &&
                      aligned(a.cos, 16) && aligned(a.sin, 16) && a.tab_ts % 4 == 0 &&
                      a.tab_bs % 4 == 0;
  const int chunks = (a.row_elems + 511) / 512;
  // K and V on separate waves: 40 x 1560 x [32, 128] 357 -> 340 us (twice the
  // waves, each streaming one tensor). The JO_KNOB_KV_SPLIT override 1 keeps
  // them on one wave (launch shape only; results are identical).
  const bool kv2 = a.src_v != nullptr && launch_knob(JO_KNOB_KV_SPLIT) != 1;
  const dim3 grid(static_cast<unsigned>(((kv2 ? 2 : 1) * rows + 3) / 4));
  bool launched = true;
  auto go = [&](auto ch) {
    constexpr int CH = decltype(ch)::value;
    if (kv2)
      hipLaunchKernelGGL((rope_commit_kernel<Tag, CH, true>), grid, dim3(kBlock), 0, stream, a);
    else
      hipLaunchKernelGGL((rope_commit_kernel<Tag, CH, false>), grid, dim3(kBlock), 0, stream, a);
  };
  if (vec_ok && chunks <= 1)
    go(std::integral_constant<int, 1>{});
  else if (vec_ok && chunks <= 2)
    go(std::integral_constant<int, 2>{});
  else if (vec_ok && chunks <= 4)
    go(std::integral_constant<int, 4>{});
  else if (vec_ok && chunks <= 6)
    go(std::integral_constant<int, 6>{});
  else if (vec_ok && chunks <= 8)
    go(std::integral_constant<int, 8>{});
  else
    launched = false;
  if (!launched)
    hipLaunchKernelGGL((rope_commit_generic_kernel<Tag>), dim3(static_cast<unsigned>(rows)),
                       dim3(kBlock), 0, stream, a);
  return launch_status("kv_commit_rope");
}

}  // namespace
}  // namespace jo

using namespace jo;

extern "C" int jo_kv_commit_rope(const void* src_k, const void* src_v, void* dst_k, void* dst_v,
                                 int64_t layers, int64_t batch, int64_t tokens,
                                 int64_t num_heads, int64_t head_dim, int64_t src_layer_stride,
                                 int64_t src_batch_stride, int64_t src_token_stride,
                                 int64_t dst_layer_stride, int64_t dst_batch_stride,
                                 int64_t dst_token_stride, int64_t dst_tokens,
                                 int64_t dst_token_offset, const float* cos, const float* sin, int64_t table_stride,
                                 int64_t table_batch_stride, int dtype, void* stream) {
  const char* op = "kv_commit_rope";
  JO_REQUIRE(dtype == JO_DTYPE_BF16 || dtype == JO_DTYPE_F16, "%s: K/V must be bf16 or fp16", op);
  JO_REQUIRE(layers >= 0 && batch >= 0 && tokens >= 0 && num_heads > 0 && head_dim > 0,
             "%s: bad shape", op);
  JO_REQUIRE(head_dim % 2 == 0, "RoPE requires an even head dimension, got %lld",
             static_cast<long long>(head_dim));
  JO_REQUIRE(num_heads * head_dim <= INT32_MAX / 2, "%s: row too long", op);
  JO_REQUIRE(src_token_stride >= num_heads * head_dim && dst_token_stride >= num_heads * head_dim &&
                 src_layer_stride >= 0 && src_batch_stride >= 0 && dst_layer_stride >= 0 &&
                 dst_batch_stride >= 0 && dst_token_offset >= 0 && table_stride >= head_dim &&
                 table_batch_stride >= 0,
             "%s: bad stride or offset", op);
  JO_REQUIRE(dst_token_offset + tokens <= dst_tokens,
             "%s: tokens %lld at offset %lld exceed the destination's %lld", op,
             static_cast<long long>(tokens), static_cast<long long>(dst_token_offset),
             static_cast<long long>(dst_tokens));
  const int64_t rows = layers * batch * tokens;
  // Zero rows: nothing to read or write (an empty tensor's data pointer may be
  // null, so the V pointer pair is checked only when there is work).
  if (rows == 0) return JO_OK;
  JO_REQUIRE((src_v == nullptr) == (dst_v == nullptr),
             "%s: V needs both a source and a destination", op);
  // Up to two waves of 64 lanes per row: the launch's work-item count must stay
  // below 2^32.
  JO_REQUIRE(rows <= int64_t{UINT32_MAX} / (2 * 64), "%s: too many rows (%lld, at most %lld)", op,
             static_cast<long long>(rows), static_cast<long long>(int64_t{UINT32_MAX} / (2 * 64)));
  JO_REQUIRE(src_k && dst_k && cos && sin, "%s: null pointer", op);
  CommitArgs a{src_k, src_v, dst_k, dst_v, layers, batch, tokens,
               static_cast<int>(num_heads * head_dim), static_cast<int>(head_dim),
               src_layer_stride, src_batch_stride, src_token_stride, dst_layer_stride,
               dst_batch_stride, dst_token_stride, dst_token_offset, cos, sin, table_stride,
               table_batch_stride};
  hipStream_t st = static_cast<hipStream_t>(stream);
  return dtype == JO_DTYPE_BF16 ? launch_commit<BF16>(a, st) : launch_commit<F16>(a, st);
}
