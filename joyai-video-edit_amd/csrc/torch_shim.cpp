// TORCH_LIBRARY(joyomni_ops) registration over the C ABI of libjoyomni_hip.so.
//
// The five reference ops keep their schema strings byte-for-byte
// (deploy/joyomni_ops/csrc/pybind.cpp:35-46) and their TORCH_CHECKs
// (fused_qknorm_rope_3d_kernel.cu:183-200, fused_norm_scale_shift.cu:176-196,
// rmsnorm.cu:77-81, per_token_quant_fp8.cu:149-156, fp8_gemm.cu:1457-1485), so
// torch.ops.joyomni_ops.* behaves as the reference does for callers. The new
// ops (grid RoPE, K ring-cache write, QK with the pre-RoPE K stage,
// add+LayerNorm, RMSNorm->FP8, norm+AdaLN->FP8, KV-pool commit,
// apply_rotary_emb, per-head RMSNorm) have their own names. Tensors on ROCm
// carry the CUDA device type, so the impls are registered on the CUDA
// dispatch key like the reference's. Every op runs
// on the current stream of the tensor's device and never synchronizes.
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/all.h>
#include <torch/library.h>

#include <vector>

#include "joyomni_hip.h"

namespace joyomni_ops {
namespace {

#define JO_CHECK_CUDA(x) TORCH_CHECK((x).is_cuda(), #x " must be a CUDA tensor")
#define JO_CHECK_CONTIGUOUS(x) TORCH_CHECK((x).is_contiguous(), #x " must be contiguous")
#define JO_CHECK_DTYPE(x, dt) \
  TORCH_CHECK((x).scalar_type() == (dt), #x " dtype is ", (x).scalar_type(), ", expected ", (dt))
#define JO_CHECK_INPUT(x, dt) \
  JO_CHECK_CUDA(x);           \
  JO_CHECK_CONTIGUOUS(x);     \
  JO_CHECK_DTYPE(x, dt)

void check_status(int status, const char* op) {
  TORCH_CHECK(status == JO_OK, op, ": ", jo_last_error());
}

// The shim is compiled against include/joyomni_hip.h; a kernel library of
// another ABI version (argument lists differ between versions) is refused at
// the first launch instead of being called with misread arguments.
void check_abi() {
  static const int lib_abi = jo_abi_version();
  TORCH_CHECK(lib_abi == JO_ABI_VERSION, "joyomni_ops: libjoyomni_hip.so has ABI version ",
              lib_abi, ", this _C.so was built for ", JO_ABI_VERSION, "; rebuild both");
}

void* current_stream(const torch::Tensor& t) {
  check_abi();
  return static_cast<void*>(
      c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.get_device()).stream());
}

int dtype_code(const torch::Tensor& t) {
  switch (t.scalar_type()) {
    case torch::kFloat32: return JO_DTYPE_F32;
    case torch::kFloat16: return JO_DTYPE_F16;
    case torch::kBFloat16: return JO_DTYPE_BF16;
    default: TORCH_CHECK(false, "Unsupported dtype; use float32/float16/bfloat16");
  }
  return -1;
}

// Row stride of a 2-D tensor whose last dim is contiguous; a size-1 leading
// dim has no meaningful stride, report the row length instead.
int64_t row_stride(const torch::Tensor& t) { return t.size(0) <= 1 ? t.size(1) : t.stride(0); }

}  // namespace

// ---------------------------------------------------------------------------
// Reference ops.
// ---------------------------------------------------------------------------
void fused_qk_norm_rope_3d_paired(torch::Tensor& q, torch::Tensor& k, int64_t seq_len,
                                  int64_t num_heads, double eps, torch::Tensor& q_weight,
                                  torch::Tensor& k_weight, torch::Tensor& cos,
                                  torch::Tensor& sin) {
  TORCH_CHECK(q.dim() == 3, "q must be 3D [batch, seq_len*num_heads, head_dim]");
  TORCH_CHECK(k.dim() == 3, "k must be 3D [batch, seq_len*num_heads, head_dim]");
  TORCH_CHECK(q.sizes() == k.sizes(), "q and k must have the same shape");
  TORCH_CHECK(q_weight.dim() == 1 && k_weight.dim() == 1, "weights must be 1D [head_dim]");
  TORCH_CHECK(cos.dim() == 2 && sin.dim() == 2, "cos/sin must be 2D [seq_len, head_dim/2]");
  JO_CHECK_INPUT(q, torch::kBFloat16);
  JO_CHECK_INPUT(k, torch::kBFloat16);
  JO_CHECK_INPUT(q_weight, torch::kBFloat16);
  JO_CHECK_INPUT(k_weight, torch::kBFloat16);
  JO_CHECK_INPUT(cos, torch::kBFloat16);
  JO_CHECK_INPUT(sin, torch::kBFloat16);
  const int64_t batch = q.size(0);
  const int64_t head_dim = q.size(2);
  TORCH_CHECK(q.size(1) == seq_len * num_heads, "q.size(1) must equal seq_len*num_heads");
  TORCH_CHECK(q_weight.size(0) == head_dim && k_weight.size(0) == head_dim,
              "weight size must match head_dim");
  TORCH_CHECK(cos.size(0) == seq_len && cos.size(1) == head_dim / 2,
              "cos shape must be [seq_len, head_dim/2]");
  TORCH_CHECK(sin.size(0) == seq_len && sin.size(1) == head_dim / 2,
              "sin shape must be [seq_len, head_dim/2]");
  TORCH_CHECK(head_dim == 64 || head_dim == 128 || head_dim == 256,
              "Unsupported head_dim for fused_qk_norm_rope_3d_paired: ", head_dim);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(q.device());
  const int64_t tok = num_heads * head_dim;
  check_status(jo_fused_qk_norm_rope_3d_paired(
                   q.data_ptr(), k.data_ptr(), batch, seq_len, num_heads, head_dim,
                   seq_len * tok, tok, seq_len * tok, tok, static_cast<float>(eps),
                   q_weight.data_ptr(), k_weight.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                   current_stream(q)),
               "fused_qk_norm_rope_3d_paired");
}

torch::Tensor fused_norm_scale_shift(const torch::Tensor& x,
                                     const c10::optional<torch::Tensor>& gamma_opt,
                                     const c10::optional<torch::Tensor>& beta_opt,
                                     const torch::Tensor& scale, const torch::Tensor& shift,
                                     int64_t norm_type, double eps) {
  JO_CHECK_CUDA(x);
  JO_CHECK_CUDA(scale);
  JO_CHECK_CUDA(shift);
  TORCH_CHECK(x.dim() == 2, "x must be 2D [M, N]");
  TORCH_CHECK(x.stride(-1) == 1, "x last dim must be contiguous");
  const int64_t M = x.size(0), N = x.size(1);
  TORCH_CHECK((N % 4) == 0, "N must be divisible by 4");
  TORCH_CHECK(scale.dim() == 2 && shift.dim() == 2, "scale/shift must be 2D [M, N]");
  TORCH_CHECK(scale.size(0) == M && shift.size(0) == M,
              "scale/shift rows must equal M (per-row modulation)");
  TORCH_CHECK(scale.size(1) == N && shift.size(1) == N, "scale/shift last dim must be N");
  TORCH_CHECK(scale.stride(-1) == 1 && shift.stride(-1) == 1,
              "scale/shift last dim must be contiguous");
  TORCH_CHECK(x.dtype() == scale.dtype() && x.dtype() == shift.dtype(),
              "x/scale/shift dtype must match");
  TORCH_CHECK(norm_type == 0 || norm_type == 1, "norm_type must be 0 (layer) or 1 (rms)");
  const bool has_gamma = gamma_opt.has_value() && gamma_opt->defined();
  const bool has_beta = beta_opt.has_value() && beta_opt->defined();
  if (has_gamma) {
    TORCH_CHECK(gamma_opt->numel() == N, "gamma must be length N");
    TORCH_CHECK(gamma_opt->is_cuda() && gamma_opt->is_contiguous() &&
                    gamma_opt->dtype() == x.dtype(),
                "gamma must be a contiguous CUDA tensor of x's dtype");
  }
  if (has_beta) {
    TORCH_CHECK(beta_opt->numel() == N, "beta must be length N");
    TORCH_CHECK(beta_opt->is_cuda() && beta_opt->is_contiguous() &&
                    beta_opt->dtype() == x.dtype(),
                "beta must be a contiguous CUDA tensor of x's dtype");
  }
  const int dt = dtype_code(x);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  auto y = torch::empty({M, N}, x.options());
  if (M == 0) return y;
  check_status(jo_fused_norm_scale_shift(
                   x.data_ptr(), row_stride(x), has_gamma ? gamma_opt->data_ptr() : nullptr,
                   has_beta ? beta_opt->data_ptr() : nullptr, scale.data_ptr(),
                   row_stride(scale), shift.data_ptr(), row_stride(shift), y.data_ptr(), N, M,
                   N, dt, static_cast<int>(norm_type), static_cast<float>(eps),
                   current_stream(x)),
               "fused_norm_scale_shift");
  return y;
}

torch::Tensor rmsnorm(const torch::Tensor& x, const torch::Tensor& weight, double eps) {
  JO_CHECK_CUDA(x);
  JO_CHECK_CUDA(weight);
  TORCH_CHECK(x.dim() == 2, "x must be 2D [M, N]");
  TORCH_CHECK(x.stride(-1) == 1, "x last dim must be contiguous");
  TORCH_CHECK(weight.dim() == 1 && weight.numel() == x.size(1), "weight must be 1D [N]");
  TORCH_CHECK(x.dtype() == weight.dtype(), "x and weight dtype must match");
  TORCH_CHECK(weight.stride(0) == 1 || weight.numel() <= 1, "weight must be contiguous");
  const int dt = dtype_code(x);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  const int64_t M = x.size(0), N = x.size(1);
  auto out = torch::empty({M, N}, x.options());
  if (M == 0 || N == 0) return out;
  check_status(jo_rmsnorm(x.data_ptr(), row_stride(x), weight.data_ptr(), out.data_ptr(), N, M,
                          N, dt, static_cast<float>(eps), current_stream(x)),
               "rmsnorm");
  return out;
}

// Per-head RMSNorm of a [..., heads, head_dim] view whose last dim is
// contiguous and whose leading dims collapse to one token stride (e.g. the q
// or k slice of a packed [B, L, 3, H, D] qkv tensor). round_first selects the
// torch RMSNorm module's rounding (dit.py:247-249) over the kernel's
// (rmsnorm.cu:57-60). Returns a new contiguous tensor of x's shape.
torch::Tensor rmsnorm_heads(const torch::Tensor& x, const torch::Tensor& weight, double eps,
                            int64_t round_first) {
  JO_CHECK_CUDA(x);
  JO_CHECK_CUDA(weight);
  TORCH_CHECK(x.dim() >= 2, "x must be [..., heads, head_dim]");
  TORCH_CHECK(x.stride(-1) == 1 || x.size(-1) <= 1, "x last dim must be contiguous");
  const int64_t D = x.size(-1), H = x.size(-2);
  TORCH_CHECK(weight.dim() == 1 && weight.numel() == D, "weight must be 1D [head_dim]");
  TORCH_CHECK(x.dtype() == weight.dtype(), "x and weight dtype must match");
  TORCH_CHECK(weight.stride(0) == 1 || weight.numel() <= 1, "weight must be contiguous");
  int64_t tokens = 1, ts = 0, next = -1;
  for (int64_t d = x.dim() - 3; d >= 0; --d) {
    if (x.size(d) == 1) continue;
    if (next < 0) ts = x.stride(d);
    else TORCH_CHECK(x.stride(d) == next, "x leading dims must collapse to one token stride");
    next = x.stride(d) * x.size(d);
    tokens *= x.size(d);
  }
  const int dt = dtype_code(x);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  auto out = torch::empty(x.sizes(), x.options());
  if (out.numel() == 0) return out;
  check_status(jo_rmsnorm_heads(x.data_ptr(), ts, H <= 1 ? D : x.stride(-2), weight.data_ptr(),
                                out.data_ptr(), D, tokens, H, D, dt, static_cast<float>(eps),
                                round_first ? 1 : 0, current_stream(x)),
               "rmsnorm_heads");
  return out;
}

void sgl_per_token_quant_fp8(torch::Tensor input, torch::Tensor output_q,
                             torch::Tensor output_s) {
  JO_CHECK_CUDA(input);
  JO_CHECK_CONTIGUOUS(input);
  JO_CHECK_CUDA(output_q);
  JO_CHECK_CUDA(output_s);
  TORCH_CHECK(input.dim() == 2, "input must be 2D [num_tokens, hidden_dim]");
  const int64_t num_tokens = input.size(0);
  const int64_t hidden_dim = input.size(1);
  TORCH_CHECK(hidden_dim % 4 == 0, "hidden_dim must be divisible by 4, got ", hidden_dim);
  TORCH_CHECK(input.scalar_type() == torch::kBFloat16 || input.scalar_type() == torch::kFloat16,
              "per_token_quant_fp8: input must be bf16 or fp16");
  // Output checks the reference leaves implicit: the kernel writes
  // output_q as a contiguous [num_tokens, hidden_dim] fp8 array and output_s
  // as num_tokens consecutive fp32 values ([M] or [M, 1]).
  TORCH_CHECK(output_q.scalar_type() == at::kFloat8_e4m3fn, "output_q must be float8_e4m3fn");
  TORCH_CHECK(output_q.is_contiguous() && output_q.numel() == input.numel(),
              "output_q must be a contiguous tensor with input's number of elements");
  TORCH_CHECK(output_s.scalar_type() == torch::kFloat32, "output_s must be float32");
  TORCH_CHECK(output_s.is_contiguous() && output_s.numel() == num_tokens,
              "output_s must be a contiguous tensor of num_tokens floats");
  if (num_tokens == 0) return;
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(input.device());
  check_status(jo_sgl_per_token_quant_fp8(input.data_ptr(), dtype_code(input), num_tokens,
                                          hidden_dim, hidden_dim, output_q.data_ptr(),
                                          hidden_dim, output_s.data_ptr<float>(),
                                          current_stream(input)),
               "sgl_per_token_quant_fp8");
}

// ---------------------------------------------------------------------------
// New ops.
// ---------------------------------------------------------------------------
// gelu(input, approximate="tanh") quantized per token as sgl_per_token_quant_fp8
// would quantize it; output_act, when given, receives the activation itself.
void gelu_tanh_quant_fp8(torch::Tensor input, torch::Tensor output_q, torch::Tensor output_s,
                         const c10::optional<torch::Tensor>& output_act) {
  JO_CHECK_CUDA(input);
  JO_CHECK_CUDA(output_q);
  JO_CHECK_CUDA(output_s);
  TORCH_CHECK(input.dim() == 2 && input.stride(-1) == 1,
              "input must be 2D [num_tokens, hidden_dim] with contiguous rows");
  const int64_t num_tokens = input.size(0);
  const int64_t hidden_dim = input.size(1);
  TORCH_CHECK(hidden_dim % 4 == 0, "hidden_dim must be divisible by 4, got ", hidden_dim);
  TORCH_CHECK(input.scalar_type() == torch::kBFloat16 || input.scalar_type() == torch::kFloat16,
              "gelu_tanh_quant_fp8: input must be bf16 or fp16");
  TORCH_CHECK(output_q.scalar_type() == at::kFloat8_e4m3fn, "output_q must be float8_e4m3fn");
  TORCH_CHECK(output_q.is_contiguous() && output_q.numel() == input.numel(),
              "output_q must be a contiguous tensor with input's number of elements");
  TORCH_CHECK(output_s.scalar_type() == torch::kFloat32, "output_s must be float32");
  TORCH_CHECK(output_s.is_contiguous() && output_s.numel() == num_tokens,
              "output_s must be a contiguous tensor of num_tokens floats");
  void* act = nullptr;
  if (output_act.has_value()) {
    const torch::Tensor& a = *output_act;
    JO_CHECK_CUDA(a);
    TORCH_CHECK(a.scalar_type() == input.scalar_type() && a.is_contiguous() &&
                    a.numel() == input.numel(),
                "output_act must be a contiguous tensor of input's dtype and size");
    act = a.data_ptr();
  }
  if (num_tokens == 0) return;
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(input.device());
  check_status(jo_gelu_tanh_quant_fp8(input.data_ptr(), dtype_code(input), num_tokens, hidden_dim,
                                      row_stride(input), output_q.data_ptr(), hidden_dim,
                                      output_s.data_ptr<float>(), act, hidden_dim,
                                      current_stream(input)),
               "gelu_tanh_quant_fp8");
}
// ---------------------------------------------------------------------------
namespace {

struct QKGeom {
  int64_t batch, seq_len, num_heads, head_dim;
  int64_t q_bs, q_ts, k_bs, k_ts;  // batch / token strides in elements
};

// Batch and token strides of a q/k tensor: either [B, seq_len*num_heads, D]
// contiguous (the paired op's layout) or a [B, seq_len, num_heads, D] view
// whose heads are contiguous within a token (e.g. q = qkv[:, :, 0] of a
// packed [B, L, 3, H, D] projection).
void qk_strides(const torch::Tensor& t, int64_t seq_len, int64_t num_heads, int64_t head_dim,
                const char* name, int64_t* bs, int64_t* ts) {
  if (t.dim() == 3) {
    TORCH_CHECK(t.is_contiguous(), name, " must be contiguous when 3D");
    TORCH_CHECK(t.size(1) == seq_len * num_heads, name, ".size(1) must equal seq_len*num_heads");
    *bs = seq_len * num_heads * head_dim;
    *ts = num_heads * head_dim;
  } else {
    TORCH_CHECK(t.dim() == 4 && t.size(1) == seq_len && t.size(2) == num_heads,
                name, " must be [B, seq_len*num_heads, D] or [B, seq_len, num_heads, D]");
    TORCH_CHECK(t.stride(3) == 1 && t.stride(2) == head_dim,
                name, ": heads of a token must be contiguous");
    *bs = t.size(0) == 1 ? seq_len * t.stride(1) : t.stride(0);
    *ts = seq_len == 1 ? num_heads * head_dim : t.stride(1);
  }
}

QKGeom check_qk_views(const torch::Tensor& q, const torch::Tensor& k, int64_t seq_len,
                      int64_t num_heads, const torch::Tensor& q_weight,
                      const torch::Tensor& k_weight) {
  TORCH_CHECK(q.dim() == 3 || q.dim() == 4, "q must be 3D or 4D");
  TORCH_CHECK(q.sizes() == k.sizes(), "q and k must have the same shape");
  JO_CHECK_CUDA(q);
  JO_CHECK_CUDA(k);
  JO_CHECK_DTYPE(q, torch::kBFloat16);
  JO_CHECK_DTYPE(k, torch::kBFloat16);
  JO_CHECK_INPUT(q_weight, torch::kBFloat16);
  JO_CHECK_INPUT(k_weight, torch::kBFloat16);
  const int64_t head_dim = q.size(q.dim() - 1);
  TORCH_CHECK(q_weight.numel() == head_dim && k_weight.numel() == head_dim,
              "weight size must match head_dim");
  TORCH_CHECK(head_dim == 64 || head_dim == 128 || head_dim == 256,
              "Unsupported head_dim: ", head_dim);
  QKGeom g{q.size(0), seq_len, num_heads, head_dim, 0, 0, 0, 0};
  qk_strides(q, seq_len, num_heads, head_dim, "q", &g.q_bs, &g.q_ts);
  qk_strides(k, seq_len, num_heads, head_dim, "k", &g.k_bs, &g.k_ts);
  return g;
}

// The pre-RoPE K output of the *_kstage ops: [B, seq_len*H, D] contiguous or
// a [B, seq_len, H, D] view with contiguous heads; returns its strides.
std::pair<int64_t, int64_t> stage_strides(const torch::Tensor& k_stage, const QKGeom& g) {
  JO_CHECK_CUDA(k_stage);
  JO_CHECK_DTYPE(k_stage, torch::kBFloat16);
  TORCH_CHECK(k_stage.dim() >= 3 && k_stage.size(0) == g.batch &&
                  k_stage.size(k_stage.dim() - 1) == g.head_dim,
              "k_stage must be [B, seq_len*num_heads, D] or [B, seq_len, num_heads, D]");
  int64_t bs = 0, ts = 0;
  qk_strides(k_stage, g.seq_len, g.num_heads, g.head_dim, "k_stage", &bs, &ts);
  return {bs, ts};
}

QKGeom check_qk_common(const torch::Tensor& q, const torch::Tensor& k, int64_t seq_len,
                       int64_t num_heads, const torch::Tensor& q_weight,
                       const torch::Tensor& k_weight, const torch::Tensor& freqs) {
  const QKGeom g = check_qk_views(q, k, seq_len, num_heads, q_weight, k_weight);
  TORCH_CHECK(freqs.device().is_cpu(),
              "freqs must be a CPU tensor (its values are passed in the kernel arguments)");
  JO_CHECK_CONTIGUOUS(freqs);
  JO_CHECK_DTYPE(freqs, torch::kFloat32);
  TORCH_CHECK(freqs.dim() == 2 && freqs.size(0) == 2 && freqs.size(1) == g.head_dim / 2,
              "freqs must be [2, head_dim/2] float32");
  return g;
}

}  // namespace

void fused_qk_norm_rope_3d_grid(torch::Tensor& q, torch::Tensor& k, int64_t seq_len,
                                int64_t num_heads, double eps, torch::Tensor& q_weight,
                                torch::Tensor& k_weight, torch::Tensor& freqs, int64_t pairs_t,
                                int64_t pairs_h, int64_t grid_h, int64_t grid_w, int64_t t0,
                                double source_id) {
  const QKGeom g = check_qk_common(q, k, seq_len, num_heads, q_weight, k_weight, freqs);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(q.device());
  check_status(jo_fused_qk_norm_rope_3d_grid(
                   q.data_ptr(), k.data_ptr(), g.batch, g.seq_len, g.num_heads, g.head_dim,
                   g.q_bs, g.q_ts, g.k_bs, g.k_ts, static_cast<float>(eps),
                   q_weight.data_ptr(), k_weight.data_ptr(), freqs.data_ptr<float>(),
                   static_cast<int32_t>(pairs_t), static_cast<int32_t>(pairs_h),
                   static_cast<int32_t>(grid_h), static_cast<int32_t>(grid_w),
                   static_cast<int32_t>(t0), static_cast<float>(source_id), current_stream(q)),
               "fused_qk_norm_rope_3d_grid");
}

void fused_qk_norm_rope_3d_grid_kstage(torch::Tensor& q, torch::Tensor& k, torch::Tensor& k_stage,
                                       int64_t seq_len, int64_t num_heads, double eps,
                                       torch::Tensor& q_weight, torch::Tensor& k_weight,
                                       torch::Tensor& freqs, int64_t pairs_t, int64_t pairs_h,
                                       int64_t grid_h, int64_t grid_w, int64_t t0,
                                       double source_id) {
  const QKGeom g = check_qk_common(q, k, seq_len, num_heads, q_weight, k_weight, freqs);
  const auto st = stage_strides(k_stage, g);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(q.device());
  check_status(jo_fused_qk_norm_rope_3d_grid_kstage(
                   q.data_ptr(), k.data_ptr(), k_stage.data_ptr(), g.batch, g.seq_len,
                   g.num_heads, g.head_dim, g.q_bs, g.q_ts, g.k_bs, g.k_ts, st.first, st.second,
                   static_cast<float>(eps), q_weight.data_ptr(), k_weight.data_ptr(),
                   freqs.data_ptr<float>(), static_cast<int32_t>(pairs_t),
                   static_cast<int32_t>(pairs_h), static_cast<int32_t>(grid_h),
                   static_cast<int32_t>(grid_w), static_cast<int32_t>(t0),
                   static_cast<float>(source_id), current_stream(q)),
               "fused_qk_norm_rope_3d_grid_kstage");
}

void fused_qk_norm_rope_3d_paired_kstage(torch::Tensor& q, torch::Tensor& k,
                                         torch::Tensor& k_stage, int64_t seq_len,
                                         int64_t num_heads, double eps, torch::Tensor& q_weight,
                                         torch::Tensor& k_weight, torch::Tensor& cos,
                                         torch::Tensor& sin) {
  const QKGeom g = check_qk_views(q, k, seq_len, num_heads, q_weight, k_weight);
  JO_CHECK_INPUT(cos, torch::kBFloat16);
  JO_CHECK_INPUT(sin, torch::kBFloat16);
  TORCH_CHECK(cos.dim() == 2 && sin.dim() == 2 && cos.size(0) == seq_len &&
                  sin.size(0) == seq_len && cos.size(1) == g.head_dim / 2 &&
                  sin.size(1) == g.head_dim / 2,
              "cos/sin must be [seq_len, head_dim/2]");
  const auto st = stage_strides(k_stage, g);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(q.device());
  check_status(jo_fused_qk_norm_rope_3d_paired_kstage(
                   q.data_ptr(), k.data_ptr(), k_stage.data_ptr(), g.batch, g.seq_len,
                   g.num_heads, g.head_dim, g.q_bs, g.q_ts, g.k_bs, g.k_ts, st.first, st.second,
                   static_cast<float>(eps), q_weight.data_ptr(), k_weight.data_ptr(),
                   cos.data_ptr(), sin.data_ptr(), current_stream(q)),
               "fused_qk_norm_rope_3d_paired_kstage");
}

void fused_qk_norm_rope_3d_kvcache(torch::Tensor& q, const torch::Tensor& k,
                                   torch::Tensor& k_cache, int64_t seq_len, int64_t num_heads,
                                   double eps, const torch::Tensor& q_weight,
                                   const torch::Tensor& k_weight, const torch::Tensor& freqs,
                                   int64_t pairs_t, int64_t pairs_h, int64_t grid_h,
                                   int64_t grid_w, int64_t t0, double source_id,
                                   int64_t slot_start) {
  const QKGeom g = check_qk_common(q, k, seq_len, num_heads, q_weight, k_weight, freqs);
  JO_CHECK_INPUT(k_cache, torch::kBFloat16);
  TORCH_CHECK(k_cache.dim() == 3 && k_cache.size(0) == g.batch && k_cache.size(2) == g.head_dim,
              "k_cache must be [batch, cache_tokens*num_heads, head_dim]");
  TORCH_CHECK(grid_h > 0 && grid_w > 0, "grid_h and grid_w must be positive");
  const int64_t frame_tokens = grid_h * grid_w;
  TORCH_CHECK(k_cache.size(1) % (frame_tokens * num_heads) == 0,
              "k_cache token count must be a whole number of frames");
  const int64_t cache_slots = k_cache.size(1) / (frame_tokens * num_heads);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(q.device());
  const int64_t tok = g.num_heads * g.head_dim;
  check_status(jo_fused_qk_norm_rope_3d_kvcache(
                   q.data_ptr(), k.data_ptr(), k_cache.data_ptr(), g.batch, g.seq_len,
                   g.num_heads, g.head_dim, g.q_bs, g.q_ts, g.k_bs, g.k_ts,
                   k_cache.size(1) * g.head_dim, tok, cache_slots, slot_start,
                   static_cast<float>(eps), q_weight.data_ptr(), k_weight.data_ptr(),
                   freqs.data_ptr<float>(), static_cast<int32_t>(pairs_t),
                   static_cast<int32_t>(pairs_h), static_cast<int32_t>(grid_h),
                   static_cast<int32_t>(grid_w), static_cast<int32_t>(t0),
                   static_cast<float>(source_id), current_stream(q)),
               "fused_qk_norm_rope_3d_kvcache");
}

namespace {
// A modulation tensor (gate, scale, shift) of the fused norm ops: [N] (one
// row for every row of x: stride 0), [M, N] (a row each) or [B, N] with B
// dividing M (one row per sample of M / B consecutive rows). Returns its row
// stride and records how many rows of x each of its rows serves in *group
// (every modulation tensor with its own rows must agree).
int64_t mod_stride(const torch::Tensor& t, int64_t M, int64_t N, const char* name,
                   int64_t* group) {
  JO_CHECK_CUDA(t);
  if (t.dim() == 1 || (t.dim() == 2 && t.size(0) == 1)) {
    TORCH_CHECK(t.size(t.dim() - 1) == N && t.stride(t.dim() - 1) == 1, name,
                " must be [N] contiguous");
    return 0;
  }
  TORCH_CHECK(t.dim() == 2 && t.size(1) == N && t.stride(1) == 1 &&
                  (t.size(0) == M || (t.size(0) > 0 && M % t.size(0) == 0)),
              name, " must be [N], [M, N] or [B, N] (B dividing M) with a contiguous last dim");
  const int64_t g = t.size(0) == M ? 1 : M / t.size(0);
  TORCH_CHECK(*group == 0 || *group == g, name,
              ": gate / scale / shift with rows of their own must have the same row count");
  *group = g;
  return row_stride(t);
}
}  // namespace

torch::Tensor fused_add_layernorm_scale_shift(const torch::Tensor& x, torch::Tensor& residual,
                                              const c10::optional<torch::Tensor>& gate_opt,
                                              const c10::optional<torch::Tensor>& gamma_opt,
                                              const c10::optional<torch::Tensor>& beta_opt,
                                              const torch::Tensor& scale,
                                              const torch::Tensor& shift, double eps) {
  JO_CHECK_CUDA(x);
  JO_CHECK_CUDA(residual);
  TORCH_CHECK(x.dim() == 2 && x.stride(-1) == 1, "x must be 2D [M, N] with contiguous rows");
  TORCH_CHECK(residual.sizes() == x.sizes() && residual.stride(-1) == 1,
              "residual must match x");
  const int64_t M = x.size(0), N = x.size(1);
  TORCH_CHECK(N % 4 == 0, "N must be divisible by 4");
  TORCH_CHECK(residual.dtype() == x.dtype() && scale.dtype() == x.dtype() &&
                  shift.dtype() == x.dtype(),
              "x/residual/scale/shift dtype must match");
  int64_t group = 0;
  const int64_t sc_stride = mod_stride(scale, M, N, "scale", &group);
  const int64_t sh_stride = mod_stride(shift, M, N, "shift", &group);
  const bool has_gate = gate_opt.has_value() && gate_opt->defined();
  int64_t g_stride = 0;
  if (has_gate) {
    TORCH_CHECK(gate_opt->dtype() == x.dtype(), "gate dtype must match x");
    g_stride = mod_stride(*gate_opt, M, N, "gate", &group);
  }
  const bool has_gamma = gamma_opt.has_value() && gamma_opt->defined();
  const bool has_beta = beta_opt.has_value() && beta_opt->defined();
  if (has_gamma)
    TORCH_CHECK(gamma_opt->numel() == N && gamma_opt->is_contiguous() &&
                    gamma_opt->dtype() == x.dtype(),
                "gamma must be [N] contiguous of x's dtype");
  if (has_beta)
    TORCH_CHECK(beta_opt->numel() == N && beta_opt->is_contiguous() &&
                    beta_opt->dtype() == x.dtype(),
                "beta must be [N] contiguous of x's dtype");
  const int dt = dtype_code(x);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  auto y = torch::empty({M, N}, x.options());
  if (M == 0) return y;
  check_status(jo_fused_add_layernorm_scale_shift(
                   x.data_ptr(), row_stride(x), residual.data_ptr(), row_stride(residual),
                   has_gate ? gate_opt->data_ptr() : nullptr, g_stride,
                   has_gamma ? gamma_opt->data_ptr() : nullptr,
                   has_beta ? beta_opt->data_ptr() : nullptr, scale.data_ptr(), sc_stride,
                   shift.data_ptr(), sh_stride, group > 0 ? group : 1, y.data_ptr(), N, M, N, dt,
                   static_cast<float>(eps), current_stream(x)),
               "fused_add_layernorm_scale_shift");
  return y;
}

// fused_norm_scale_shift with scale / shift of [N], [M, N] or [B, N] (B
// dividing M: one row per sample of M / B consecutive rows of x), read in
// place: the per-sample AdaLN vectors of a [B, L, D] batch without the
// [B * L, D] copies the reference's caller makes (sgl_fused_ops.py:44-51).
torch::Tensor fused_norm_scale_shift_per_sample(const torch::Tensor& x,
                                                const c10::optional<torch::Tensor>& gamma_opt,
                                                const c10::optional<torch::Tensor>& beta_opt,
                                                const torch::Tensor& scale,
                                                const torch::Tensor& shift, int64_t norm_type,
                                                double eps) {
  JO_CHECK_CUDA(x);
  TORCH_CHECK(x.dim() == 2 && x.stride(-1) == 1, "x must be 2D [M, N] with contiguous rows");
  const int64_t M = x.size(0), N = x.size(1);
  TORCH_CHECK(N % 4 == 0, "N must be divisible by 4");
  TORCH_CHECK(scale.dtype() == x.dtype() && shift.dtype() == x.dtype(),
              "x/scale/shift dtype must match");
  TORCH_CHECK(norm_type == 0 || norm_type == 1, "norm_type must be 0 (layer) or 1 (rms)");
  int64_t group = 0;
  const int64_t sc_stride = mod_stride(scale, M, N, "scale", &group);
  const int64_t sh_stride = mod_stride(shift, M, N, "shift", &group);
  const bool has_gamma = gamma_opt.has_value() && gamma_opt->defined();
  const bool has_beta = beta_opt.has_value() && beta_opt->defined();
  if (has_gamma)
    TORCH_CHECK(gamma_opt->is_cuda() && gamma_opt->numel() == N && gamma_opt->is_contiguous() &&
                    gamma_opt->dtype() == x.dtype(),
                "gamma must be [N] contiguous of x's dtype");
  if (has_beta)
    TORCH_CHECK(beta_opt->is_cuda() && beta_opt->numel() == N && beta_opt->is_contiguous() &&
                    beta_opt->dtype() == x.dtype(),
                "beta must be [N] contiguous of x's dtype");
  const int dt = dtype_code(x);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  auto y = torch::empty({M, N}, x.options());
  if (M == 0) return y;
  check_status(jo_fused_norm_scale_shift_per_sample(
                   x.data_ptr(), row_stride(x), has_gamma ? gamma_opt->data_ptr() : nullptr,
                   has_beta ? beta_opt->data_ptr() : nullptr, scale.data_ptr(), sc_stride,
                   shift.data_ptr(), sh_stride, group > 0 ? group : 1, y.data_ptr(), N, M, N, dt,
                   static_cast<int>(norm_type), static_cast<float>(eps), current_stream(x)),
               "fused_norm_scale_shift_per_sample");
  return y;
}

void rmsnorm_quant_fp8(const torch::Tensor& x, const torch::Tensor& weight, double eps,
                       torch::Tensor output_q, torch::Tensor output_s, int64_t group_size) {
  JO_CHECK_CUDA(x);
  JO_CHECK_CUDA(weight);
  JO_CHECK_CUDA(output_q);
  JO_CHECK_CUDA(output_s);
  TORCH_CHECK(x.dim() == 2 && x.stride(-1) == 1, "x must be 2D [M, N] with contiguous rows");
  const int64_t M = x.size(0), N = x.size(1);
  TORCH_CHECK(x.scalar_type() == torch::kBFloat16 || x.scalar_type() == torch::kFloat16,
              "x must be bf16 or fp16");
  TORCH_CHECK(weight.dtype() == x.dtype() && weight.numel() == N && weight.is_contiguous(),
              "weight must be [N] contiguous of x's dtype");
  TORCH_CHECK(group_size == 0 || group_size == 128, "group_size must be 0 or 128");
  TORCH_CHECK(output_q.scalar_type() == at::kFloat8_e4m3fn && output_q.is_contiguous() &&
                  output_q.numel() == M * N,
              "output_q must be a contiguous float8_e4m3fn tensor with M*N elements");
  const int64_t ns = group_size == 0 ? M : (N % 128 == 0 ? M * (N / 128) : -1);
  TORCH_CHECK(output_s.scalar_type() == torch::kFloat32 && output_s.is_contiguous() &&
                  output_s.numel() == ns,
              "output_s must be contiguous float32 with M (per-token) or M*N/128 elements");
  if (M == 0) return;
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  check_status(jo_rmsnorm_quant_fp8(x.data_ptr(), row_stride(x), weight.data_ptr(),
                                    output_q.data_ptr(), N, output_s.data_ptr<float>(), M, N,
                                    dtype_code(x), static_cast<float>(eps), group_size,
                                    current_stream(x)),
               "rmsnorm_quant_fp8");
}

void norm_scale_shift_quant_fp8(const torch::Tensor& x,
                                const c10::optional<torch::Tensor>& residual_opt,
                                const c10::optional<torch::Tensor>& gate_opt,
                                const c10::optional<torch::Tensor>& gamma_opt,
                                const c10::optional<torch::Tensor>& beta_opt,
                                const torch::Tensor& scale, const torch::Tensor& shift,
                                int64_t norm_type, double eps, torch::Tensor output_q,
                                torch::Tensor output_s) {
  JO_CHECK_CUDA(x);
  JO_CHECK_CUDA(output_q);
  JO_CHECK_CUDA(output_s);
  TORCH_CHECK(x.dim() == 2 && x.stride(-1) == 1, "x must be 2D [M, N] with contiguous rows");
  TORCH_CHECK(x.scalar_type() == torch::kBFloat16 || x.scalar_type() == torch::kFloat16,
              "x must be bf16 or fp16");
  TORCH_CHECK(norm_type == 0 || norm_type == 1, "norm_type must be 0 (layer) or 1 (rms)");
  const int64_t M = x.size(0), N = x.size(1);
  TORCH_CHECK(N % 4 == 0, "N must be divisible by 4");
  TORCH_CHECK(scale.dtype() == x.dtype() && shift.dtype() == x.dtype(),
              "x/scale/shift dtype must match");
  int64_t group = 0;
  const int64_t sc_stride = mod_stride(scale, M, N, "scale", &group);
  const int64_t sh_stride = mod_stride(shift, M, N, "shift", &group);
  const bool has_res = residual_opt.has_value() && residual_opt->defined();
  if (has_res) {
    JO_CHECK_CUDA(*residual_opt);
    TORCH_CHECK(residual_opt->sizes() == x.sizes() && residual_opt->stride(-1) == 1 &&
                    residual_opt->dtype() == x.dtype(),
                "residual must match x");
  }
  const bool has_gate = gate_opt.has_value() && gate_opt->defined();
  TORCH_CHECK(!has_gate || has_res, "a gate needs a residual");
  int64_t g_stride = 0;
  if (has_gate) {
    TORCH_CHECK(gate_opt->dtype() == x.dtype(), "gate dtype must match x");
    g_stride = mod_stride(*gate_opt, M, N, "gate", &group);
  }
  const bool has_gamma = gamma_opt.has_value() && gamma_opt->defined();
  const bool has_beta = beta_opt.has_value() && beta_opt->defined();
  if (has_gamma)
    TORCH_CHECK(gamma_opt->numel() == N && gamma_opt->is_contiguous() &&
                    gamma_opt->dtype() == x.dtype(),
                "gamma must be [N] contiguous of x's dtype");
  if (has_beta)
    TORCH_CHECK(beta_opt->numel() == N && beta_opt->is_contiguous() &&
                    beta_opt->dtype() == x.dtype(),
                "beta must be [N] contiguous of x's dtype");
  TORCH_CHECK(output_q.scalar_type() == at::kFloat8_e4m3fn && output_q.is_contiguous() &&
                  output_q.numel() == M * N,
              "output_q must be a contiguous float8_e4m3fn tensor with M*N elements");
  TORCH_CHECK(output_s.scalar_type() == torch::kFloat32 && output_s.is_contiguous() &&
                  output_s.numel() == M,
              "output_s must be contiguous float32 with M elements");
  if (M == 0) return;
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  check_status(jo_norm_scale_shift_quant_fp8(
                   x.data_ptr(), row_stride(x), has_res ? residual_opt->data_ptr() : nullptr,
                   has_res ? row_stride(*residual_opt) : 0,
                   has_gate ? gate_opt->data_ptr() : nullptr, g_stride,
                   has_gamma ? gamma_opt->data_ptr() : nullptr,
                   has_beta ? beta_opt->data_ptr() : nullptr, scale.data_ptr(), sc_stride,
                   shift.data_ptr(), sh_stride, group > 0 ? group : 1, output_q.data_ptr(), N,
                   output_s.data_ptr<float>(), M, N, dtype_code(x),
                   static_cast<int>(norm_type), static_cast<float>(eps), current_stream(x)),
               "norm_scale_shift_quant_fp8");
}

namespace {
// Strides of a [B, T, H, D] (L = 1) or [L, B, T, H, D] K/V tensor whose
// heads are contiguous per token: {layer, batch, token} in elements.
struct KVLayout {
  int64_t L, B, T, H, D, ls, bs, ts;
};
KVLayout kv_layout(const torch::Tensor& t, const char* name) {
  JO_CHECK_CUDA(t);
  TORCH_CHECK(t.dim() == 4 || t.dim() == 5, name, " must be [B, T, H, D] or [L, B, T, H, D]");
  TORCH_CHECK(t.scalar_type() == torch::kBFloat16 || t.scalar_type() == torch::kFloat16, name,
              " must be bf16 or fp16");
  const int64_t o = t.dim() - 4;
  KVLayout k{o ? t.size(0) : 1, t.size(o), t.size(o + 1), t.size(o + 2), t.size(o + 3),
             o ? t.stride(0) : 0, t.stride(o), t.stride(o + 1)};
  TORCH_CHECK(t.stride(-1) == 1 && (k.H <= 1 || t.stride(-2) == k.D), name,
              " must have contiguous heads per token");
  return k;
}
// Table batch stride for fp32 [T, D] / [1, T, D] (shared) or [B, T, D] tables.
int64_t table_batch_stride(const torch::Tensor& c, int64_t B, int64_t T, int64_t D,
                           const char* name) {
  JO_CHECK_CUDA(c);
  TORCH_CHECK(c.scalar_type() == torch::kFloat32 && c.is_contiguous(), name,
              " must be a contiguous float32 table");
  if (c.numel() == T * D) return 0;
  TORCH_CHECK(c.numel() == B * T * D, name, " must hold [T, D] or [B, T, D] values");
  return T * D;
}
}  // namespace

void kv_commit_rope(const torch::Tensor& src_k, const c10::optional<torch::Tensor>& src_v_opt,
                    torch::Tensor dst_k, const c10::optional<torch::Tensor>& dst_v_opt,
                    int64_t dst_offset, const torch::Tensor& cos, const torch::Tensor& sin) {
  const KVLayout s = kv_layout(src_k, "src_k");
  const KVLayout d = kv_layout(dst_k, "dst_k");
  TORCH_CHECK(src_k.dim() == dst_k.dim() && s.L == d.L && s.B == d.B && s.H == d.H && s.D == d.D,
              "src_k and dst_k must agree in layers, batch and heads");
  TORCH_CHECK(dst_k.scalar_type() == src_k.scalar_type(), "dst_k dtype must match src_k");
  TORCH_CHECK(dst_offset >= 0 && dst_offset + s.T <= d.T,
              "dst_offset + tokens must fit in dst_k's token dim");
  const bool has_v = src_v_opt.has_value() && src_v_opt->defined();
  TORCH_CHECK(has_v == (dst_v_opt.has_value() && dst_v_opt->defined()),
              "src_v and dst_v go together");
  if (has_v) {
    const KVLayout sv = kv_layout(*src_v_opt, "src_v");
    const KVLayout dv = kv_layout(*dst_v_opt, "dst_v");
    TORCH_CHECK(src_v_opt->sizes() == src_k.sizes() && dst_v_opt->sizes() == dst_k.sizes() &&
                    sv.ls == s.ls && sv.bs == s.bs && sv.ts == s.ts && dv.ls == d.ls &&
                    dv.bs == d.bs && dv.ts == d.ts &&
                    src_v_opt->scalar_type() == src_k.scalar_type() &&
                    dst_v_opt->scalar_type() == src_k.scalar_type(),
                "V tensors must have the shapes, strides and dtype of the K tensors");
  }
  const int64_t tbs = table_batch_stride(cos, s.B, s.T, s.D, "cos");
  TORCH_CHECK(table_batch_stride(sin, s.B, s.T, s.D, "sin") == tbs, "cos and sin must match");
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(src_k.device());
  check_status(jo_kv_commit_rope(src_k.data_ptr(), has_v ? src_v_opt->data_ptr() : nullptr,
                                 dst_k.data_ptr(), has_v ? dst_v_opt->data_ptr() : nullptr, s.L,
                                 s.B, s.T, s.H, s.D, s.ls, s.bs, s.ts, d.ls, d.bs, d.ts, d.T,
                                 dst_offset, cos.data_ptr<float>(), sin.data_ptr<float>(), s.D,
                                 tbs, dtype_code(src_k), current_stream(src_k)),
               "kv_commit_rope");
}

torch::Tensor apply_rotary_emb(const torch::Tensor& x, const torch::Tensor& cos,
                               const torch::Tensor& sin) {
  TORCH_CHECK(x.dim() == 4, "x must be [B, T, H, D]");
  const KVLayout s = kv_layout(x, "x");
  auto out = torch::empty({s.B, s.T, s.H, s.D}, x.options());
  const int64_t tbs = table_batch_stride(cos, s.B, s.T, s.D, "cos");
  TORCH_CHECK(table_batch_stride(sin, s.B, s.T, s.D, "sin") == tbs, "cos and sin must match");
  if (out.numel() == 0) return out;
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  check_status(jo_kv_commit_rope(x.data_ptr(), nullptr, out.data_ptr(), nullptr, 1, s.B, s.T,
                                 s.H, s.D, 0, s.bs, s.ts, 0, s.T * s.H * s.D, s.H * s.D, s.T, 0,
                                 cos.data_ptr<float>(), sin.data_ptr<float>(), s.D, tbs,
                                 dtype_code(x), current_stream(x)),
               "apply_rotary_emb");
  return out;
}

// Checks of fp8_gemm.cu:1457-1485 (messages verbatim), plus the leading
// dimensions the kernel needs (multiples of 16 bytes).
torch::Tensor fp8_scaled_mm(const torch::Tensor& mat_a, const torch::Tensor& mat_b,
                            const torch::Tensor& scales_a, const torch::Tensor& scales_b,
                            c10::ScalarType out_dtype, const c10::optional<torch::Tensor>& bias) {
  TORCH_CHECK(mat_a.is_cuda(), "mat_a must be a CUDA tensor");
  TORCH_CHECK(mat_b.is_cuda(), "mat_b must be a CUDA tensor");
  TORCH_CHECK(mat_a.dim() == 2, "mat_a must be a 2D tensor");
  TORCH_CHECK(mat_b.dim() == 2, "mat_b must be a 2D tensor");
  TORCH_CHECK(mat_a.stride(1) == 1, "mat_a must be a row major tensor");
  TORCH_CHECK(mat_b.stride(0) == 1, "mat_b must be a column major tensor");
  TORCH_CHECK(mat_a.size(1) == mat_b.size(0), "mat_a and mat_b shapes cannot be multiplied");
  TORCH_CHECK((mat_a.size(1) * mat_a.element_size()) % 16 == 0,
              "mat_a must be multiple of 16 bytes for memory alignment");
  TORCH_CHECK((mat_b.size(0) * mat_b.element_size()) % 16 == 0,
              "mat_b must be multiple of 16 bytes for memory alignment");
  TORCH_CHECK(mat_a.scalar_type() == torch::kFloat8_e4m3fn, "mat_a must be Float8_e4m3fn");
  TORCH_CHECK(mat_b.scalar_type() == torch::kFloat8_e4m3fn, "mat_b must be Float8_e4m3fn");
  TORCH_CHECK(out_dtype == torch::kHalf || out_dtype == torch::kBFloat16,
              "out_dtype must be Half or BFloat16");
  TORCH_CHECK(scales_a.numel() == mat_a.size(0), "size of scales_a is not matched");
  TORCH_CHECK(scales_b.numel() == mat_b.size(1), "size of scales_b is not matched");
  TORCH_CHECK(scales_a.is_contiguous(), "scales_a must be contiguous");
  TORCH_CHECK(scales_b.is_contiguous(), "scales_b msut be contiguous");
  TORCH_CHECK(scales_a.scalar_type() == torch::kFloat32, "scales_a must be Float32");
  TORCH_CHECK(scales_b.scalar_type() == torch::kFloat32, "scales_b must be Float32");
  const bool has_bias = bias.has_value() && bias->defined();
  if (has_bias) {
    TORCH_CHECK(bias->numel() == mat_b.size(1), "size of bias is not matched");
    TORCH_CHECK(bias->is_contiguous(), "bias must be contiguous");
    TORCH_CHECK(bias->dtype() == out_dtype, "bias dtype must match output dtype");
  }
  const int64_t M = mat_a.size(0), K = mat_a.size(1), N = mat_b.size(1);
  const int64_t lda = M <= 1 ? K : mat_a.stride(0);
  const int64_t ldb = N <= 1 ? K : mat_b.stride(1);
  TORCH_CHECK(lda % 16 == 0 && ldb % 16 == 0,
              "mat_a / mat_b leading dimensions must be multiples of 16 bytes");
  torch::Tensor out = torch::empty({M, N}, mat_a.options().dtype(out_dtype));
  TORCH_CHECK((out.size(1) * out.element_size()) % 16 == 0,
              "out must be multiple of 16 bytes for memory alignment");
  if (M == 0 || N == 0) return out;
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(mat_a.device());
  // A split-K workspace when the library would use one (few rows, long K),
  // from the caching allocator on this stream (so also under graph capture);
  // it goes back to the cache when this call returns, stream-ordered.
  const int64_t ws_bytes = jo_fp8_scaled_mm_workspace_bytes(M, N, K);
  torch::Tensor ws;
  if (ws_bytes > 0) ws = torch::empty({ws_bytes}, mat_a.options().dtype(torch::kUInt8));
  check_status(jo_fp8_scaled_mm_ws(mat_a.data_ptr(), lda, mat_b.data_ptr(), ldb,
                                   scales_a.data_ptr<float>(), scales_b.data_ptr<float>(),
                                   has_bias ? bias->data_ptr() : nullptr, out.data_ptr(), N, M, N,
                                   K, out_dtype == torch::kBFloat16 ? JO_DTYPE_BF16 : JO_DTYPE_F16,
                                   ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes,
                                   current_stream(mat_a)),
               "fp8_scaled_mm");
  return out;
}

}  // namespace joyomni_ops

TORCH_LIBRARY(joyomni_ops, m) {
  // Reference schemas (deploy/joyomni_ops/csrc/pybind.cpp:35-43), unchanged.
  m.def(
      "fused_qk_norm_rope_3d_paired(Tensor! q, Tensor! k, int seq_len, int num_heads, float eps, "
      "Tensor q_weight, Tensor k_weight, Tensor cos, Tensor sin) -> ()");
  m.def(
      "fused_norm_scale_shift(Tensor x, Tensor? gamma_opt, Tensor? beta_opt, "
      "Tensor scale, Tensor shift, int norm_type, float eps) -> Tensor");
  m.def("rmsnorm(Tensor x, Tensor weight, float eps) -> Tensor");
  m.def("sgl_per_token_quant_fp8(Tensor input, Tensor! output_q, Tensor! output_s) -> ()");
  m.def(
      "fp8_scaled_mm(Tensor mat_a, Tensor mat_b, Tensor scales_a, Tensor scales_b, "
      "ScalarType out_dtype, Tensor? bias) -> Tensor");
  // New ops.
  m.def(
      "fused_qk_norm_rope_3d_grid(Tensor! q, Tensor! k, int seq_len, int num_heads, float eps, "
      "Tensor q_weight, Tensor k_weight, Tensor freqs, int pairs_t, int pairs_h, int grid_h, "
      "int grid_w, int t0, float source_id) -> ()");
  m.def(
      "fused_qk_norm_rope_3d_paired_kstage(Tensor! q, Tensor! k, Tensor! k_stage, int seq_len, "
      "int num_heads, float eps, Tensor q_weight, Tensor k_weight, Tensor cos, Tensor sin) -> ()");
  m.def(
      "fused_qk_norm_rope_3d_grid_kstage(Tensor! q, Tensor! k, Tensor! k_stage, int seq_len, "
      "int num_heads, float eps, Tensor q_weight, Tensor k_weight, Tensor freqs, int pairs_t, "
      "int pairs_h, int grid_h, int grid_w, int t0, float source_id) -> ()");
  m.def(
      "fused_qk_norm_rope_3d_kvcache(Tensor! q, Tensor k, Tensor! k_cache, int seq_len, "
      "int num_heads, float eps, Tensor q_weight, Tensor k_weight, Tensor freqs, int pairs_t, "
      "int pairs_h, int grid_h, int grid_w, int t0, float source_id, int slot_start) -> ()");
  m.def(
      "fused_add_layernorm_scale_shift(Tensor x, Tensor! residual, Tensor? gate, "
      "Tensor? gamma_opt, Tensor? beta_opt, Tensor scale, Tensor shift, float eps) -> Tensor");
  m.def(
      "rmsnorm_quant_fp8(Tensor x, Tensor weight, float eps, Tensor! output_q, "
      "Tensor! output_s, int group_size) -> ()");
  m.def(
      "norm_scale_shift_quant_fp8(Tensor x, Tensor(a!)? residual, Tensor? gate, "
      "Tensor? gamma_opt, Tensor? beta_opt, Tensor scale, Tensor shift, int norm_type, "
      "float eps, Tensor! output_q, Tensor! output_s) -> ()");
  m.def(
      "kv_commit_rope(Tensor src_k, Tensor? src_v, Tensor(a!) dst_k, Tensor(b!)? dst_v, "
      "int dst_offset, Tensor cos, Tensor sin) -> ()");
  m.def(
      "gelu_tanh_quant_fp8(Tensor input, Tensor! output_q, Tensor! output_s, "
      "Tensor(a!)? output_act=None) -> ()");
  m.def("apply_rotary_emb(Tensor x, Tensor cos, Tensor sin) -> Tensor");
  m.def("rmsnorm_heads(Tensor x, Tensor weight, float eps, int round_first) -> Tensor");
  m.def(
      "fused_norm_scale_shift_per_sample(Tensor x, Tensor? gamma_opt, Tensor? beta_opt, "
      "Tensor scale, Tensor shift, int norm_type, float eps) -> Tensor");
}

TORCH_LIBRARY_IMPL(joyomni_ops, CUDA, m) {
  m.impl("fused_qk_norm_rope_3d_paired", &joyomni_ops::fused_qk_norm_rope_3d_paired);
  m.impl("fused_norm_scale_shift", &joyomni_ops::fused_norm_scale_shift);
  m.impl("rmsnorm", &joyomni_ops::rmsnorm);
  m.impl("sgl_per_token_quant_fp8", &joyomni_ops::sgl_per_token_quant_fp8);
  m.impl("fp8_scaled_mm", &joyomni_ops::fp8_scaled_mm);
  m.impl("fused_qk_norm_rope_3d_grid", &joyomni_ops::fused_qk_norm_rope_3d_grid);
  m.impl("fused_qk_norm_rope_3d_kvcache", &joyomni_ops::fused_qk_norm_rope_3d_kvcache);
  m.impl("fused_qk_norm_rope_3d_paired_kstage",
         &joyomni_ops::fused_qk_norm_rope_3d_paired_kstage);
  m.impl("fused_qk_norm_rope_3d_grid_kstage", &joyomni_ops::fused_qk_norm_rope_3d_grid_kstage);
  m.impl("fused_add_layernorm_scale_shift", &joyomni_ops::fused_add_layernorm_scale_shift);
  m.impl("rmsnorm_quant_fp8", &joyomni_ops::rmsnorm_quant_fp8);
  m.impl("norm_scale_shift_quant_fp8", &joyomni_ops::norm_scale_shift_quant_fp8);
  m.impl("kv_commit_rope", &joyomni_ops::kv_commit_rope);
  m.impl("gelu_tanh_quant_fp8", &joyomni_ops::gelu_tanh_quant_fp8);
  m.impl("apply_rotary_emb", &joyomni_ops::apply_rotary_emb);
  m.impl("rmsnorm_heads", &joyomni_ops::rmsnorm_heads);
  m.impl("fused_norm_scale_shift_per_sample", &joyomni_ops::fused_norm_scale_shift_per_sample);
}
