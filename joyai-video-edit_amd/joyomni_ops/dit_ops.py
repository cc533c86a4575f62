"""DiT-side call shims over joyomni_ops, with the reference's names and signatures.

Counterpart of deploy/xvideo/models/dit/sgl_fused_ops.py:1-117 (the functions
MMDoubleStreamBlock.forward calls, dit.py:351-476) and of the activation
quantization step of Fp8Linear.forward (deploy/xvideo/models/dit/fp8_linear.py:138-169).
Same arguments, same results; the differences are in the HBM traffic:

  fused_layernorm_modulate  reads per-sample shift/scale [B, D] in place, one
                            row per sample, instead of materialising [B*L, D]
                            copies (sgl_fused_ops.py:44-51 expands and copies them).
  fused_qk_norm_rope_3d     identical contract (contiguous copies of q/k, tables
                            halved and cast to bf16 as sgl_fused_ops.py:73-94).
  rmsnorm_qk_bf16           normalizes the K slice of the packed qkv in place of
                            its .contiguous() copy (sgl_fused_ops.py:108).

Additional entry points for callers that can use the new fused ops:

  fused_qk_norm_rope_3d_grid_views  RMSNorm + RoPE in place on q/k views of the
                            packed qkv [B, L, 3, H, D] with angles computed from
                            grid positions (no tables, no .contiguous() copies).
  fused_qk_norm_rope_3d_kstage  the pre-RoPE K-cache path of dit.py:360-370
                            (rmsnorm_qk_bf16 of K, then fused_qk_norm_rope_3d) in one
                            pass that reads K once; q / k rotated in place on their
                            packed-qkv views (no .contiguous() copies).
  fused_add_gate_layernorm_modulate residual + x * gate and the following
                            fused_layernorm_modulate in one pass (dit.py:447-457).
  quantize_activation_fp8   x_q, x_scale of Fp8Linear.forward (fp8_linear.py:140-166).
  layernorm_modulate_fp8    fused_layernorm_modulate followed by that quantization,
                            in one pass (the bf16 output is never written).
  fused_add_gate_layernorm_modulate_fp8  the same after residual + x * gate.
  commit_kv_pool            StreamingGraphRunner.run_commit (graph_runner.py:137-142)
                            for all layers in one launch.
  rms_norm_module           the torch RMSNorm module's forward (dit.py:244-249) that
                            the text stream applies to q and k (dit.py:384-385),
                            read from the packed qkv view.
  gelu_quantize_activation_fp8  the MLP activation gelu(h, approximate="tanh")
                            (dit.py:91-92, 433) and the quantization of the
                            following Fp8Linear.forward in one pass (the bf16
                            activation is never written).
  fp8_linear                Fp8Linear.forward (fp8_linear.py:155-169): per-token
                            quantization + fp8_scaled_mm; quantize_weight_per_channel
                            is its weight preparation (fp8_linear.py:100-110).
"""
from __future__ import annotations

from typing import Optional, Sequence, Tuple

import torch

from . import (fp8_scaled_mm, fused_add_layernorm_scale_shift, fused_norm_scale_shift,
               fused_norm_scale_shift_per_sample, fused_qk_norm_rope_3d_grid, fused_qk_norm_rope_3d_grid_kstage, gelu_tanh_quant_fp8,
               fused_qk_norm_rope_3d_paired, fused_qk_norm_rope_3d_paired_kstage,
               kv_commit_rope, norm_scale_shift_quant_fp8, rmsnorm, rmsnorm_heads,
               rope_freqs, sgl_per_token_quant_fp8)


def available() -> bool:
    """The reference's availability probe (sgl_fused_ops.py:14-27): the ops load at import."""
    return True


def fused_layernorm_modulate(
    x: torch.Tensor,
    shift: torch.Tensor,
    scale: torch.Tensor,
    *,
    weight: Optional[torch.Tensor] = None,
    bias: Optional[torch.Tensor] = None,
    eps: float = 1e-6,
) -> torch.Tensor:
    """LayerNorm(x; weight, bias) * (1 + scale) + shift for x [B, L, D]
    (sgl_fused_ops.py:30-54). shift/scale: [B, D], [B, 1, D] or [B, L, D].

    Per-sample vectors are read in place, one row per sample of L tokens
    (fused_norm_scale_shift_per_sample), for any B: no [B*L, D] expanded
    copies; per-token modulation is read a row each."""
    B, L, D = x.shape
    out = fused_norm_scale_shift_per_sample(x.reshape(-1, D), weight, bias,
                                            _mod_per_sample(scale, B, L, D),
                                            _mod_per_sample(shift, B, L, D), "layer", eps)
    return out.reshape(B, L, D)


def fused_qk_norm_rope_3d(
    q: torch.Tensor,
    k: torch.Tensor,
    q_norm_weight: torch.Tensor,
    k_norm_weight: torch.Tensor,
    freqs_cis: Tuple[torch.Tensor, torch.Tensor],
    *,
    eps: float = 1e-6,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-head RMSNorm + interleaved RoPE of q, k [B, L, H, D] from
    (cos, sin) tables [1, L, D] or [L, D/2] (sgl_fused_ops.py:57-99). Returns
    contiguous (q, k): copies when q / k are strided views (such as the slices
    of a packed qkv), which leaves the inputs untouched; q / k themselves,
    rotated in place, when they are already contiguous (.contiguous() is then
    a no-op), as in the reference."""
    if q.dtype != torch.bfloat16:
        raise RuntimeError(f"fused_qk_norm_rope_3d requires bf16 q/k, got {q.dtype}")
    B, L, H, D = q.shape
    q = q.contiguous()
    k = k.contiguous()
    q_r = q.view(B, L * H, D)
    k_r = k.view(B, L * H, D)
    cos_bf16, sin_bf16 = _half_tables_bf16(freqs_cis, L, D, q.device)
    qw = q_norm_weight.to(torch.bfloat16)
    kw = k_norm_weight.to(torch.bfloat16)
    fused_qk_norm_rope_3d_paired(q_r, k_r, L, H, eps, qw, kw, cos_bf16, sin_bf16)
    return q, k


def _half_tables_bf16(freqs_cis, L: int, D: int, device):
    """cos/sin as the paired op takes them: [L, D/2] bf16, from [1, L, D] or
    [L, D/2] tables, squeezed, halved and cast as sgl_fused_ops.py:80-94 does."""
    cos, sin = freqs_cis
    cos = cos.to(device)
    sin = sin.to(device)
    while cos.dim() > 2:
        if cos.shape[0] != 1:
            raise RuntimeError(f"freqs_cis cos has non-singleton leading dim: {cos.shape}")
        cos = cos.squeeze(0)
        sin = sin.squeeze(0)
    if cos.shape[-1] == D:
        cos = cos[..., ::2]
        sin = sin[..., ::2]
    return cos.contiguous().to(torch.bfloat16), sin.contiguous().to(torch.bfloat16)


def fused_qk_norm_rope_3d_kstage(
    q: torch.Tensor,
    k: torch.Tensor,
    q_norm_weight: torch.Tensor,
    k_norm_weight: torch.Tensor,
    freqs_cis: Tuple[torch.Tensor, torch.Tensor],
    *,
    eps: float = 1e-6,
    k_stage: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The K-cache-before-RoPE branch of MMDoubleStreamBlock.forward
    (dit.py:360-370): k_for_cache = rmsnorm_qk_bf16(k, k_norm_weight) and
    q, k = fused_qk_norm_rope_3d(q, k, ...), in one pass that reads K once.

    q, k: bf16 [B, L, H, D], typically the q / k slices of the packed qkv
    [B, L, 3, H, D] (heads contiguous per token); they are normalized and
    rotated IN PLACE and returned (the reference returns rotated contiguous
    copies and leaves the qkv slices as they were; the DiT forward reads only
    the returned q, k and the v slice afterwards). freqs_cis: (cos, sin) of
    [1, L, D] or [L, D/2]. k_stage: bf16 [B, L, H, D] destination of the
    pre-RoPE normalized K (e.g. a layer's slice of the graph runner's stage
    buffer), allocated when None. Returns (q, k, k_stage); k_stage equals
    rmsnorm_qk_bf16(k) of the input k bit for bit."""
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16:
        raise RuntimeError(f"fused_qk_norm_rope_3d_kstage requires bf16 q/k, got {q.dtype}")
    B, L, H, D = q.shape
    if k_stage is None:
        k_stage = torch.empty((B, L, H, D), dtype=torch.bfloat16, device=q.device)
    cos, sin = _half_tables_bf16(freqs_cis, L, D, q.device)
    fused_qk_norm_rope_3d_paired_kstage(q, k, k_stage, L, H, eps,
                                        q_norm_weight.to(torch.bfloat16).contiguous(),
                                        k_norm_weight.to(torch.bfloat16).contiguous(), cos, sin)
    return q, k, k_stage


def _heads_view(x: torch.Tensor) -> bool:
    """x [..., H, D] with a contiguous last dim whose leading dims collapse to
    one token stride (what rmsnorm_heads reads without a copy)."""
    if x.dim() < 2 or (x.stride(-1) != 1 and x.shape[-1] > 1):
        return False
    nxt = None
    for d in range(x.dim() - 3, -1, -1):
        if x.shape[d] == 1:
            continue
        if nxt is not None and x.stride(d) != nxt:
            return False
        nxt = x.stride(d) * x.shape[d]
    return True


def rmsnorm_qk_bf16(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm over the last dim of a bf16 tensor (sgl_fused_ops.py:102-111).

    A [..., H, D] view such as the K slice of the packed qkv is read in place
    (the reference copies it with .contiguous() first, :108); the result is a
    new contiguous tensor of x's shape, bit-identical to the rmsnorm op on the
    copy (same kernel, same summation order)."""
    assert x.dtype == torch.bfloat16, f"rmsnorm_qk_bf16 needs bf16, got {x.dtype}"
    w = weight.to(dtype=torch.bfloat16)
    if _heads_view(x):
        return rmsnorm_heads(x, w, eps)
    orig_shape = x.shape
    D = orig_shape[-1]
    out = rmsnorm(x.reshape(-1, D).contiguous(), w, eps)
    return out.reshape(orig_shape)


def rms_norm_module(x: torch.Tensor, weight: Optional[torch.Tensor] = None,
                    eps: float = 1e-6) -> torch.Tensor:
    """The torch RMSNorm module's forward (dit.py:244-249):
    (x.float() * rsqrt(mean(x.float()^2) + eps)).type_as(x), times weight
    (a separately rounded product) when the module is affine. x: [..., D]
    (the text stream's q or k view, [B, Lt, H, D] inside the packed qkv);
    weight: [D] in x's dtype or None. Returns a new contiguous tensor."""
    D = x.shape[-1]
    if weight is None:
        weight = torch.ones(D, dtype=x.dtype, device=x.device)
    if weight.dtype != x.dtype:
        raise RuntimeError(f"rms_norm_module: weight dtype {weight.dtype} != x dtype {x.dtype}")
    if _heads_view(x):
        return rmsnorm_heads(x, weight, eps, round_first=True)
    return rmsnorm_heads(x.reshape(-1, 1, D).contiguous(), weight, eps,
                         round_first=True).reshape(x.shape)


def fused_add_gate(residual: torch.Tensor, x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """residual + x * gate[:, None] (sgl_fused_ops.py:114-117), a torch op as in the reference."""
    return torch.addcmul(residual, x, gate.unsqueeze(1))


# ---------------------------------------------------------------------------
# Fused forms for callers that can use them.
# ---------------------------------------------------------------------------
def fused_add_gate_layernorm_modulate(
    residual: torch.Tensor,
    x: torch.Tensor,
    gate: torch.Tensor,
    shift: torch.Tensor,
    scale: torch.Tensor,
    *,
    weight: Optional[torch.Tensor] = None,
    bias: Optional[torch.Tensor] = None,
    eps: float = 1e-6,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """(residual', modulated) with residual' = residual + x * gate[:, None] and
    modulated = fused_layernorm_modulate(residual', shift, scale) — the pair of
    calls at dit.py:447-457 in one pass. residual [B, L, D] is updated in place
    (it must be contiguous in its rows) and returned; gate/shift/scale [B, D]."""
    B, L, D = x.shape
    if not residual.is_contiguous():
        raise RuntimeError("residual must be contiguous (it is updated in place)")
    out = fused_add_layernorm_scale_shift(x.reshape(B * L, D), residual.view(B * L, D),
                                          _mod_per_sample(scale, B, L, D),
                                          _mod_per_sample(shift, B, L, D),
                                          gate=_mod_per_sample(gate, B, L, D), gamma=weight,
                                          beta=bias, eps=eps)
    return residual, out.reshape(B, L, D)


def fused_qk_norm_rope_3d_grid_views(
    q: torch.Tensor,
    k: torch.Tensor,
    q_norm_weight: torch.Tensor,
    k_norm_weight: torch.Tensor,
    *,
    grid_hw: Tuple[int, int],
    t0: int,
    rope_dims: Sequence[int],
    theta: float,
    source_id: float = 0.0,
    source_theta: float = 256.0,
    source_dim: int = 128,
    eps: float = 1e-6,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """In-place RMSNorm + RoPE of q, k [B, L, H, D] that may be strided views of
    a packed qkv [B, L, 3, H, D] (heads contiguous per token). Angles come from
    the grid position (frame f of L / (H_grid * W_grid) at t0 + f), with the
    optional source-id rotation over the first min(source_dim, D) dims (the
    model's source_id_rope_dim = 128 and source_id_rope_theta = 256,
    dit.py:549-550,792), exactly as Transformer3DModel builds its tables
    (dit.py:745-809, 918-933); no tables are read. Returns (q, k)."""
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16:
        raise RuntimeError("q/k must be bf16")
    B, L, H, D = q.shape
    if q.stride(-1) != 1 or q.stride(-2) != D or k.stride(-1) != 1 or k.stride(-2) != D:
        raise RuntimeError("heads of a token must be contiguous in q and k")
    freqs = rope_freqs(D, rope_dims, theta, source_theta, source_dim)
    qw = q_norm_weight.to(torch.bfloat16).contiguous()
    kw = k_norm_weight.to(torch.bfloat16).contiguous()
    fused_qk_norm_rope_3d_grid(q, k, L, H, eps, qw, kw, freqs, rope_dims, grid_hw, t0, source_id)
    return q, k


def quantize_activation_fp8(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """The activation side of Fp8Linear.forward (fp8_linear.py:140-144, 166):
    x [..., K] -> (x_q fp8 e4m3fn [M, K], x_scale fp32 [M, 1]) with M = numel / K."""
    x_2d = x.reshape(-1, x.shape[-1]).contiguous()
    M, K = x_2d.shape
    x_q = torch.empty((M, K), device=x_2d.device, dtype=torch.float8_e4m3fn)
    x_scale = torch.empty((M, 1), device=x_2d.device, dtype=torch.float32)
    sgl_per_token_quant_fp8(x_2d, x_q, x_scale)
    return x_q, x_scale


def gelu_quantize_activation_fp8(h: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """quantize_activation_fp8(torch.nn.functional.gelu(h, approximate="tanh")) in
    one pass (the MLP activation of dit.py:433 and the activation side of the
    next Fp8Linear.forward, fp8_linear.py:140-166): h [..., K] bf16/fp16 ->
    (x_q fp8 e4m3fn [M, K], x_scale fp32 [M, 1]). The activation is evaluated
    in fp32 and rounded to h's dtype before it is quantized, as the two calls do."""
    h_2d = h.reshape(-1, h.shape[-1])
    if h_2d.stride(-1) != 1:
        h_2d = h_2d.contiguous()
    M, K = h_2d.shape
    x_q, x_scale = _fp8_outputs(M, K, h_2d.device)
    gelu_tanh_quant_fp8(h_2d, x_q, x_scale)
    return x_q, x_scale


def _mod_per_sample(t: torch.Tensor, B: int, L: int, D: int) -> torch.Tensor:
    """A modulation vector as the fused norm ops take it, without copies: [B, D]
    or [B, 1, D] -> [B, D] (one row per sample of L rows; [D] when B == 1),
    [B, L, D] -> [B*L, D] (a row per token)."""
    if t.numel() == B * D:
        return t.reshape(D) if B == 1 else t.reshape(B, D)
    return t.reshape(B * L, D)


def _fp8_outputs(M: int, D: int, device) -> Tuple[torch.Tensor, torch.Tensor]:
    """x_q fp8 e4m3fn [M, D] and x_scale fp32 [M, 1], as Fp8Linear.forward allocates them."""
    return (torch.empty((M, D), device=device, dtype=torch.float8_e4m3fn),
            torch.empty((M, 1), device=device, dtype=torch.float32))


def layernorm_modulate_fp8(
    x: torch.Tensor,
    shift: torch.Tensor,
    scale: torch.Tensor,
    *,
    weight: Optional[torch.Tensor] = None,
    bias: Optional[torch.Tensor] = None,
    eps: float = 1e-6,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """quantize_activation_fp8(fused_layernorm_modulate(x, shift, scale)) in one
    pass: x [B, L, D], shift/scale [B, D], [B, 1, D] or [B, L, D] ->
    (x_q [B*L, D], x_scale [B*L, 1]), byte-identical to the two calls."""
    B, L, D = x.shape
    x_q, x_scale = _fp8_outputs(B * L, D, x.device)
    norm_scale_shift_quant_fp8(x.reshape(B * L, D), _mod_per_sample(scale, B, L, D),
                               _mod_per_sample(shift, B, L, D), x_q, x_scale, gamma=weight,
                               beta=bias, eps=eps)
    return x_q, x_scale


def fused_add_gate_layernorm_modulate_fp8(
    residual: torch.Tensor,
    x: torch.Tensor,
    gate: torch.Tensor,
    shift: torch.Tensor,
    scale: torch.Tensor,
    *,
    weight: Optional[torch.Tensor] = None,
    bias: Optional[torch.Tensor] = None,
    eps: float = 1e-6,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """fused_add_gate_layernorm_modulate followed by quantize_activation_fp8 of
    its modulated output, in one pass: returns (residual', x_q [B*L, D],
    x_scale [B*L, 1]); residual [B, L, D] is updated in place."""
    B, L, D = x.shape
    if not residual.is_contiguous():
        raise RuntimeError("residual must be contiguous (it is updated in place)")
    x_q, x_scale = _fp8_outputs(B * L, D, x.device)
    norm_scale_shift_quant_fp8(x.reshape(B * L, D), _mod_per_sample(scale, B, L, D),
                               _mod_per_sample(shift, B, L, D), x_q, x_scale,
                               residual=residual.view(B * L, D),
                               gate=_mod_per_sample(gate, B, L, D), gamma=weight, beta=bias,
                               eps=eps)
    return residual, x_q, x_scale


def commit_kv_pool(pool_k: torch.Tensor, pool_v: torch.Tensor, stage_k: torch.Tensor,
                   stage_v: torch.Tensor, offset: int, commit_cos: torch.Tensor,
                   commit_sin: torch.Tensor) -> None:
    """The graph runner's commit (graph_runner.py:137-142): for every layer li,
    pool_k[li, :, offset:offset+T] = apply_rotary_emb(stage_k[li], (cos, sin)) and
    pool_v[li, :, offset:offset+T] = stage_v[li], as one launch instead of one
    RoPE and two copies per layer. pool_*: [L, B, P, H, D]; stage_*: [L, B, T, H, D];
    commit_cos/sin: fp32 [1, T, D]. Bit-identical to the loop."""
    kv_commit_rope(stage_k, pool_k, offset, commit_cos, commit_sin, src_v=stage_v, dst_v=pool_v)


FP8_MAX = 448.0


def quantize_weight_per_channel(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Fp8Linear's weight preparation (fp8_linear.py:100-110, the path without
    fast accumulation): w [N, K] -> (w_q fp8 [K, N] column-major, scale fp32 [N])
    with scale = max|w[n, :]| / 448 (floored at 1e-8 / 448)."""
    w_kn = w.to(torch.bfloat16).t().contiguous()
    absmax = w_kn.abs().amax(dim=0).to(torch.float32).clamp_min(1e-8)
    scale = absmax / FP8_MAX
    w_q_rm = (w_kn.float() / scale.unsqueeze(0)).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return w_q_rm.t().contiguous().t(), scale


def fp8_linear(x: torch.Tensor, weight_fp8: torch.Tensor, weight_scale: torch.Tensor,
               bias: Optional[torch.Tensor] = None, out_dtype=torch.bfloat16) -> torch.Tensor:
    """Fp8Linear.forward (fp8_linear.py:155-169): x [..., K] bf16 -> per-token
    fp8 + scales -> fp8_scaled_mm with the per-channel weight scales and bias."""
    x_q, x_scale = quantize_activation_fp8(x)
    y = fp8_scaled_mm(x_q, weight_fp8, x_scale, weight_scale, out_dtype, bias)
    return y.reshape(*x.shape[:-1], weight_fp8.shape[1])


def fp8_linear_quantized(x_q: torch.Tensor, x_scale: torch.Tensor, weight_fp8: torch.Tensor,
                         weight_scale: torch.Tensor, bias: Optional[torch.Tensor] = None,
                         out_dtype=torch.bfloat16) -> torch.Tensor:
    """The GEMM half of fp8_linear for activations already quantized in a norm's
    epilogue (layernorm_modulate_fp8 / fused_add_gate_layernorm_modulate_fp8)."""
    return fp8_scaled_mm(x_q, weight_fp8, x_scale, weight_scale, out_dtype, bias)
