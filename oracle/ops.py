"""Torch-on-CPU restatements of the reference's joyomni_ops formulas.

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg. Every function takes and returns CPU tensors and
computes in fp32 exactly as the cited reference lines (kernel semantics) or
test formulas do. Paths are relative to jd-opensource/JoyAI-Video-Edit.
"""
from __future__ import annotations

import torch

FP8_MAX = 448.0


# ---------------------------------------------------------------------------
# FP8 per-token quantization — deploy/joyomni_ops/csrc/per_token_quant_fp8.cu:56-82
# ---------------------------------------------------------------------------
def fp8_quant_with_inv(v: torch.Tensor, inv: torch.Tensor) -> torch.Tensor:
    """q = e4m3fn(fmax(fmin(v * inv, 448), -448)) as uint8 (per_token_quant_fp8.cu:72-74).

    torch.fmin/fmax return the non-NaN operand like CUDA fminf/fmaxf, so a NaN
    becomes +448. The clamp keeps the cast's input finite; torch's cast then
    rounds to nearest-even, which equals the reference's satfinite conversion.
    """
    t = v * inv
    t = torch.fmax(torch.fmin(t, torch.tensor(FP8_MAX)), torch.tensor(-FP8_MAX))
    return t.to(torch.float8_e4m3fn).view(torch.uint8)


def scale_and_inv(amax: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """scale = amax / 448; inv = (scale == 0) ? 0 : 1 / scale (per_token_quant_fp8.cu:63-65)."""
    scale = amax / FP8_MAX
    inv = torch.where(scale == 0, torch.zeros_like(scale), 1.0 / scale)
    return scale, inv


def nan_ignoring_amax(v: torch.Tensor, dim: int = -1) -> torch.Tensor:
    """max(0, max |v|) with NaNs skipped, as fmaxf(max, fabsf(v)) from 0 does (:56-61)."""
    a = v.abs()
    a = torch.where(torch.isnan(a), torch.zeros_like(a), a)
    return a.amax(dim=dim) if a.shape[dim] > 0 else torch.zeros(a.shape[:-1])


def per_token_quant_fp8(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """x: bf16/fp16 [M, K] -> (q uint8 [M, K] e4m3fn bytes, s fp32 [M])."""
    xf = x.float()
    scale, inv = scale_and_inv(nan_ignoring_amax(xf))
    return fp8_quant_with_inv(xf, inv[:, None]), scale


# ---------------------------------------------------------------------------
# MLP activation of the DiT block's FP8 mode, deploy/xvideo/models/dit/dit.py:91-92
# and :433 (torch.nn.functional.gelu(h, approximate="tanh") on the up-projection's
# bf16 output), followed by the next Fp8Linear's activation quantization
# (fp8_linear.py:140-166 -> per_token_quant_fp8 above).
# ---------------------------------------------------------------------------
def gelu_tanh_f32(x: torch.Tensor) -> torch.Tensor:
    """0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) in fp32 (torch's CPU kernel)."""
    return torch.nn.functional.gelu(x.float(), approximate="tanh")


def gelu_tanh_quant_fp8(x: torch.Tensor, act: torch.Tensor | None = None):
    """x bf16/fp16 [M, K] -> (q uint8 [M, K], s fp32 [M], act [M, K] in x's dtype):
    the activation rounded to x's dtype, then per_token_quant_fp8 of it. With
    `act` given, the quantization is applied to that activation instead (the
    check of a kernel's quantization given its own activation)."""
    a = gelu_tanh_f32(x).to(x.dtype) if act is None else act
    q, s = per_token_quant_fp8(a)
    return q, s, a


# ---------------------------------------------------------------------------
# RMSNorm — deploy/joyomni_ops/csrc/rmsnorm.cu:41-60; formula of
# deploy/joyomni_ops/tests/test_bench.py:65-67 and test_parity_light.py:31-32.
# ---------------------------------------------------------------------------
def rmsnorm_f32(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)) * w.float()


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    return rmsnorm_f32(x, w, eps).to(x.dtype)


def f32_op(fn, *args: torch.Tensor) -> torch.Tensor:
    """One IEEE binary32 operation (+, -, *, /, sqrt) on fp32 operands, evaluated
    in float64 and rounded once to fp32. For these operations float64 carries
    more than 2*24+2 bits, so the double rounding is innocuous and the result
    is the correctly rounded fp32 value (torch's own CPU sqrt is not)."""
    return fn(*(a.double() for a in args)).float()


def rms_rstd_exact(x: torch.Tensor, eps: float) -> torch.Tensor:
    """r = 1 / sqrt(ms + eps) with ms the mean square summed in float64 and
    rounded once to fp32 (the torch RMSNorm module's kernel, rms_norm_module
    below).

    The reference sums x^2 in fp32 in its kernel's own order (rmsnorm.cu:47-53);
    any fp32 sum lands within a few ulps of the exact value, in an
    order-dependent way. This restatement takes the sum exactly (squares of
    bf16/fp16 are exact in fp32, their float64 sum is exact to ~1e-16), rounds
    the mean once to fp32, then applies the fp32 add of eps (eps itself as
    fp32), an IEEE sqrt and an IEEE division.
    """
    xf = x.float()
    ms = (xf.double().pow(2).sum(-1, keepdim=True) / xf.shape[-1]).float()
    e = torch.tensor(eps, dtype=torch.float32)
    t = f32_op(torch.add, ms, e)
    s = f32_op(torch.sqrt, t)
    return f32_op(torch.div, torch.ones_like(s), s)


def rmsnorm_exact_f32(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """(x * r) * w in fp32 with r from rms_rstd_exact (order of rmsnorm.cu:57)."""
    xr = f32_op(torch.mul, x.float(), rms_rstd_exact(x, eps))
    return f32_op(torch.mul, xr, w.float())


# ---------------------------------------------------------------------------
# torch RMSNorm module — deploy/xvideo/models/dit/dit.py:228-250 (forward
# :244-249), applied to the text stream's q and k (dit.py:384-385).
# ---------------------------------------------------------------------------
def rms_norm_module(x: torch.Tensor, w, eps: float) -> torch.Tensor:
    """_norm(x.float()).type_as(x) * weight: x * r in fp32 rounded to x's dtype,
    then the product with the weight (two tensors of that dtype: an fp32
    product rounded once). r from rms_rstd_exact; w None = a non-affine module."""
    t = f32_op(torch.mul, x.float(), rms_rstd_exact(x, eps)).to(x.dtype)
    if w is None:
        return t
    return f32_op(torch.mul, t.float(), w.float()).to(x.dtype)


# ---------------------------------------------------------------------------
# (Layer|RMS)Norm + AdaLN — deploy/joyomni_ops/csrc/fused_norm_scale_shift.cu:88-142;
# formula of test_parity_light.py:47-51 / test_bench.py:91-96.
# gamma is the affine switch (:125, :192); beta only applies with gamma (:130).
# ---------------------------------------------------------------------------
def norm_scale_shift_f32(x, gamma, beta, scale, shift, norm_type: int, eps: float):
    xf = x.float()
    affine = gamma is not None
    if norm_type == 0:
        mean = xf.mean(-1, keepdim=True)
        var = (xf - mean).pow(2).mean(-1, keepdim=True)
        n = (xf - mean) * torch.rsqrt(var + eps)
        if affine:
            n = n * gamma.float()
            if beta is not None:
                n = n + beta.float()
    elif norm_type == 1:
        n = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
        if affine:
            n = n * gamma.float()
    else:
        raise ValueError("norm_type must be 0 (layer) or 1 (rms)")
    return n * (1 + scale.float()) + shift.float()


def norm_scale_shift(x, gamma, beta, scale, shift, norm_type: int, eps: float):
    return norm_scale_shift_f32(x, gamma, beta, scale, shift, norm_type, eps).to(x.dtype)


# ---------------------------------------------------------------------------
# Residual (optionally gated) add + LayerNorm + AdaLN: composition of
# deploy/xvideo/models/dit/sgl_fused_ops.py:114-117 (torch.addcmul, one
# rounding) and the LayerNorm path above, on the rounded residual.
# ---------------------------------------------------------------------------
def residual_add(x, residual, gate):
    """round(residual + x * gate) (gate None: residual + x), fp32 then one rounding."""
    xf = x.float()
    rf = residual.float()
    upd = rf + (xf * gate.float() if gate is not None else xf)
    return upd.to(residual.dtype)


def add_layernorm_scale_shift(x, residual, gate, gamma, beta, scale, shift, eps: float):
    new_res = residual_add(x, residual, gate)
    y = norm_scale_shift_f32(new_res, gamma, beta, scale, shift, 0, eps)
    return new_res, y


# ---------------------------------------------------------------------------
# (Gated residual add +) norm + AdaLN with the per-token FP8 epilogue: the
# calls the DiT makes back to back — the residual update and modulated norm
# above (dit.py:447-476), the 16-bit y as that op returns it, then
# per_token_quant_fp8 (per_token_quant_fp8.cu:56-82) as Fp8Linear.forward
# runs it on y (fp8_linear.py:138-169).
# ---------------------------------------------------------------------------
def norm_scale_shift_quant_fp8(x, residual, gate, gamma, beta, scale, shift, norm_type: int,
                               eps: float, y=None):
    """Returns (new residual or None, q uint8 [M, N], s fp32 [M], y [M, N] 16-bit).
    y, when given, is the 16-bit output to quantize (e.g. a device op's own y,
    whose summation order the fp32 restatement does not follow)."""
    new_res = residual_add(x, residual, gate) if residual is not None else None
    src = new_res if residual is not None else x
    if y is None:
        y = norm_scale_shift_f32(src, gamma, beta, scale, shift, norm_type, eps).to(x.dtype)
    q, s = per_token_quant_fp8(y)
    return new_res, q, s, y


# ---------------------------------------------------------------------------
# QK RMSNorm + interleaved RoPE from tables —
# deploy/joyomni_ops/csrc/fused_qknorm_rope_3d_kernel.cu:98-142; formula of
# deploy/joyomni_ops/tests/test_parity_light.py:77-87 / test_bench.py:123-132.
# ---------------------------------------------------------------------------
def qk_norm_rope_f32(x: torch.Tensor, w: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                     eps: float) -> torch.Tensor:
    """x: [B, L, H, D]; cos/sin: [L, D/2] (any float dtype). Returns fp32 [B, L, H, D]."""
    B, L, H, D = x.shape
    xf = x.float()
    xn = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.float()
    c = cos.float().reshape(L, 1, D // 2)
    s = sin.float().reshape(L, 1, D // 2)
    x1 = xn[..., 0::2]
    x2 = xn[..., 1::2]
    o = torch.empty_like(xn)
    o[..., 0::2] = x1 * c - x2 * s
    o[..., 1::2] = x1 * s + x2 * c
    return o


# ---------------------------------------------------------------------------
# RoPE tables — deploy/xvideo/models/dit/rope.py:31-52 (1-D tables),
# dit.py:745-783 (t/h/w axes, meshgrid "ij", concatenation) and
# dit.py:785-809, 918-933 (source-id rotation composed by angle addition).
# ---------------------------------------------------------------------------
def axis_freqs(dim: int, theta: float) -> torch.Tensor:
    """1 / theta^(2j/dim) for j < dim/2, fp32 (rope.py:46-48)."""
    return 1.0 / (theta ** (torch.arange(0, dim, 2)[: (dim // 2)].float() / dim))


def rope_1d(dim: int, pos: torch.Tensor, theta: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(cos, sin) [len(pos), dim] with repeat_interleave(2) (rope.py:31-52)."""
    freqs = torch.outer(pos.float(), axis_freqs(dim, theta))
    return freqs.cos().repeat_interleave(2, dim=1), freqs.sin().repeat_interleave(2, dim=1)


def grid_positions(num_frames: int, grid_h: int, grid_w: int, t0: int):
    """(t, h, w) fp32 positions of every token, frame-major, then h, then w (dit.py:757-764)."""
    t = (torch.arange(num_frames, dtype=torch.float32) + t0).repeat_interleave(grid_h * grid_w)
    hg, wg = torch.meshgrid(torch.arange(grid_h, dtype=torch.float32),
                            torch.arange(grid_w, dtype=torch.float32), indexing="ij")
    h = hg.reshape(-1).repeat(num_frames)
    w = wg.reshape(-1).repeat(num_frames)
    return t, h, w


def rope_grid_tables(num_frames: int, grid_h: int, grid_w: int, t0: int, rope_dims,
                     theta: float, source_id: float = 0.0, source_theta: float = 256.0,
                     source_dim: int | None = None):
    """Full-width fp32 (cos, sin) [L, D] exactly as Transformer3DModel builds them.

    The 3D tables concatenate the t/h/w 1-D tables (dit.py:775-781). A non-zero
    source id composes a second rotation over the first `source_dim` dims
    (default all) by angle addition (dit.py:792-808, 931-932).
    """
    t, h, w = grid_positions(num_frames, grid_h, grid_w, t0)
    cs, ss = [], []
    for dim, pos in zip(rope_dims, (t, h, w)):
        c, s = rope_1d(dim, pos, theta)
        cs.append(c)
        ss.append(s)
    cos3, sin3 = torch.cat(cs, dim=1), torch.cat(ss, dim=1)
    if source_id == 0.0:
        return cos3, sin3
    D = cos3.shape[1]
    role_dim = D if source_dim is None else max(0, min(int(source_dim), D))
    L = cos3.shape[0]
    sid = torch.full((L,), float(source_id), dtype=torch.float32)
    cos_half = torch.ones(L, D // 2, dtype=torch.float32)
    sin_half = torch.zeros(L, D // 2, dtype=torch.float32)
    inv_freq = 1.0 / (source_theta ** (torch.arange(0, role_dim, 2, dtype=torch.float32) / role_dim))
    ang = sid.unsqueeze(-1) * inv_freq
    cos_half[..., : role_dim // 2] = torch.cos(ang)
    sin_half[..., : role_dim // 2] = torch.sin(ang)
    cr = cos_half.repeat_interleave(2, dim=-1)
    sr = sin_half.repeat_interleave(2, dim=-1)
    return cos3 * cr - sin3 * sr, sin3 * cr + cos3 * sr


def half_tables(cos_full: torch.Tensor, sin_full: torch.Tensor):
    """[L, D] -> [L, D/2] by taking every other column (sgl_fused_ops.py:87-89)."""
    return cos_full[..., ::2].contiguous(), sin_full[..., ::2].contiguous()


def qk_norm_rope_grid_f32(x, w, num_frames, grid_h, grid_w, t0, rope_dims, theta, eps,
                          source_id=0.0, source_theta=256.0):
    """Grid-mode oracle: the table-mode formula fed with fp32 (unrounded) tables."""
    cos, sin = half_tables(*rope_grid_tables(num_frames, grid_h, grid_w, t0, rope_dims, theta,
                                             source_id, source_theta))
    return qk_norm_rope_f32(x, w, cos, sin, eps)


def ring_slots(num_frames: int, cache_slots: int, slot_start: int) -> list[int]:
    """Cache frame slot of each chunk frame: (slot_start + f) % cache_slots."""
    return [(slot_start + f) % cache_slots for f in range(num_frames)]


# ---------------------------------------------------------------------------
# RMSNorm -> FP8 (per token / per 1x128 block): rmsnorm.cu:41-60 in fp32
# (no rounding to the input type) followed by per_token_quant_fp8.cu:56-82
# over each row or 1x128 block. The reference sums the squares in fp32 in its
# own block-reduction order (rmsnorm.cu:47-53); the build's kernels sum them
# in fp32 in a fixed order of their own, which rms_sum_squares_fixed restates
# step by step, so the CPU result is bit-exact with the kernels'.
# ---------------------------------------------------------------------------
# (chunks of 8 values, lanes per row, chunks per lane) of the kernels' row
# shapes: the smallest shape whose lanes x chunks cover the row.
_C4_ROW_SHAPES = [(8, 8, 1), (16, 16, 1), (32, 32, 1), (64, 64, 1), (128, 64, 2), (192, 64, 3),
                  (256, 64, 4), (384, 64, 6), (512, 64, 8), (768, 64, 12), (1024, 64, 16),
                  (2048, 256, 8), (3072, 256, 12), (4096, 256, 16)]


def c4_row_shape(N: int, group_size: int = 0) -> tuple[int, int]:
    """(lanes per row, 16-byte chunks per lane) of the RMSNorm -> FP8 kernels
    for rows of N 16-bit values; the per-block kernel uses at least 16 lanes
    (a 1x128 block is one chunk on each of 16 lanes)."""
    chunks = -(-N // 8)
    for limit, lpr, ch in _C4_ROW_SHAPES:
        if chunks <= limit:
            return (max(lpr, 16) if group_size else lpr), ch
    raise ValueError(f"no row shape covers {N} values")


def _lane_tree(a, W: int):
    """Sum over aligned groups of W lanes of a [M, W*k] float32 array, in the
    kernels' butterfly order: partner lane l^7 (W = 8) or l^8 then l^4 (W >= 16),
    then l^2, l^1, l^16 (W >= 32), and for W = 64 lane 0's value plus lane 32's.
    Each step is one IEEE fp32 addition (a + b == b + a). Returns [M, k]."""
    import numpy as np
    M, L = a.shape
    g = a.reshape(M, L // W, W)
    idx = np.arange(W)
    steps = ([7] if W == 8 else [8, 4]) + [2, 1] + ([16] if W >= 32 else [])
    for d in steps:
        g = (g + g[:, :, idx ^ d]).astype(np.float32)
    if W == 64:
        return (g[:, :, 0] + g[:, :, 32]).astype(np.float32)
    return g[:, :, 0]


def rms_sum_squares_fixed(x: torch.Tensor, lpr: int, ch: int) -> torch.Tensor:
    """Sum of x^2 over each row in fp32, in the RMSNorm -> FP8 kernels' order.

    Element e of a row sits on lane (e // 8) % lpr as value j = e % 8 of that
    lane's chunk i = e // (8 * lpr); values past the row are 0. Each lane keeps
    two fp32 accumulators, chunks in order and j = 0..7 within a chunk, value j
    going to accumulator j % 2 as acc + x^2 rounded once (a fused multiply-add;
    x^2 of a 16-bit value is exact in fp32, and float64 carries the sum of two
    fp32 values exactly enough for one correct rounding); the lane's sum is
    acc0 + acc1; lanes are summed per wave (64 lanes, fewer when lpr < 64) by
    _lane_tree, and the waves of a wider row in order."""
    import numpy as np
    xf = x.float().numpy().astype(np.float64)
    M, N = xf.shape
    pad = np.zeros((M, lpr * ch * 8), dtype=np.float64)
    pad[:, :N] = xf
    sq = (pad * pad).reshape(M, ch, lpr, 8)
    acc = [np.zeros((M, lpr), dtype=np.float32), np.zeros((M, lpr), dtype=np.float32)]
    for i in range(ch):
        for j in range(8):
            acc[j & 1] = (acc[j & 1].astype(np.float64) + sq[:, i, :, j]).astype(np.float32)
    lane = (acc[0] + acc[1]).astype(np.float32)
    W = min(lpr, 64)
    waves = _lane_tree(lane, W)           # [M, lpr // W] (one group per row when lpr <= 64)
    total = waves[:, 0]
    for k in range(1, waves.shape[1]):
        total = (total + waves[:, k]).astype(np.float32)
    return torch.from_numpy(np.ascontiguousarray(total))


def rms_rstd_fixed(x: torch.Tensor, eps: float, lpr: int, ch: int) -> torch.Tensor:
    """r = 1 / sqrt(ss / N + eps) [M, 1], ss = rms_sum_squares_fixed, each step an
    IEEE fp32 operation (eps taken as fp32)."""
    ss = rms_sum_squares_fixed(x, lpr, ch)[:, None]
    n = torch.tensor(float(x.shape[-1]), dtype=torch.float32)
    ms = f32_op(torch.div, ss, n)
    t = f32_op(torch.add, ms, torch.tensor(eps, dtype=torch.float32))
    sq = f32_op(torch.sqrt, t)
    return f32_op(torch.div, torch.ones_like(sq), sq)


def rmsnorm_quant_f32(x, w, eps: float, group_size: int = 0) -> torch.Tensor:
    """v = (x * r) * w in fp32 as the RMSNorm -> FP8 kernels compute it (r from
    rms_rstd_fixed with the kernels' row shape for N)."""
    lpr, ch = c4_row_shape(x.shape[-1], group_size)
    xr = f32_op(torch.mul, x.float(), rms_rstd_fixed(x, eps, lpr, ch))
    return f32_op(torch.mul, xr, w.float())


def rmsnorm_quant_fp8(x, w, eps: float, group_size: int = 0, v: torch.Tensor | None = None):
    """Returns (q uint8 [M, N], s fp32 [M] or [M, N/128], v fp32 [M, N])."""
    if v is None:
        v = rmsnorm_quant_f32(x, w, eps, group_size)
    M, N = v.shape
    if group_size == 0:
        scale, inv = scale_and_inv(nan_ignoring_amax(v))
        return fp8_quant_with_inv(v, inv[:, None]), scale, v
    g = v.reshape(M, N // group_size, group_size)
    scale, inv = scale_and_inv(nan_ignoring_amax(g))
    return fp8_quant_with_inv(g, inv[..., None]).reshape(M, N), scale, v


# ---------------------------------------------------------------------------
# apply_rotary_emb — deploy/xvideo/models/dit/rope.py:14-28: rotate_half of the
# fp32 input, then x*cos + rotate_half(x)*sin as three separately rounded fp32
# tensor operations, then type_as(x). The tables broadcast over heads
# (reshape_for_broadcast, rope.py:5-11). The graph runner's commit loop
# (deploy/xvideo/serving/graph_runner.py:137-142) applies it per layer and
# copies the result and V into the pool.
# ---------------------------------------------------------------------------
def rotate_half(x: torch.Tensor) -> torch.Tensor:
    xr, xi = x.float().reshape(*x.shape[:-1], -1, 2).unbind(-1)
    return torch.stack([-xi, xr], dim=-1).flatten(-2)


def apply_rotary_emb(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [B, T, H, D]; cos, sin [T, D] / [1, T, D] / [B, T, D] (float32)."""
    B, T, H, D = x.shape
    c = cos.float().reshape(-1, T, 1, D)
    s = sin.float().reshape(-1, T, 1, D)
    return (x.float() * c + rotate_half(x.float()) * s).to(x.dtype)


def commit_kv(pool_k, pool_v, stage_k, stage_v, offset: int, cos, sin):
    """New (pool_k, pool_v) after run_commit: per layer, the RoPE'd stage_k and
    the stage_v at tokens offset .. offset+T of the pool. pool_*: [L, B, P, H, D];
    stage_*: [L, B, T, H, D]; pool_v / stage_v may be None."""
    pk = pool_k.clone()
    pv = pool_v.clone() if pool_v is not None else None
    T = stage_k.shape[2]
    for li in range(stage_k.shape[0]):
        pk[li, :, offset:offset + T] = apply_rotary_emb(stage_k[li], cos, sin)
        if pv is not None:
            pv[li, :, offset:offset + T] = stage_v[li]
    return pk, pv


# ---------------------------------------------------------------------------
# Row-wise scaled FP8 GEMM — deploy/joyomni_ops/csrc/fp8_gemm.cu:1450-1546, the
# epilogue of its visitor tree (:99-136): t = acc * scale_b (fp32), then
# scale_a * t + bias (multiply-add), rounded to the output dtype.
# The float64 product of e4m3fn operands is exact: every product is a
# multiple of 2^-18 below 2^18, so any sum of up to 2^16 of them fits in a
# double's 53 bits, whatever the order.
# ---------------------------------------------------------------------------
def fp8_scaled_mm(a_q: torch.Tensor, b_q: torch.Tensor, scale_a: torch.Tensor,
                  scale_b: torch.Tensor, out_dtype, bias: torch.Tensor | None = None):
    """a_q fp8 [M, K], b_q fp8 [K, N] (any strides). Returns (out [M, N] of
    out_dtype, acc float64 [M, N] exact, mag float64 [M, N] = sum |a||b| scaled
    by the row and column scales — the size of the terms, for tolerances)."""
    a = a_q.float().double()
    b = b_q.float().double()
    acc = a @ b
    sa = scale_a.reshape(-1, 1).float()
    sb = scale_b.reshape(1, -1).float()
    t = acc.float() * sb
    out = sa.double() * t.double()
    if bias is not None:
        out = out + bias.float().double().reshape(1, -1)
    out32 = out.float()  # one rounding of the multiply-add
    mag = (a.abs() @ b.abs()) * sa.double() * sb.double()
    return out32.to(out_dtype), acc, mag
