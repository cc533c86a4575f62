"""CPU tests that pin the oracle before it is trusted as the parity checker.

The reference ships no golden vectors (its tests print fp32-formula diffs), so
each oracle function is checked against something independent of it: hand
known answers, a brute-force C encoder, torch library routines, complex
arithmetic, float64 closed forms and invariants. A few tests plant a mistake
in a copy of the oracle and show the check catches it.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import fp8ref, ops
import kat


# ---------------------------------------------------------------------------
# FP8 encoding and per-token quantization
# ---------------------------------------------------------------------------
def test_kat_table_is_self_consistent():
    kat.check_table()


@pytest.mark.parametrize("idx", range(len(kat.KAT_ROWS)))
def test_quant_kat_rows(idx):
    row, scale, codes = kat.KAT_ROWS[idx]
    x = torch.tensor([row], dtype=torch.float32).to(torch.bfloat16)
    assert torch.equal(x.float(), torch.tensor([row], dtype=torch.float32), ) or any(
        math.isnan(v) for v in row)
    q, s = ops.per_token_quant_fp8(x)
    assert q[0].tolist() == codes
    exp_s = torch.tensor(scale, dtype=torch.float32)
    assert torch.equal(s[0], exp_s) or (math.isinf(scale) and math.isinf(s[0].item()))
    qc, sc = fp8ref.per_token_quant(x.float().numpy())
    assert qc[0].tolist() == codes
    assert sc[0] == np.float32(scale)


def test_torch_cast_matches_bruteforce_on_all_bf16():
    bits = torch.arange(0, 65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float()
    v = bits[(bits.abs() <= 448)]
    t = v.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    c = fp8ref.encode_array(v.numpy())
    assert (t == c).all()


def test_torch_cast_matches_bruteforce_on_midpoints_and_random():
    vals = np.array([fp8ref.decode(k) for k in range(0, 0x7f)])
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    # midpoints +- 1 fp32 ulp on both sides as well
    near = np.concatenate([mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9))])
    near = np.concatenate([near, -near]).astype(np.float32)
    g = torch.Generator().manual_seed(0)
    r = ((torch.rand(500_000, generator=g) * 2 - 1) * 448).numpy()
    for arr in (near, r):
        t = torch.from_numpy(arr).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        assert (t == fp8ref.encode_array(arr)).all()


def test_quant_oracle_matches_c_on_random_rows_with_outliers():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(300, 3072, generator=g)
    from joyomni_ops.workloads import with_outliers
    x = with_outliers(x, g).to(torch.bfloat16)
    q, s = ops.per_token_quant_fp8(x)
    qc, sc = fp8ref.per_token_quant(x.float().numpy())
    assert (q.numpy() == qc).all() and (s.numpy() == sc).all()
    # and every code decodes to within half a code step of the fp32 x*inv
    inv = torch.where(s == 0, torch.zeros_like(s), 1.0 / s)
    dec = torch.from_numpy(np.array([fp8ref.decode(k) for k in range(256)]))
    err = (dec[q.long()] - (x.float() * inv[:, None]).double()).abs()
    step = torch.where(dec[q.long()].abs() < 2 ** -6, torch.tensor(2.0 ** -9),
                       dec[q.long()].abs() * 2.0 ** -3)
    assert bool((err <= step / 2 + 1e-12).all())


def test_planted_mistake_x_over_s_is_caught():
    """x / s instead of x * (1/s) (a plausible slip) changes a few codes; the
    C restatement of the reference rule disagrees with it."""
    g = torch.Generator().manual_seed(2)
    x = (torch.randn(2048, 3072, generator=g) * 3).to(torch.bfloat16)
    q, s = ops.per_token_quant_fp8(x)
    xf = x.float()
    qc, _ = fp8ref.per_token_quant(xf.numpy())
    assert (q.numpy() == qc).all()
    wrong = torch.fmax(torch.fmin(xf / s[:, None], torch.tensor(448.0)), torch.tensor(-448.0))
    wrong = wrong.to(torch.float8_e4m3fn).view(torch.uint8)
    n_diff = int((wrong.numpy() != qc).sum())
    assert 0 < n_diff < xf.numel() // 1000
    # a sign slip in the clamp is visible everywhere below zero
    wrong2 = torch.fmax(torch.fmin(xf * (1 / s[:, None]), torch.tensor(448.0)),
                        torch.tensor(448.0)).to(torch.float8_e4m3fn).view(torch.uint8)
    assert (wrong2.numpy() != qc).any()


def test_exact_mean_square_rstd():
    """rms_rstd_exact: the mean square is the fp64 value rounded once; it sits
    within a few fp32 ulps of the reference's fp32-accumulated formula and
    within 1 ulp (plus the two IEEE roundings) of the float64 closed form."""
    g = torch.Generator().manual_seed(31)
    from joyomni_ops.workloads import with_outliers
    x = with_outliers(torch.randn(256, 3072, generator=g), g).to(torch.bfloat16)
    r = ops.rms_rstd_exact(x, 1e-6)
    r64 = 1.0 / torch.sqrt(x.double().pow(2).mean(-1, keepdim=True) + 1e-6)
    assert bool(((r.double() - r64).abs() <= 2 * torch.exp2(torch.floor(torch.log2(r64)) - 23)).all())
    r32 = torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + 1e-6)
    assert bool(((r - r32).abs() <= 8 * torch.exp2(torch.floor(torch.log2(r.abs())) - 23)).all())
    # a planted slip (mean over N-1) is far outside that band
    rw = 1.0 / torch.sqrt((x.double().pow(2).sum(-1, keepdim=True) / 3071).float() + 1e-6)
    assert not torch.allclose(rw, r, rtol=1e-5, atol=0)


def _row_with(N, vals):
    x = torch.zeros(1, N)
    for e, v in vals:
        x[0, e] = v
    return x.to(torch.bfloat16)


def test_fixed_order_sum_known_answers():
    """rms_sum_squares_fixed against hand-derived sums where the order decides
    the fp32 result (fp32 spacing is 2 at 2^24, ties go to even):
      one lane, x = 2^12 then seven 1s: accumulator 0 takes 2^24 and three 1s
        (each lost: 2^24 + 1 ties to 2^24), accumulator 1 four 1s -> 2^24 + 4;
      16 lanes (l^8, l^4, l^2, l^1), lane 0 = 2^24, 15 lanes of 1:
        2^24+1 -> 2^24; +2 -> 2^24+2; +4 -> 2^24+6; +8 -> 2^24+14;
      64 lanes (then l^16, then lane 0 + lane 32): 2^24+14 + 16 = 2^24+30 on
        lanes 0-31, 32 on lanes 32-63 -> 2^24+62.
    The exact sums (2^24 + 7, + 15, + 63) and a left-to-right sum (2^24)
    differ from each."""
    cases = [(16, [(0, 2.0 ** 12)] + [(j, 1.0) for j in range(1, 8)], 4.0),
             (128, [(0, 2.0 ** 12)] + [(8 * l, 1.0) for l in range(1, 16)], 14.0),
             (512, [(0, 2.0 ** 12)] + [(8 * l, 1.0) for l in range(1, 64)], 62.0)]
    for N, vals, extra in cases:
        x = _row_with(N, vals)
        got = ops.rms_sum_squares_fixed(x, *ops.c4_row_shape(N)).double().item()
        assert got == 2.0 ** 24 + extra, (N, got - 2.0 ** 24)
        # planted slips: one accumulator per lane, or a left-to-right row sum
        seq = torch.tensor(0.0)
        for v in x.float()[0]:
            seq = (seq + v * v).float()
        assert seq.item() != got


def test_fixed_order_sum_shapes_and_closeness():
    """The row shapes follow the kernels' dispatch (smallest lanes x chunks
    covering the row; per block at least 16 lanes), and for every shape the
    fixed-order mean square lies within (log2 N + 2) fp32 ulps of the exact
    one; a planted slip (mean over N - 1) lies far outside."""
    assert ops.c4_row_shape(3072) == (64, 6) and ops.c4_row_shape(3072, 128) == (64, 6)
    assert ops.c4_row_shape(64) == (8, 1) and ops.c4_row_shape(64, 128) == (16, 1)
    assert ops.c4_row_shape(4096) == (64, 8) and ops.c4_row_shape(16384) == (256, 8)
    assert ops.c4_row_shape(24576) == (256, 12) and ops.c4_row_shape(32768) == (256, 16)
    with pytest.raises(ValueError):
        ops.c4_row_shape(32776)
    from joyomni_ops.workloads import with_outliers
    g = torch.Generator().manual_seed(41)
    for N in (8, 100, 128, 512, 1000, 3072, 6144, 16384, 20000):
        x = with_outliers(torch.randn(24, N, generator=g), g).to(torch.bfloat16)
        lpr, ch = ops.c4_row_shape(N)
        ss = ops.rms_sum_squares_fixed(x, lpr, ch).double()
        exact = x.double().pow(2).sum(-1)
        ulp = torch.exp2(torch.floor(torch.log2(exact)) - 23)
        bound = (torch.log2(torch.tensor(float(N))).ceil() + 2) * ulp
        assert bool(((ss - exact).abs() <= bound).all()), N
        assert bool(((exact * N / (N - 1) - ss).abs() > bound).all()), N
    r = ops.rms_rstd_fixed(x, 1e-6, lpr, ch)
    r64 = 1.0 / torch.sqrt(x.double().pow(2).mean(-1, keepdim=True) + 1e-6)
    assert bool(((r.double() - r64).abs() <= 24 * torch.exp2(torch.floor(torch.log2(r64)) - 23)).all())


@pytest.mark.parametrize("group", [0, 128])
def test_fixed_order_against_the_reference_torch_formula(group):
    """The kernels' fixed order against the reference's own torch RMSNorm
    (test_parity_light.py:31-32: fp32 mean in torch's order, torch's rsqrt,
    then x * r * w) followed by the same quantization, on C4-shaped rows: the
    scales lie within a few fp32 ulps (torch's rsqrt is itself up to 2 ulps
    off the correctly rounded value here; the exact fp64 mean is no closer)
    and the fp8 bytes agree on all but a few thousandths of a percent."""
    from joyomni_ops.workloads import with_outliers
    g = torch.Generator().manual_seed(5)
    x = with_outliers(torch.randn(512, 3072, generator=g), g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(3072, generator=g)).to(torch.bfloat16)
    q1, s1, _ = ops.rmsnorm_quant_fp8(x, w, 1e-6, group)
    q2, s2, _ = ops.rmsnorm_quant_fp8(x, w, 1e-6, group, v=ops.rmsnorm_f32(x, w, 1e-6))
    ulp = torch.exp2(torch.floor(torch.log2(s2.abs())) - 23)
    assert bool(((s1 - s2).abs() <= 8 * ulp).all())
    assert (q1 == q2).float().mean().item() > 0.9999


def test_group_quant_oracle_matches_c():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(40, 1024, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(1024, generator=g)).to(torch.bfloat16)
    for group in (0, 128):
        q, s, v = ops.rmsnorm_quant_fp8(x, w, 1e-6, group)
        if group == 0:
            qc, sc = fp8ref.per_token_quant(v.numpy())
        else:
            qc, sc = fp8ref.group_quant(v.numpy(), group)
        assert (q.numpy() == qc).all() and (s.numpy() == sc).all()


# ---------------------------------------------------------------------------
# Norms
# ---------------------------------------------------------------------------
def test_rmsnorm_oracle_matches_library_and_invariant():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(64, 512, generator=g)
    w = torch.randn(512, generator=g)
    ref = F.rms_norm(x, (512,), w, eps=1e-6)
    assert torch.allclose(ops.rmsnorm_f32(x, w, 1e-6), ref, rtol=1e-5, atol=1e-6)
    unit = ops.rmsnorm_f32(x, torch.ones(512), 0.0)
    assert torch.allclose(unit.pow(2).mean(-1), torch.ones(64), rtol=1e-5)


def _module_forward_torch(x, w, eps):
    """RMSNorm.forward as dit.py:244-249 writes it, evaluated by torch on the CPU
    (its own fp32 summation order and rsqrt)."""
    xf = x.float()
    out = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).type_as(x)
    return out if w is None else out * w


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("affine", [True, False])
def test_rms_norm_module_oracle_matches_the_module_formula(dtype, affine):
    """Against the module's own torch expression: equal wherever torch's fp32
    r agrees with the exactly rounded one (nearly everywhere), within one
    ulp of the intermediate row (times |w|) elsewhere."""
    g = torch.Generator().manual_seed(21)
    x = (torch.randn(512, 4, 128, generator=g) * 2).to(dtype)
    w = (1 + 0.1 * torch.randn(128, generator=g)).to(dtype) if affine else None
    ref = _module_forward_torch(x, w, 1e-6).float()
    out = ops.rms_norm_module(x, w, 1e-6).float()
    assert out.dtype == ref.dtype and out.shape == ref.shape
    same = (out == ref).float().mean().item()
    assert same > 0.995, same
    mb = 7 if dtype == torch.bfloat16 else 10
    wf = torch.ones(128) if w is None else w.float().abs()
    ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -30))) - mb)
    assert bool(((out - ref).abs() <= 2 * ulp * torch.maximum(wf, torch.ones(128))).all())


def test_rms_norm_module_oracle_rounds_before_the_weight():
    """A planted slip — no rounding between x * r and the weight (the kernel
    rmsnorm's single rounding) — differs from the oracle on a visible share of
    elements; with a unit weight the two coincide."""
    g = torch.Generator().manual_seed(22)
    x = torch.randn(256, 128, generator=g).to(torch.bfloat16)
    w = (1 + 0.3 * torch.randn(128, generator=g)).to(torch.bfloat16)
    out = ops.rms_norm_module(x, w, 1e-6)
    slip = ops.rmsnorm_exact_f32(x, w, 1e-6).to(torch.bfloat16)
    assert (out != slip).float().mean().item() > 0.05
    one = torch.ones(128, dtype=torch.bfloat16)
    assert torch.equal(ops.rms_norm_module(x, one, 1e-6),
                       ops.rmsnorm_exact_f32(x, one, 1e-6).to(torch.bfloat16))
    assert torch.equal(ops.rms_norm_module(x, None, 1e-6), ops.rms_norm_module(x, one, 1e-6))


def test_rms_norm_module_oracle_special_rows():
    """Closed forms: a zero row stays zero; a row of +-a has r = 1/sqrt(a^2 + eps)
    (fp32 ops), so every element is round(+-a * r); NaN spreads over its row;
    an inf makes r = 0 (inf element NaN, the rest zero)."""
    x = torch.zeros(4, 64)
    x[1] = 3.0
    x[1, ::2] = -3.0
    x[2, 5] = float("nan")
    x[3, 7] = float("inf")
    x = x.to(torch.bfloat16)
    out = ops.rms_norm_module(x, None, 1e-6).float()
    assert bool((out[0] == 0).all())
    f32 = np.float32
    r32 = f32(1) / np.sqrt(f32(9) + f32(1e-6))  # numpy: IEEE fp32 add, sqrt, division
    expect = (torch.tensor(3.0) * torch.tensor(float(r32))).to(torch.bfloat16).float()
    assert bool((out[1, 1::2] == expect).all()) and bool((out[1, ::2] == -expect).all())
    assert bool(torch.isnan(out[2]).all())
    assert torch.isnan(out[3, 7]) and bool((out[3, :7] == 0).all()) and bool((out[3, 8:] == 0).all())


@pytest.mark.parametrize("affine", [False, True])
def test_layernorm_modulate_oracle_matches_library(affine):
    g = torch.Generator().manual_seed(5)
    M, N = 32, 256
    x = torch.randn(M, N, generator=g) * 3 + 1
    gamma = torch.randn(N, generator=g) if affine else None
    beta = torch.randn(N, generator=g) if affine else None
    sc = torch.randn(M, N, generator=g)
    sh = torch.randn(M, N, generator=g)
    ref = F.layer_norm(x.double(), (N,), None if gamma is None else gamma.double(),
                       None if beta is None else beta.double(), eps=1e-5)
    ref = ref * (1 + sc.double()) + sh.double()
    out = ops.norm_scale_shift_f32(x, gamma, beta, sc, sh, 0, 1e-5)
    assert torch.allclose(out.double(), ref, rtol=1e-5, atol=1e-5)
    # RMS flavour vs F.rms_norm
    ref_rms = F.rms_norm(x.double(), (N,), None if gamma is None else gamma.double(), eps=1e-5)
    ref_rms = ref_rms * (1 + sc.double()) + sh.double()
    out_rms = ops.norm_scale_shift_f32(x, gamma, beta, sc, sh, 1, 1e-5)
    assert torch.allclose(out_rms.double(), ref_rms, rtol=1e-5, atol=1e-5)


def test_layernorm_beta_without_gamma_is_ignored_like_reference():
    x = torch.randn(4, 16)
    sc = torch.zeros(4, 16)
    sh = torch.zeros(4, 16)
    a = ops.norm_scale_shift_f32(x, None, torch.ones(16), sc, sh, 0, 1e-6)
    b = ops.norm_scale_shift_f32(x, None, None, sc, sh, 0, 1e-6)
    assert torch.equal(a, b)


def test_add_layernorm_oracle_is_addcmul_then_layernorm():
    g = torch.Generator().manual_seed(6)
    M, N = 16, 384
    x = torch.randn(M, N, generator=g).to(torch.bfloat16)
    res = torch.randn(M, N, generator=g).to(torch.bfloat16)
    gate = torch.randn(N, generator=g).to(torch.bfloat16)
    sc = (0.2 * torch.randn(N, generator=g)).to(torch.bfloat16)
    sh = (0.2 * torch.randn(N, generator=g)).to(torch.bfloat16)
    new_res, y = ops.add_layernorm_scale_shift(x, res, gate, None, None, sc, sh, 1e-6)
    ref_res = torch.addcmul(res.float(), x.float(), gate.float()).to(torch.bfloat16)
    assert torch.equal(new_res, ref_res)
    ref_y = F.layer_norm(ref_res.double(), (N,), eps=1e-6) * (1 + sc.double()) + sh.double()
    assert torch.allclose(y.double(), ref_y, rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------------------
# QK norm + RoPE
# ---------------------------------------------------------------------------
def _complex_rope(xn, cos, sin):
    """Rotation of interleaved pairs as complex multiplication (float64)."""
    B, L, H, D = xn.shape
    z = torch.view_as_complex(xn.double().reshape(B, L, H, D // 2, 2).contiguous())
    rot = torch.complex(cos.double(), sin.double()).reshape(1, L, 1, D // 2)
    return torch.view_as_real(z * rot).reshape(B, L, H, D)


def test_qk_rope_oracle_is_complex_rotation():
    g = torch.Generator().manual_seed(7)
    B, L, H, D = 2, 9, 3, 64
    x = torch.randn(B, L, H, D, generator=g)
    w = torch.randn(D, generator=g)
    ang = torch.randn(L, D // 2, generator=g) * 4
    out = ops.qk_norm_rope_f32(x, w, ang.cos(), ang.sin(), 1e-6)
    xn = F.rms_norm(x.double(), (D,), w.double(), eps=1e-6)
    ref = _complex_rope(xn, ang.cos(), ang.sin())
    assert torch.allclose(out.double(), ref, rtol=1e-5, atol=1e-5)
    # norm preservation per pair and identity rotation
    assert torch.allclose(out.reshape(B, L, H, D // 2, 2).norm(dim=-1).double(),
                          xn.reshape(B, L, H, D // 2, 2).norm(dim=-1), rtol=1e-5, atol=1e-6)
    ident = ops.qk_norm_rope_f32(x, w, torch.ones(L, D // 2), torch.zeros(L, D // 2), 1e-6)
    assert torch.allclose(ident.double(), xn, rtol=1e-6, atol=1e-6)


def test_planted_sign_mistake_in_rotation_is_caught():
    g = torch.Generator().manual_seed(8)
    B, L, H, D = 1, 5, 2, 64
    x = torch.randn(B, L, H, D, generator=g)
    w = torch.ones(D)
    ang = torch.randn(L, D // 2, generator=g)
    xn = ops.rmsnorm_f32(x, w, 1e-6)
    c = ang.cos().reshape(L, 1, D // 2)
    s = ang.sin().reshape(L, 1, D // 2)
    wrong = torch.empty_like(xn)
    wrong[..., 0::2] = xn[..., 0::2] * c + xn[..., 1::2] * s   # sign slip
    wrong[..., 1::2] = xn[..., 0::2] * s + xn[..., 1::2] * c
    ref = _complex_rope(xn, ang.cos(), ang.sin())
    assert not torch.allclose(wrong.double(), ref, rtol=1e-3, atol=1e-3)


def test_rope_grid_tables_closed_form():
    frames, gh, gw, t0 = 2, 5, 7, 21
    dims = (44, 42, 42)
    cos, sin = ops.rope_grid_tables(frames, gh, gw, t0, dims, 10000.0)
    L, D = cos.shape
    assert (L, D) == (frames * gh * gw, 128)
    n = torch.arange(L)
    t = (t0 + n // (gh * gw)).double()
    h = ((n % (gh * gw)) // gw).double()
    w = (n % gw).double()
    cols_c, cols_s = [], []
    for dim, pos in zip(dims, (t, h, w)):
        f = 1.0 / (10000.0 ** (torch.arange(0, dim, 2).double() / dim))
        a = pos[:, None] * f[None, :]
        cols_c.append(a.cos().repeat_interleave(2, 1))
        cols_s.append(a.sin().repeat_interleave(2, 1))
    ref_c, ref_s = torch.cat(cols_c, 1), torch.cat(cols_s, 1)
    # fp32 angle rounding at |angle| <= 77 rad moves cos/sin by < 1e-5
    assert torch.allclose(cos.double(), ref_c, atol=2e-5)
    assert torch.allclose(sin.double(), ref_s, atol=2e-5)
    assert torch.allclose(cos.double() ** 2 + sin.double() ** 2, torch.ones(L, D, dtype=torch.float64), atol=1e-6)


def test_source_id_composition_is_angle_addition():
    frames, gh, gw, t0 = 1, 3, 4, 5
    dims = (16, 56, 56)
    c0, s0 = ops.rope_grid_tables(frames, gh, gw, t0, dims, 256.0)
    c1, s1 = ops.rope_grid_tables(frames, gh, gw, t0, dims, 256.0, source_id=2.0, source_theta=256.0)
    a0 = torch.atan2(s0.double(), c0.double())
    fr = 1.0 / (256.0 ** (torch.arange(0, 128, 2).double() / 128))
    ar = (2.0 * fr).repeat_interleave(2)
    ref_c, ref_s = torch.cos(a0 + ar), torch.sin(a0 + ar)
    assert torch.allclose(c1.double(), ref_c, atol=1e-5)
    assert torch.allclose(s1.double(), ref_s, atol=1e-5)


def test_ring_slots():
    assert ops.ring_slots(3, 7, 0) == [0, 1, 2]
    assert ops.ring_slots(3, 7, 6) == [6, 0, 1]


def test_gelu_tanh_oracle_matches_float64_closed_form():
    """gelu_tanh_f32 (torch's fp32 kernel) against the formula in float64 with
    math.tanh: within a few fp32 ulps where 1 + tanh(u) does not cancel, and
    within one fp32 step of tanh near -1 (2^-24 * 0.5|x|) where it does; known
    values; the erf form (approximate="none"), a plausible slip, differs."""
    xs = torch.cat([torch.linspace(-12, 12, 20001), torch.tensor([0.0, -0.0, 1e-30, -1e-30, 1e10])])
    got = ops.gelu_tanh_f32(xs)
    c = math.sqrt(2.0 / math.pi)
    for x, g in zip(xs.tolist(), got.tolist()):
        want = 0.5 * x * (1.0 + math.tanh(c * (x + 0.044715 * x ** 3)))
        tol = 4 * abs(want) * 2.0 ** -23 + 0.5 * abs(x) * 2.0 ** -23
        assert abs(g - want) <= tol, (x, g, want)
    # 0.5 (1 + tanh(sqrt(2/pi) * 1.044715)) = 0.841191990...
    assert abs(ops.gelu_tanh_f32(torch.tensor([1.0])).item() - 0.8411919906) < 1e-7
    assert ops.gelu_tanh_f32(torch.tensor([0.0])).item() == 0.0
    special = ops.gelu_tanh_f32(torch.tensor([float("inf"), float("-inf"), float("nan"), -20.0]))
    assert special[0].item() == float("inf") and math.isnan(special[1].item())
    assert math.isnan(special[2].item()) and special[3].item() == 0.0
    erf_form = F.gelu(xs, approximate="none")
    assert (erf_form - got).abs().max().item() > 1e-4


def test_gelu_quant_oracle_quantizes_the_rounded_activation():
    """The fused op's oracle quantizes the bf16 activation torch would return:
    bytes and scales equal the C encoder's on that activation, and a planted
    slip (quantizing the fp32 activation) changes scales."""
    g = torch.Generator().manual_seed(5)
    # rows whose largest activation is not simply x (gelu(x) = x only for large x)
    x = (0.5 * torch.randn(32, 512, generator=g)).to(torch.bfloat16)
    q, s, a = ops.gelu_tanh_quant_fp8(x)
    assert a.dtype == torch.bfloat16
    assert torch.equal(a, ops.gelu_tanh_f32(x).to(torch.bfloat16))
    qc, sc = fp8ref.per_token_quant(a.float().numpy())
    assert np.array_equal(q.numpy(), qc) and np.array_equal(s.numpy(), sc)
    _, s_slip = ops.per_token_quant_fp8(ops.gelu_tanh_f32(x))
    assert not torch.equal(s_slip, s)


def test_norm_quant_oracle_quantizes_the_rounded_y():
    """The FP8 epilogue quantizes the 16-bit y the unfused op returns: its
    scale is amax|bf16 y| / 448 (checked against torch's max and the C
    encoder's bytes), and a planted slip (quantizing the fp32 y instead)
    changes scales on random rows."""
    g = torch.Generator().manual_seed(3)
    M, N = 16, 256
    x = torch.randn(M, N, generator=g).to(torch.bfloat16)
    res = torch.randn(M, N, generator=g).to(torch.bfloat16)
    gate = torch.randn(N, generator=g).to(torch.bfloat16)
    sc = (0.2 * torch.randn(N, generator=g)).to(torch.bfloat16)
    sh = (0.2 * torch.randn(N, generator=g)).to(torch.bfloat16)
    new_res, q, s, y = ops.norm_scale_shift_quant_fp8(x, res, gate, None, None, sc, sh, 0, 1e-6)
    assert torch.equal(new_res, torch.addcmul(res.float(), x.float(), gate.float()).to(torch.bfloat16))
    assert y.dtype == torch.bfloat16
    assert torch.equal(s, (y.float().abs().amax(-1) / 448.0))
    qc, sc_c = fp8ref.per_token_quant(y.float().numpy())
    assert np.array_equal(q.numpy(), qc) and np.array_equal(s.numpy(), sc_c)
    y32 = ops.norm_scale_shift_f32(new_res, None, None, sc, sh, 0, 1e-6)
    _, s_slip = ops.per_token_quant_fp8(y32)
    assert not torch.equal(s_slip, s)


def test_apply_rotary_emb_oracle_pins():
    """Identity and quarter-turn tables give exact results; a general table
    matches complex multiplication (x0 + i x1)(c + i s) in float64 to the
    fp32 rounding; a planted sign slip in sin is caught."""
    g = torch.Generator().manual_seed(11)
    B, T, H, D = 2, 5, 3, 16
    x = torch.randn(B, T, H, D, generator=g).to(torch.bfloat16)
    one, zero = torch.ones(T, D), torch.zeros(T, D)
    assert torch.equal(ops.apply_rotary_emb(x, one, zero), x)
    quarter = ops.apply_rotary_emb(x, zero, one).float()
    x0, x1 = x.float()[..., 0::2], x.float()[..., 1::2]
    assert torch.equal(quarter[..., 0::2], (-x1).to(torch.bfloat16).float())
    assert torch.equal(quarter[..., 1::2], x0)
    ang = torch.rand(T, D // 2, generator=g, dtype=torch.float64) * 40
    cos = ang.cos().float().repeat_interleave(2, 1)
    sin = ang.sin().float().repeat_interleave(2, 1)
    got = ops.apply_rotary_emb(x, cos, sin).float()
    z = torch.complex(x0.double(), x1.double()) * torch.complex(
        cos[:, 0::2].double(), sin[:, 0::2].double())[None, :, None, :]
    ref = torch.stack([z.real, z.imag], -1).flatten(-2)
    ulp = 2.0 ** (torch.floor(torch.log2(ref.abs().clamp_min(1e-30))) - 7)
    assert ((got.double() - ref).abs() <= ulp * 1.01 + 1e-6).all()

    def slipped(x, c, s):
        return (x.float() * c.reshape(1, T, 1, D) - ops.rotate_half(x) * s.reshape(1, T, 1, D)
                ).to(x.dtype)
    bad = slipped(x, cos, sin).float()
    assert not ((bad.double() - ref).abs() <= ulp * 1.01 + 1e-6).all()


def test_commit_kv_oracle_touches_only_its_segment():
    g = torch.Generator().manual_seed(12)
    L, B, T, P, H, D = 2, 1, 4, 12, 2, 8
    pool_k = torch.randn(L, B, P, H, D, generator=g).to(torch.bfloat16)
    pool_v = torch.randn(L, B, P, H, D, generator=g).to(torch.bfloat16)
    sk = torch.randn(L, B, T, H, D, generator=g).to(torch.bfloat16)
    sv = torch.randn(L, B, T, H, D, generator=g).to(torch.bfloat16)
    cos, sin = torch.ones(T, D), torch.zeros(T, D)
    pk, pv = ops.commit_kv(pool_k, pool_v, sk, sv, 4, cos, sin)
    assert torch.equal(pk[:, :, 4:8], sk) and torch.equal(pv[:, :, 4:8], sv)
    assert torch.equal(pk[:, :, :4], pool_k[:, :, :4]) and torch.equal(pk[:, :, 8:], pool_k[:, :, 8:])
    assert torch.equal(pv[:, :, :4], pool_v[:, :, :4]) and torch.equal(pv[:, :, 8:], pool_v[:, :, 8:])


def test_fp8_gemm_oracle_accumulation_is_exact():
    """The float64 accumulation of e4m3fn products equals an exact int64
    matmul of the same values scaled by 2^9 (each code is a multiple of
    2^-9), on random codes spanning the whole range, NaN excluded."""
    g = torch.Generator().manual_seed(2)
    M, K, N = 9, 512, 7
    codes_a = torch.randint(0, 256, (M, K), generator=g, dtype=torch.uint8)
    codes_b = torch.randint(0, 256, (K, N), generator=g, dtype=torch.uint8)
    codes_a[(codes_a & 0x7F) == 0x7F] = 0x7E
    codes_b[(codes_b & 0x7F) == 0x7F] = 0x7E
    a = codes_a.view(torch.float8_e4m3fn)
    b = codes_b.view(torch.float8_e4m3fn)
    ai = (a.float().double() * 512).round().long()
    bi = (b.float().double() * 512).round().long()
    assert torch.equal(ai.double() / 512, a.float().double())
    exact = (ai @ bi).double() / 2.0 ** 18
    _, acc, _ = ops.fp8_scaled_mm(a, b, torch.ones(M), torch.ones(N), torch.bfloat16)
    assert torch.equal(acc, exact)


def test_fp8_decode_matches_c_encoder_table():
    codes = torch.arange(256, dtype=torch.uint8)
    vals = codes.view(torch.float8_e4m3fn).float()
    for c in range(256):
        ref = fp8ref.decode(c)
        if math.isnan(ref):
            assert math.isnan(vals[c].item())
        else:
            assert vals[c].item() == ref, c


def test_fp8_gemm_oracle_epilogue_order():
    """scale_a * (acc * scale_b) + bias with fp32 roundings between, not
    (scale_a * scale_b) * acc: a row where the two orders differ in fp32."""
    a = torch.tensor([[12.0, 0.0]]).to(torch.float8_e4m3fn)
    b = torch.tensor([[1.0], [0.0]]).to(torch.float8_e4m3fn)
    sa = torch.tensor([1032143960], dtype=torch.int32).view(torch.float32)   # 0.0650717616...
    sb = torch.tensor([1031643931], dtype=torch.int32).view(torch.float32)   # 0.0619231276...
    out, acc, _ = ops.fp8_scaled_mm(a, b, sa, sb, torch.float32)
    t = torch.tensor(12.0, dtype=torch.float32) * sb[0]
    assert out.item() == (sa[0] * t).item()
    assert out.item() != ((sa[0] * sb[0]) * torch.tensor(12.0)).item()
