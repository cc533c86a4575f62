"""GPU parity of the norm + AdaLN -> FP8 epilogue (jo_norm_scale_shift_quant_fp8,
torch op norm_scale_shift_quant_fp8, DiT shims *_fp8).

Bar:
  - the updated residual is bit-exact against the oracle (one fp32 add or
    product-then-add, one rounding), as for the add + LayerNorm op;
  - the fused op equals the unfused pair byte for byte: its fp8 bytes and
    scales are bit-exact against the oracle's per-token quantizer
    (per_token_quant_fp8.cu:56-82 restated, pinned by the C brute-force
    encoder) applied to the 16-bit y that jo_fused_norm_scale_shift returns
    for the same row on the device;
  - that y is within 1 ulp of the fp32-accumulated oracle (the norm ops' bar).
"""
from __future__ import annotations

import pytest
import torch

from helpers import assert_within_ulp
from oracle import ops

pytestmark = pytest.mark.gpu

SHAPES = [(7, 64), (33, 512), (17, 3072), (5, 4096), (3, 16384), (4, 100), (2, 40000)]
NORM = {"layer": 0, "rms": 1}


def make_case(M, N, dtype, mode, per_row, affine, seed):
    g = torch.Generator().manual_seed(seed)
    shape = (M, N) if per_row else (N,)
    t = dict(
        x=(torch.randn(M, N, generator=g) * 2 + 0.3).to(dtype),
        residual=torch.randn(M, N, generator=g).to(dtype) if mode != "plain" else None,
        gate=torch.randn(shape, generator=g).to(dtype) if mode == "add_gate" else None,
        gamma=(1 + 0.1 * torch.randn(N, generator=g)).to(dtype) if affine else None,
        beta=(0.1 * torch.randn(N, generator=g)).to(dtype) if affine else None,
        scale=(0.2 * torch.randn(shape, generator=g)).to(dtype),
        shift=(0.2 * torch.randn(shape, generator=g)).to(dtype),
    )
    return t


def to_dev(t, dev):
    return {k: (v.to(dev) if v is not None else None) for k, v in t.items()}


def ptr(v):
    return v.data_ptr() if v is not None else None


def run_fused(abi, stream, d, M, N, dtype, norm, eps, x_stride=None, q_stride=None):
    """The fused op through the C ABI; returns (q uint8 [M, N], s [M]) on the device."""
    xs = x_stride or N
    qs = q_stride or N
    q = torch.full((M, qs), 0x55, dtype=torch.uint8, device=d["x"].device)
    s = torch.full((M,), -1.0, dtype=torch.float32, device=d["x"].device)
    rs = N if d["scale"].dim() == 2 else 0
    abi.call("jo_norm_scale_shift_quant_fp8", d["x"].data_ptr(), xs, ptr(d["residual"]), N,
             ptr(d["gate"]), rs, ptr(d["gamma"]), ptr(d["beta"]), d["scale"].data_ptr(), rs,
             d["shift"].data_ptr(), rs, 1, q.data_ptr(), qs, s.data_ptr(), M, N,
             abi.dtype_code(dtype), NORM[norm], eps, stream)
    return q, s


def run_unfused_y(abi, stream, src, d, M, N, dtype, norm, eps, y_stride=None):
    """jo_fused_norm_scale_shift on the (updated) source rows: the y the pair
    stores. y_stride picks the same kernel (vector or element-wise) as the
    fused call's q stride does, so both sum a row in the same order."""
    ys = y_stride or N
    y = torch.empty(M, ys, dtype=dtype, device=src.device)
    rs = N if d["scale"].dim() == 2 else 0
    abi.call("jo_fused_norm_scale_shift", src.data_ptr(), N, ptr(d["gamma"]),
             ptr(d["beta"]), d["scale"].data_ptr(), rs, d["shift"].data_ptr(), rs, y.data_ptr(),
             ys, M, N, abi.dtype_code(dtype), NORM[norm], eps, stream)
    return y[:, :N]


def check_case(t, d, q, s, y_dev, norm, eps, what):
    """residual bit-exact, (q, s) == quant(device y) bit-exact, y within 1 ulp."""
    new_res, q_ref, s_ref, _ = ops.norm_scale_shift_quant_fp8(
        t["x"], t["residual"], t["gate"], t["gamma"], t["beta"], t["scale"], t["shift"],
        NORM[norm], eps, y=y_dev)
    if new_res is not None:
        got = d["residual"].cpu()
        assert torch.equal(got.view(torch.int16), new_res.view(torch.int16)), f"{what}: residual"
    assert torch.equal(q.cpu(), q_ref), f"{what}: fp8 bytes differ from quant(unfused y)"
    assert torch.equal(s.cpu().view(torch.int32), s_ref.view(torch.int32)), f"{what}: scales"
    src = new_res if new_res is not None else t["x"]
    ref = ops.norm_scale_shift_f32(src, t["gamma"], t["beta"], t["scale"], t["shift"],
                                   NORM[norm], eps)
    if torch.isfinite(ref).all():
        assert_within_ulp(y_dev, ref, y_dev.dtype, ref.abs().amax(dim=-1, keepdim=True),
                          what=f"{what}: y")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N", SHAPES)
@pytest.mark.parametrize("norm", ["layer", "rms"])
@pytest.mark.parametrize("mode", ["plain", "add", "add_gate"])
@pytest.mark.parametrize("per_row", [False, True])
def test_norm_quant_matches_unfused_pair(abi, dev, stream_handle, dtype, M, N, norm, mode,
                                         per_row):
    t = make_case(M, N, dtype, mode, per_row, affine=(M % 2 == 1), seed=M * 7 + N)
    d = to_dev(t, dev)
    q, s = run_fused(abi, stream_handle, d, M, N, dtype, norm, 1e-6)
    src = d["residual"] if mode != "plain" else d["x"]
    y = run_unfused_y(abi, stream_handle, src, d, M, N, dtype, norm, 1e-6)
    torch.cuda.synchronize()
    check_case(t, d, q, s, y.cpu(), norm, 1e-6, f"{norm}/{mode} {dtype} [{M},{N}] per_row={per_row}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("N", [3072, 4096, 100])
def test_norm_quant_nonfinite_and_special_rows(abi, dev, stream_handle, dtype, N):
    """NaN / inf inputs, a constant row (LN -> y = shift), a zero row with zero
    modulation (scale 0, inv 0), and y overflowing the 16-bit range."""
    M = 8
    t = make_case(M, N, dtype, "add", False, affine=False, seed=N)
    t["x"][0, 5] = float("nan")
    t["x"][1, 7] = float("inf")
    t["residual"][2, :] = 0.75
    t["x"][2, :] = 0.25
    t["x"][3, :] = 0
    t["residual"][3, :] = 0
    t["x"][4, 1] = -float("inf")
    t["x"][4, 2] = float("inf")
    big = 60000.0 if dtype == torch.float16 else 3e38
    t["x"][5, :] = torch.linspace(-big, big, N).to(dtype)
    t["residual"][5, :] = 0
    t0 = dict(t)
    t0["shift"] = torch.zeros_like(t["shift"])
    t0["scale"] = torch.zeros_like(t["scale"])
    for case in (t, t0):
        d = to_dev(case, dev)
        q, s = run_fused(abi, stream_handle, d, M, N, dtype, "layer", 1e-6)
        y = run_unfused_y(abi, stream_handle, d["residual"], d, M, N, dtype, "layer", 1e-6)
        torch.cuda.synchronize()
        new_res, q_ref, s_ref, _ = ops.norm_scale_shift_quant_fp8(
            case["x"], case["residual"], None, None, None, case["scale"], case["shift"], 0, 1e-6,
            y=y.cpu())
        got = d["residual"].cpu()
        same = (got.view(torch.int16) == new_res.view(torch.int16)) | (got.isnan() & new_res.isnan())
        bad = (~same).nonzero()
        assert bad.numel() == 0, (f"residual differs at {bad[:4].tolist()}: "
                                  f"{got[tuple(bad[0])]} vs {new_res[tuple(bad[0])]}")
        assert torch.equal(q.cpu(), q_ref), f"special rows {dtype} N={N}"
        assert torch.equal(s.cpu().view(torch.int32), s_ref.view(torch.int32))


def test_norm_quant_strided_and_generic_paths(abi, dev, stream_handle):
    """x with a padded row stride; q with a row stride that is not a multiple of
    8 (element-wise kernel); both against the unfused pair."""
    M, N = 9, 3072
    for xs, qs in ((N + 64, N), (N, N + 4), (N + 8, N + 12)):
        t = make_case(M, N, torch.bfloat16, "add_gate", True, affine=True, seed=xs + qs)
        xpad = torch.zeros(M, xs, dtype=torch.bfloat16)
        xpad[:, :N] = t["x"]
        d = to_dev(t, dev)
        d["x"] = xpad.to(dev)
        q, s = run_fused(abi, stream_handle, d, M, N, torch.bfloat16, "layer", 1e-6, x_stride=xs,
                         q_stride=qs)
        y = run_unfused_y(abi, stream_handle, d["residual"], d, M, N, torch.bfloat16, "layer", 1e-6,
                          y_stride=qs)
        torch.cuda.synchronize()
        assert (q.cpu()[:, N:] == 0x55).all(), "bytes beyond N of a padded q row were written"
        check_case(t, d, q[:, :N], s, y.cpu(), "layer", 1e-6, f"strided xs={xs} qs={qs}")


def test_norm_quant_rejects(abi, dev, stream_handle):
    x = torch.zeros(4, 64, dtype=torch.float32, device=dev)
    q = torch.empty(4, 64, dtype=torch.uint8, device=dev)
    s = torch.empty(4, dtype=torch.float32, device=dev)
    with pytest.raises(RuntimeError, match="bf16 or fp16"):
        abi.call("jo_norm_scale_shift_quant_fp8", x.data_ptr(), 64, None, 0, None, 0, None, None,
                 x.data_ptr(), 0, x.data_ptr(), 0, 1, q.data_ptr(), 64, s.data_ptr(), 4, 64,
                 abi.dtype_code(torch.float32), 0, 1e-6, stream_handle)
    xb = x.to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="gate needs a residual"):
        abi.call("jo_norm_scale_shift_quant_fp8", xb.data_ptr(), 64, None, 0, xb.data_ptr(), 0,
                 None, None, xb.data_ptr(), 0, xb.data_ptr(), 0, 1, q.data_ptr(), 64, s.data_ptr(),
                 4, 64, abi.dtype_code(torch.bfloat16), 0, 1e-6, stream_handle)


@pytest.mark.parametrize("B,L,N", [(2, 300, 3072), (3, 17, 512)])
def test_norm_quant_per_sample_modulation(abi, dev, stream_handle, B, L, N):
    """One call for a batch (mod_rows = L, gate / scale / shift [B, N]): the
    residual bit-exact against the oracle, the fp8 bytes and scales bit-exact
    against the C quantizer applied to the y the unfused device op stores for
    the same rows, and that y within 1 ulp of the oracle."""
    import joyomni_ops as jo
    dtype = torch.bfloat16
    M = B * L
    g = torch.Generator().manual_seed(B * 10 + L + N)
    x = torch.randn(M, N, generator=g).to(dtype)
    res = torch.randn(M, N, generator=g).to(dtype)
    gate = torch.randn(B, N, generator=g).to(dtype)
    sc = (0.2 * torch.randn(B, N, generator=g)).to(dtype)
    sh = (0.2 * torch.randn(B, N, generator=g)).to(dtype)
    xd, rd, gd, scd, shd = (t.to(dev) for t in (x, res, gate, sc, sh))
    r2 = rd.clone()
    q = torch.full((M, N), 0x55, dtype=torch.uint8, device=dev)
    s = torch.full((M,), -1.0, dtype=torch.float32, device=dev)
    abi.call("jo_norm_scale_shift_quant_fp8", xd.data_ptr(), N, rd.data_ptr(), N, gd.data_ptr(),
             N, None, None, scd.data_ptr(), N, shd.data_ptr(), N, L, q.data_ptr(), N,
             s.data_ptr(), M, N, abi.dtype_code(dtype), 0, 1e-6, stream_handle)
    ex = lambda t: t.repeat_interleave(L, dim=0)  # noqa: E731
    y_dev = jo.fused_add_layernorm_scale_shift(xd, r2, ex(scd), ex(shd), gate=ex(gd), eps=1e-6)
    torch.cuda.synchronize()
    new_res, qo, so, yo = ops.norm_scale_shift_quant_fp8(x, res, ex(gate), None, None, ex(sc),
                                                         ex(sh), 0, 1e-6, y=y_dev.cpu())
    assert torch.equal(rd.cpu(), new_res) and torch.equal(r2.cpu(), new_res), "residual"
    assert torch.equal(q.cpu(), qo), "fp8 bytes"
    assert torch.equal(s.cpu(), so), "scales"
    ref = ops.norm_scale_shift_f32(new_res, None, None, ex(sc), ex(sh), 0, 1e-6)
    assert_within_ulp(yo, ref, dtype, ref.abs().amax(-1, keepdim=True), what="y per sample")


def test_torch_op_and_dit_shims(dev):
    """Torch op with and without a residual, and the DiT shims against the
    unfused DiT calls (fused_layernorm_modulate / fused_add_gate_layernorm_modulate
    followed by quantize_activation_fp8), batch 2."""
    import joyomni_ops as jo
    from joyomni_ops import dit_ops
    B, L, D = 2, 300, 3072
    g = torch.Generator().manual_seed(5)
    x = torch.randn(B, L, D, generator=g).to(torch.bfloat16).to(dev)
    res = torch.randn(B, L, D, generator=g).to(torch.bfloat16).to(dev)
    gate = torch.randn(B, D, generator=g).to(torch.bfloat16).to(dev)
    shift = (0.2 * torch.randn(B, D, generator=g)).to(torch.bfloat16).to(dev)
    scale = (0.2 * torch.randn(B, D, generator=g)).to(torch.bfloat16).to(dev)

    q1, s1 = dit_ops.layernorm_modulate_fp8(x, shift, scale)
    q1r, s1r = dit_ops.quantize_activation_fp8(dit_ops.fused_layernorm_modulate(x, shift, scale))
    torch.cuda.synchronize()
    assert torch.equal(q1.view(torch.uint8), q1r.view(torch.uint8))
    assert torch.equal(s1, s1r) and s1.shape == (B * L, 1)

    r_a, r_b = res.clone(), res.clone()
    _, q2, s2 = dit_ops.fused_add_gate_layernorm_modulate_fp8(r_a, x, gate, shift, scale)
    _, y2 = dit_ops.fused_add_gate_layernorm_modulate(r_b, x, gate, shift, scale)
    q2r, s2r = dit_ops.quantize_activation_fp8(y2)
    torch.cuda.synchronize()
    assert torch.equal(r_a, r_b)
    assert torch.equal(q2.view(torch.uint8), q2r.view(torch.uint8))
    assert torch.equal(s2, s2r)

    # Torch op directly, RMS without a residual, per-row modulation.
    M, N = 64, 1024
    xr = torch.randn(M, N, generator=g).to(torch.float16).to(dev)
    sc = (0.2 * torch.randn(M, N, generator=g)).to(torch.float16).to(dev)
    sh = (0.2 * torch.randn(M, N, generator=g)).to(torch.float16).to(dev)
    q3 = torch.empty(M, N, dtype=torch.float8_e4m3fn, device=dev)
    s3 = torch.empty(M, dtype=torch.float32, device=dev)
    jo.norm_scale_shift_quant_fp8(xr, sc, sh, q3, s3, norm_type="rms")
    y3 = jo.fused_norm_scale_shift(xr, None, None, sc, sh, "rms", 1e-6)
    q3r = torch.empty_like(q3)
    s3r = torch.empty_like(s3)
    jo.sgl_per_token_quant_fp8(y3, q3r, s3r)
    torch.cuda.synchronize()
    assert torch.equal(q3.view(torch.uint8), q3r.view(torch.uint8))
    assert torch.equal(s3, s3r)
    with pytest.raises(RuntimeError, match="output_s"):
        jo.norm_scale_shift_quant_fp8(xr, sc, sh, q3, torch.empty(M + 1, device=dev))


@pytest.mark.parametrize("M,N", [(17, 3072), (33, 512)])
@pytest.mark.parametrize("norm", ["layer", "rms"])
def test_norm_quant_per_row_gate_broadcast_modulation(abi, dev, stream_handle, M, N, norm):
    """A gate with a row per row of x beside broadcast scale / shift (the
    bounds-free kernel for rows that fill the lanes exactly; M leaves a partly
    filled last workgroup): residual bit-exact, bytes and scales those of the
    unfused pair, and nothing written past row M."""
    dtype = torch.bfloat16
    t = make_case(M, N, dtype, "add_gate", False, False, M * 7 + N)
    g = torch.Generator().manual_seed(M + N)
    t["gate"] = torch.randn(M, N, generator=g).to(dtype)
    d = to_dev(t, dev)
    q = torch.full((M + 2, N), 0x55, dtype=torch.uint8, device=dev)
    s = torch.full((M + 2,), -1.0, dtype=torch.float32, device=dev)
    abi.call("jo_norm_scale_shift_quant_fp8", d["x"].data_ptr(), N, d["residual"].data_ptr(), N,
             d["gate"].data_ptr(), N, None, None, d["scale"].data_ptr(), 0, d["shift"].data_ptr(),
             0, 1, q.data_ptr(), N, s.data_ptr(), M, N, abi.dtype_code(dtype), NORM[norm], 1e-6,
             stream_handle)
    y = run_unfused_y(abi, stream_handle, d["residual"], d, M, N, dtype, norm, 1e-6)
    torch.cuda.synchronize()
    check_case(t, d, q[:M], s[:M], y.cpu(), norm, 1e-6, f"per-row gate [{M},{N}] {norm}")
    assert bool((q[M:] == 0x55).all()) and bool((s[M:] == -1.0).all()), "rows past M written"
