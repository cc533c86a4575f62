"""GPU parity of gelu_tanh_quant_fp8: the MLP activation gelu(h, approximate="tanh")
(dit.py:91-92, 433) and the next Fp8Linear's per-token FP8 quantization
(fp8_linear.py:140-166, per_token_quant_fp8.cu:56-82) in one pass.

Two parts, as the op is a floating-point activation followed by an integer-exact
quantization:
  - the activation the kernel quantized (written to output_act) is within 1 ulp
    of its dtype (the subnormal spacing for fp16 subnormals) of the fp32 formula (the oracle, torch's CPU kernel), plus one
    two fp32 steps of tanh near -1 (2^-23) scaled by 0.5|x| where 1 + tanh(u)
    cancels (x below about -3: the formula itself only resolves the result to
    that step); NaN and inf positions match;
  - the FP8 bytes and scales are bit-exact against the oracle's per-token
    quantization of that same activation, and identical without output_act.
"""
from __future__ import annotations

import pytest
import torch

from oracle import ops
from joyomni_ops import workloads as W

pytestmark = pytest.mark.gpu

MANT = {torch.bfloat16: 7, torch.float16: 10}
# spacing of the dtype's subnormals: fp16 tail activations (|x| ~ 4-5 gives
# |gelu| ~ 1e-5 .. 1e-7) round on this grid
SUBNORMAL_ULP = {torch.bfloat16: 2.0 ** -133, torch.float16: 2.0 ** -24}


def inputs(M, K, dtype, seed, special=False):
    g = torch.Generator().manual_seed(seed)
    x = 3.0 * torch.randn(M, K, generator=g)
    x = W.with_outliers(x, g)
    if special and M >= 3:
        x[0, :4] = torch.tensor([float("nan"), float("inf"), float("-inf"), 0.0])
        x[1] = 0.0
        x[2, : K // 2] = -20.0
    return x.to(dtype)


def check_activation(act, x, what):
    ref = ops.gelu_tanh_f32(x)
    a = act.float().cpu()
    assert torch.equal(torch.isnan(a), torch.isnan(ref)), f"{what}: NaN pattern"
    inf = torch.isinf(ref)
    assert torch.equal(a[inf], ref[inf]), f"{what}: inf values"
    fin = torch.isfinite(ref)
    mb = MANT[act.dtype]
    ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -126))) - mb)
    ulp = ulp.clamp_min(SUBNORMAL_ULP[act.dtype])
    tol = ulp + 0.5 * x.float().abs() * 2.0 ** -23
    err = (a - ref).abs()
    bad = (err > tol) & fin
    assert not bool(bad.any()), (
        f"{what}: {int(bad.sum())} activations beyond tolerance, max err/tol "
        f"{(err / tol)[fin].max().item():.3f}")


SHAPES = [(3120, 16384, torch.bfloat16), (257, 4096, torch.bfloat16), (64, 3072, torch.float16),
          (33, 1000, torch.bfloat16), (5, 12, torch.float16), (1, 16384, torch.bfloat16)]


@pytest.mark.parametrize("M,K,dtype", SHAPES)
def test_gelu_tanh_quant_fp8(dev, M, K, dtype):
    import joyomni_ops as jo
    print(f"gelu_tanh_quant_fp8 [{M}, {K}] {dtype}", flush=True)
    x = inputs(M, K, dtype, M + K, special=True)
    xd = x.to(dev)
    q = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=dev)
    s = torch.empty(M, 1, dtype=torch.float32, device=dev)
    act = torch.empty(M, K, dtype=dtype, device=dev)
    jo.gelu_tanh_quant_fp8(xd, q, s, act)
    q2 = torch.empty_like(q)
    s2 = torch.empty_like(s)
    jo.gelu_tanh_quant_fp8(xd, q2, s2)
    torch.cuda.synchronize()
    check_activation(act, x, f"[{M}, {K}] {dtype}")
    qo, so, _ = ops.gelu_tanh_quant_fp8(x, act=act.cpu())
    assert torch.equal(q.view(torch.uint8).cpu(), qo), "fp8 bytes differ from the oracle's"
    assert torch.equal(s.cpu().reshape(-1), so), "scales differ from the oracle's"
    assert torch.equal(q2.view(torch.uint8).cpu(), qo) and torch.equal(s2.cpu().reshape(-1), so)


def test_gelu_tanh_quant_fp8_strided_rows(dev):
    """Rows of a wider buffer (row stride > K) through the vector path, and an
    unaligned view through the element-wise path."""
    import joyomni_ops as jo
    M, K = 40, 2048
    x = inputs(M, K + 64, torch.bfloat16, 9)
    xd = x.to(dev)
    for view, what in ((xd[:, :K], "strided"), (xd[:, 4:K + 4], "unaligned")):
        q = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=dev)
        s = torch.empty(M, dtype=torch.float32, device=dev)
        act = torch.empty(M, K, dtype=torch.bfloat16, device=dev)
        jo.gelu_tanh_quant_fp8(view, q, s, act)
        torch.cuda.synchronize()
        xv = view.cpu()
        check_activation(act, xv, what)
        qo, so, _ = ops.gelu_tanh_quant_fp8(xv, act=act.cpu())
        assert torch.equal(q.view(torch.uint8).cpu(), qo) and torch.equal(s.cpu(), so), what


def test_gelu_quantize_activation_fp8_caller(dev):
    """dit_ops.gelu_quantize_activation_fp8 on a [B, L, K] tensor gives the op's
    bytes and [M, 1] scales."""
    import joyomni_ops as jo
    from joyomni_ops import dit_ops
    B, L, K = 2, 100, 4096
    x = inputs(B * L, K, torch.bfloat16, 4).reshape(B, L, K).to(dev)
    x_q, x_s = dit_ops.gelu_quantize_activation_fp8(x)
    q = torch.empty(B * L, K, dtype=torch.float8_e4m3fn, device=dev)
    s = torch.empty(B * L, dtype=torch.float32, device=dev)
    jo.gelu_tanh_quant_fp8(x.reshape(B * L, K), q, s)
    torch.cuda.synchronize()
    assert x_s.shape == (B * L, 1)
    assert torch.equal(x_q.view(torch.uint8).cpu(), q.view(torch.uint8).cpu())
    assert torch.equal(x_s.reshape(-1).cpu(), s.cpu())
