"""The row ops on tensors past 2^31 elements (4.3 GB of bf16): 64-bit row
offsets end to end (the C ABI's int64 sizes and strides, the kernels' row
index times stride). Inputs are generated on the device; the rows on either
side of the 2^31-element boundary, the first, a middle and the last rows are
checked against the CPU oracle to the same bars as the ops' own tests
(per_token_quant_fp8.cu:56-82 and RMSNorm -> FP8 bit-exact, rmsnorm.cu:41-60 /
fused_norm_scale_shift.cu:88-142 / fused_qknorm_rope_3d_kernel.cu:98-142
within 1 bf16 ulp).
"""
from __future__ import annotations

import pytest
import torch

from oracle import ops
from helpers import assert_within_ulp, assert_bf16_within_ulp

pytestmark = pytest.mark.gpu

N = 3072
EDGE = (1 << 31) // N                  # first row at or past element 2^31
M = EDGE + 4096
ROWS = [0, 1, M // 2, EDGE - 1, EDGE, EDGE + 1, M - 2, M - 1]


@pytest.fixture(scope="module")
def big(dev):
    """x [M, 3072] bf16 with M * 3072 > 2^31 and a bf16 weight row, shared by
    the tests of this module and freed after them."""
    g = torch.Generator(device=dev).manual_seed(2031)
    x = torch.randn(M, N, generator=g, device=dev, dtype=torch.bfloat16)
    w = (1 + 0.1 * torch.randn(N, generator=g, device=dev, dtype=torch.float32)).to(torch.bfloat16)
    assert x.numel() > (1 << 31)
    yield x, w
    del x
    torch.cuda.empty_cache()


def fp8_rows(q):
    """The checked rows of an e4m3fn tensor as their bytes, on the CPU."""
    return q.view(torch.uint8)[ROWS].cpu()


def test_per_token_quant_past_2_31_elements(big):
    import joyomni_ops as jo
    x, _ = big
    q = torch.empty(M, N, dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.full((M, 1), -1.0, dtype=torch.float32, device=x.device)
    jo.sgl_per_token_quant_fp8(x, q, s)
    torch.cuda.synchronize()
    qo, so = ops.per_token_quant_fp8(x[ROWS].cpu())
    assert torch.equal(fp8_rows(q), qo), "fp8 bytes differ"
    assert torch.equal(s[ROWS].cpu().reshape(-1), so.reshape(-1)), "scales differ"
    del q, s


@pytest.mark.parametrize("group", [0, 128])
def test_rmsnorm_quant_past_2_31_elements(big, group):
    import joyomni_ops as jo
    x, w = big
    q = torch.empty(M, N, dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.full((M,) if group == 0 else (M, N // group), -1.0, dtype=torch.float32,
                   device=x.device)
    jo.rmsnorm_quant_fp8(x, w, 1e-6, q, s, group)
    torch.cuda.synchronize()
    qo, so, _ = ops.rmsnorm_quant_fp8(x[ROWS].cpu(), w.cpu(), 1e-6, group)
    assert torch.equal(s[ROWS].cpu(), so), "scales differ"
    assert torch.equal(fp8_rows(q), qo), "fp8 bytes differ"
    del q, s


def test_rmsnorm_past_2_31_elements(big):
    import joyomni_ops as jo
    x, w = big
    y = jo.rmsnorm(x, w, 1e-6)
    torch.cuda.synchronize()
    ref = ops.rmsnorm_f32(x[ROWS].cpu(), w.cpu(), 1e-6)
    assert_within_ulp(y[ROWS].cpu(), ref, torch.bfloat16, ref.abs().amax(dim=-1, keepdim=True),
                      what="rmsnorm past 2^31")
    del y


def test_layernorm_modulate_past_2_31_elements(big):
    """Per-row [M, N] scale and shift, as the reference caller materialises
    them (three 4.3 GB inputs and the output)."""
    import joyomni_ops as jo
    x, _ = big
    g = torch.Generator(device=x.device).manual_seed(7)
    sc = (0.2 * torch.randn(M, N, generator=g, device=x.device, dtype=torch.bfloat16))
    sh = (0.2 * torch.randn(M, N, generator=g, device=x.device, dtype=torch.bfloat16))
    y = jo.fused_norm_scale_shift(x, None, None, sc, sh, "layer", 1e-6)
    torch.cuda.synchronize()
    ref = ops.norm_scale_shift_f32(x[ROWS].cpu(), None, None, sc[ROWS].cpu(), sh[ROWS].cpu(), 0,
                                   1e-6)
    assert_within_ulp(y[ROWS].cpu(), ref, torch.bfloat16, ref.abs().amax(dim=-1, keepdim=True),
                      what="layernorm + modulate past 2^31")
    del sc, sh, y


def test_qk_norm_rope_past_2_31_elements(dev):
    """q, k [1, L, 32, 128] with L * 32 * 128 > 2^31, in place, from bf16
    tables; the heads of the tokens on either side of element 2^31 checked."""
    import joyomni_ops as jo
    H, D = 32, 128
    L = (1 << 31) // (H * D) + 64
    edge = (1 << 31) // (H * D)
    toks = [0, L // 2, edge - 1, edge, L - 1]
    g = torch.Generator(device=dev).manual_seed(31)
    q = torch.randn(1, L * H, D, generator=g, device=dev, dtype=torch.bfloat16)
    k = torch.randn(1, L * H, D, generator=g, device=dev, dtype=torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    cos = torch.randn(L, D // 2, generator=g, device=dev, dtype=torch.bfloat16)
    sin = torch.randn(L, D // 2, generator=g, device=dev, dtype=torch.bfloat16)
    q0 = q.view(L, H, D)[toks].cpu()
    k0 = k.view(L, H, D)[toks].cpu()
    jo.fused_qk_norm_rope_3d_paired(q, k, L, H, 1e-6, qw, kw, cos, sin)
    torch.cuda.synchronize()
    for name, before, after, w in (("q", q0, q, qw), ("k", k0, k, kw)):
        ref = ops.qk_norm_rope_f32(before.reshape(1, len(toks), H, D), w.cpu(), cos[toks].cpu(),
                                   sin[toks].cpu(), 1e-6)
        out = after.view(L, H, D)[toks].cpu().reshape(1, len(toks), H, D)
        assert_bf16_within_ulp(out, ref, ref.abs().amax(dim=-1, keepdim=True),
                               what=f"{name} past 2^31")
    del q, k
    torch.cuda.empty_cache()
