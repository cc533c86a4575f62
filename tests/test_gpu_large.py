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


def test_add_gate_layernorm_modulate_fp8_past_2_31_elements(big):
    """N3 (gated residual + LN + AdaLN -> FP8) on [1, M, 3072]: the updated
    residual bit-exact against the oracle's residual_add, the fp8 bytes and
    scales bit-exact against the quantization of the unfused pair's y (the
    same kernel family and summation order), y within 1 bf16 ulp."""
    from joyomni_ops import dit_ops
    x, _ = big
    g = torch.Generator(device=x.device).manual_seed(9)
    res = torch.randn(1, M, N, generator=g, device=x.device, dtype=torch.bfloat16)
    gate, shift, scale = (0.2 * torch.randn(1, N, generator=g, device=x.device,
                                            dtype=torch.bfloat16) for _ in range(3))
    res0 = res.view(M, N)[ROWS].cpu()
    res_out, q, s = dit_ops.fused_add_gate_layernorm_modulate_fp8(
        res, x.view(1, M, N), gate, shift, scale)
    y = dit_ops.fused_layernorm_modulate(res_out, shift, scale)  # the unfused pair's y
    torch.cuda.synchronize()
    xr = x[ROWS].cpu()
    new_res = ops.residual_add(xr, res0, gate.cpu().reshape(1, N))
    assert torch.equal(res_out.view(M, N)[ROWS].cpu().view(torch.int16),
                       new_res.view(torch.int16)), "residual differs"
    y_rows = y.reshape(M, N)[ROWS].cpu()
    q_ref, s_ref = ops.per_token_quant_fp8(y_rows)
    assert torch.equal(fp8_rows(q), q_ref), "fp8 bytes differ from quant(unfused y)"
    assert torch.equal(s[ROWS].cpu().reshape(-1), s_ref), "scales differ"
    ref = ops.norm_scale_shift_f32(new_res, None, None, scale.cpu().reshape(1, N),
                                   shift.cpu().reshape(1, N), 0, 1e-6)
    assert_within_ulp(y_rows, ref, torch.bfloat16, ref.abs().amax(dim=-1, keepdim=True),
                      what="N3 y past 2^31")
    del res, res_out, q, s, y


def test_fp8_scaled_mm_output_past_2_31_elements(dev):
    """An FP8 GEMM whose [131584, 16384] bf16 output (4.3 GB) crosses element
    2^31 (multi-round 224x256 tiles): rows on either side of it against the
    exact oracle, to the GEMM tests' bar."""
    import joyomni_ops as jo
    Mg, Ng, Kg = (1 << 31) // 16384 + 512, 16384, 256
    edge = (1 << 31) // Ng
    rows = [0, edge - 1, edge, Mg - 1]
    g = torch.Generator(device=dev).manual_seed(5)
    a = (torch.randn(Mg, Kg, generator=g, device=dev) * 2).to(torch.float8_e4m3fn)
    w = (torch.randn(Ng, Kg, generator=g, device=dev) * 2).to(torch.float8_e4m3fn)
    sa = torch.rand(Mg, 1, generator=g, device=dev) * 0.02 + 1e-3
    sb = torch.rand(1, Ng, generator=g, device=dev) * 0.02 + 1e-3
    bias = torch.randn(Ng, generator=g, device=dev).to(torch.bfloat16)
    out = jo.fp8_scaled_mm(a, w.t(), sa, sb, torch.bfloat16, bias)
    torch.cuda.synchronize()
    assert out.numel() > (1 << 31)
    ar = a.view(torch.uint8)[rows].cpu().view(torch.float8_e4m3fn)
    _, acc, mag = ops.fp8_scaled_mm(ar, w.cpu().t(), sa[rows].cpu(), sb.cpu(), torch.bfloat16,
                                    bias.cpu())
    ref = acc * sa[rows].cpu().double().reshape(-1, 1) * sb.cpu().double().reshape(1, -1) \
        + bias.cpu().double().reshape(1, -1)
    # one bf16 ulp of the exact value (2^(floor(log2|ref|) - 7)) plus the fp32
    # summation slack of the matrix cores, as in the GEMM's own tests
    ulp = 2.0 ** (torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -14))) - 7)
    err = (out[rows].cpu().double() - ref).abs()
    bad = err > ulp + mag * 2.0 ** -13
    assert not bool(bad.any()), f"{int(bad.sum())} outputs off"
    del a, w, out
    torch.cuda.empty_cache()
