"""Zero-row and zero-token inputs through the torch ops: each returns (or
fills) an empty result of the right shape and dtype and launches nothing
(the C ABI returns before any launch when there are no rows; the CPU tests
check that entry point by entry point)."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

BF = torch.bfloat16
FP8 = torch.float8_e4m3fn


def _rows(dev, N=256):
    return torch.empty(0, N, dtype=BF, device=dev)


def case_norm_scale_shift(jo, dev):
    x = _rows(dev)
    y = jo.fused_norm_scale_shift(x, None, None, x, x, "layer", 1e-6)
    return [(y, (0, 256), BF)]


def case_rmsnorm(jo, dev):
    y = jo.rmsnorm(_rows(dev), torch.ones(256, dtype=BF, device=dev), 1e-6)
    return [(y, (0, 256), BF)]


def case_per_token_quant(jo, dev):
    q = torch.empty(0, 256, dtype=FP8, device=dev)
    s = torch.empty(0, 1, dtype=torch.float32, device=dev)
    jo.sgl_per_token_quant_fp8(_rows(dev), q, s)
    return [(q, (0, 256), FP8), (s, (0, 1), torch.float32)]


def case_gelu_quant(jo, dev):
    q = torch.empty(0, 256, dtype=FP8, device=dev)
    s = torch.empty(0, 1, dtype=torch.float32, device=dev)
    a = torch.empty(0, 256, dtype=BF, device=dev)
    jo.gelu_tanh_quant_fp8(_rows(dev), q, s, a)
    return [(q, (0, 256), FP8), (s, (0, 1), torch.float32), (a, (0, 256), BF)]


def case_fp8_scaled_mm(jo, dev):
    a = torch.empty(0, 64, dtype=FP8, device=dev)
    b = torch.zeros(32, 64, dtype=FP8, device=dev).t()
    y = jo.fp8_scaled_mm(a, b, torch.empty(0, device=dev), torch.ones(32, device=dev), BF, None)
    return [(y, (0, 32), BF)]


def case_add_layernorm(jo, dev):
    x, r = _rows(dev), _rows(dev)
    sc = torch.zeros(256, dtype=BF, device=dev)
    y = jo.fused_add_layernorm_scale_shift(x, r, sc, sc, eps=1e-6)
    return [(y, (0, 256), BF)]


def case_rmsnorm_quant(jo, dev):
    q = torch.empty(0, 256, dtype=FP8, device=dev)
    s = torch.empty(0, dtype=torch.float32, device=dev)
    jo.rmsnorm_quant_fp8(_rows(dev), torch.ones(256, dtype=BF, device=dev), 1e-6, q, s)
    return [(q, (0, 256), FP8), (s, (0,), torch.float32)]


def case_norm_quant(jo, dev):
    q = torch.empty(0, 256, dtype=FP8, device=dev)
    s = torch.empty(0, dtype=torch.float32, device=dev)
    sc = torch.zeros(256, dtype=BF, device=dev).expand(0, 256)
    jo.norm_scale_shift_quant_fp8(_rows(dev), sc, sc, q, s)
    return [(q, (0, 256), FP8), (s, (0,), torch.float32)]


def case_rmsnorm_heads(jo, dev):
    x = torch.empty(1, 0, 4, 128, dtype=BF, device=dev)
    y = jo.rmsnorm_heads(x, torch.ones(128, dtype=BF, device=dev), 1e-6, True)
    return [(y, (1, 0, 4, 128), BF)]


def case_apply_rotary_emb(jo, dev):
    x = torch.empty(1, 0, 4, 128, dtype=BF, device=dev)
    t = torch.empty(0, 128, dtype=torch.float32, device=dev)
    y = jo.apply_rotary_emb(x, (t, t))
    return [(y, (1, 0, 4, 128), BF)]


def _qk(dev, H=4, D=128):
    q = torch.empty(1, 0, D, dtype=BF, device=dev)
    k = torch.empty(1, 0, D, dtype=BF, device=dev)
    return q, k, torch.ones(D, dtype=BF, device=dev)


def case_qk_paired(jo, dev):
    q, k, w = _qk(dev)
    t = torch.empty(0, 64, dtype=BF, device=dev)
    jo.fused_qk_norm_rope_3d_paired(q, k, 0, 4, 1e-6, w, w, t, t)
    return [(q, (1, 0, 128), BF), (k, (1, 0, 128), BF)]


def case_qk_grid(jo, dev):
    q, k, w = _qk(dev)
    freqs = jo.rope_freqs(128, (44, 42, 42), 10000.0)
    jo.fused_qk_norm_rope_3d_grid(q, k, 0, 4, 1e-6, w, w, freqs, (44, 42, 42), (3, 5), 0)
    return [(q, (1, 0, 128), BF), (k, (1, 0, 128), BF)]


def case_qk_kvcache(jo, dev):
    q, k, w = _qk(dev)
    cache = torch.zeros(1, 2 * 15 * 4, 128, dtype=BF, device=dev)  # 2 slots of 3x5-token frames
    freqs = jo.rope_freqs(128, (44, 42, 42), 10000.0)
    jo.fused_qk_norm_rope_3d_kvcache(q, k, cache, 0, 4, 1e-6, w, w, freqs, (44, 42, 42), (3, 5),
                                     0, 0)
    assert torch.count_nonzero(cache).item() == 0  # nothing written
    return [(q, (1, 0, 128), BF), (cache, (1, 120, 128), BF)]


def case_kv_commit(jo, dev):
    src = torch.empty(2, 1, 0, 4, 128, dtype=BF, device=dev)
    dst = torch.zeros(2, 1, 8, 4, 128, dtype=BF, device=dev)
    t = torch.empty(0, 128, dtype=torch.float32, device=dev)
    jo.kv_commit_rope(src, dst, 8, t, t, src_v=src, dst_v=dst.clone())
    assert torch.count_nonzero(dst).item() == 0
    return [(dst, (2, 1, 8, 4, 128), BF)]


CASES = [case_norm_scale_shift, case_rmsnorm, case_per_token_quant, case_gelu_quant,
         case_fp8_scaled_mm,
         case_add_layernorm, case_rmsnorm_quant, case_norm_quant, case_rmsnorm_heads,
         case_apply_rotary_emb, case_qk_paired, case_qk_grid, case_qk_kvcache, case_kv_commit]


@pytest.mark.parametrize("case", CASES, ids=[c.__name__[5:] for c in CASES])
def test_empty_input(dev, case):
    import joyomni_ops as jo
    outs = case(jo, dev)
    torch.cuda.synchronize()
    for t, shape, dtype in outs:
        assert tuple(t.shape) == shape and t.dtype == dtype, (tuple(t.shape), t.dtype)


@pytest.mark.parametrize("shape", [-1, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11])
@pytest.mark.parametrize("with_bias", [True, False])
def test_fp8_scaled_mm_zero_k(dev, shape, with_bias):
    """K == 0: the output is the epilogue of a zero accumulator, the bias (or
    zeros), under every GEMM launch shape — through the torch op on
    zero-width views (which torch hands over as null pointers) and through
    the C ABI with non-null operand pointers into larger buffers of random
    bytes, none of which may be read."""
    import joyomni_ops as jo
    from joyomni_ops import _abi
    M, N = 300, 512
    g = torch.Generator().manual_seed(5)
    big_a = torch.randint(0, 120, (M, 128), generator=g, dtype=torch.uint8).to(dev).view(FP8)
    big_w = torch.randint(0, 120, (N, 128), generator=g, dtype=torch.uint8).to(dev).view(FP8)
    a = big_a[:, :0]
    b = big_w[:, :0].t()
    assert a.stride(0) == 128 and b.stride(1) == 128
    sa = torch.rand(M, generator=g).to(dev) + 0.5
    sb = torch.rand(N, generator=g).to(dev) + 0.5
    bias = (torch.randn(N, generator=g) * 4).to(BF).to(dev) if with_bias else None
    _abi.call("jo_set_launch_override", _abi.JO_KNOB_GEMM_SHAPE, shape)
    try:
        y = jo.fp8_scaled_mm(a, b, sa, sb, BF, bias)
        # the same call through the C ABI, into a buffer filled with NaN
        out = torch.full((M, N), float("nan"), dtype=BF, device=dev)
        _abi.call("jo_fp8_scaled_mm", big_a.data_ptr(), 128, big_w.data_ptr(), 128, sa.data_ptr(),
                  sb.data_ptr(), None if bias is None else bias.data_ptr(), out.data_ptr(), N,
                  M, N, 0, _abi.JO_DTYPE_BF16, torch.cuda.current_stream(dev).cuda_stream)
    finally:
        _abi.call("jo_set_launch_override", _abi.JO_KNOB_GEMM_SHAPE, -1)
    torch.cuda.synchronize()
    want = (bias.float() if bias is not None else torch.zeros(N, device=dev)).expand(M, N)
    assert y.shape == (M, N) and y.dtype == BF
    assert torch.equal(y.float(), want), "K == 0 output is not the bias"
    assert torch.equal(out.float(), want), "K == 0 output (C ABI) is not the bias"
