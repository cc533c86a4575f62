"""GPU parity of the per-head RMSNorm (jo_rmsnorm_heads, torch op rmsnorm_heads,
dit_ops.rmsnorm_qk_bf16 and dit_ops.rms_norm_module).

Bars:
  round_first (the torch RMSNorm module, dit.py:244-249): bit-exact against the
      oracle — its mean square is the exactly rounded one on both sides, so the
      intermediate rounding to the row dtype and the weight product agree;
  kernel rounding (rmsnorm_qk_bf16 on the K slice of a packed qkv): bit-identical
      to the rmsnorm op on a contiguous copy of the same rows (same kernel, same
      summation order) and within 1 ulp of the fp32 oracle.
"""
from __future__ import annotations

import pytest
import torch

from helpers import assert_within_ulp
from oracle import ops

pytestmark = pytest.mark.gpu


def packed_qkv(B, L, H, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    qkv = (torch.randn(B, L, 3, H, D, generator=g) * 2).to(dtype)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(dtype)
    return qkv, w


def equal_or_both_nan(a: torch.Tensor, b: torch.Tensor) -> bool:
    a, b = a.float(), b.float()
    return bool(((a == b) | (torch.isnan(a) & torch.isnan(b))).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("B,L,H,D", [(1, 77, 32, 128), (2, 5, 3, 64), (1, 9, 2, 256),
                                     (1, 16, 4, 100), (3, 1, 1, 128)])
def test_module_on_packed_qkv_slices_is_exact(dev, dtype, B, L, H, D):
    import joyomni_ops as jo
    qkv, w = packed_qkv(B, L, H, D, dtype, B * 100 + L + H + D)
    dq = qkv.to(dev)
    for part in (0, 1):  # q and k slices of the packed tensor
        out = jo.rmsnorm_heads(dq[:, :, part], w.to(dev), 1e-6, round_first=True)
        torch.cuda.synchronize()
        assert out.is_contiguous() and out.shape == (B, L, H, D)
        ref = ops.rms_norm_module(qkv[:, :, part].contiguous(), w, 1e-6)
        assert torch.equal(out.cpu(), ref), f"part {part}: module rmsnorm differs"


def test_module_special_rows_and_no_weight(dev):
    from joyomni_ops import dit_ops
    x = torch.randn(6, 4, 128, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    x[1] = 0.0
    x[2, 1, 9] = float("nan")
    x[3, 2, 0] = float("inf")
    x[4] = 1e-30   # tiny rows: the mean square underflows, r = 1/sqrt(eps)
    out = dit_ops.rms_norm_module(x.to(dev), None, 1e-6)
    torch.cuda.synchronize()
    assert equal_or_both_nan(out.cpu(), ops.rms_norm_module(x, None, 1e-6))
    w = (1 + 0.1 * torch.randn(128)).to(torch.bfloat16)
    out = dit_ops.rms_norm_module(x.to(dev), w.to(dev), 1e-6)
    torch.cuda.synchronize()
    assert equal_or_both_nan(out.cpu(), ops.rms_norm_module(x, w, 1e-6))


@pytest.mark.parametrize("B,L,H,D", [(1, 3120, 32, 128), (2, 33, 24, 128), (1, 7, 5, 64)])
def test_rmsnorm_qk_bf16_reads_the_packed_k_slice(dev, B, L, H, D):
    """dit_ops.rmsnorm_qk_bf16 on the strided K view == rmsnorm on its copy, bit for bit."""
    import joyomni_ops as jo
    from joyomni_ops import dit_ops
    qkv, w = packed_qkv(B, L, H, D, torch.bfloat16, 7 + L)
    dq, dw = qkv.to(dev), w.to(dev)
    k = dq[:, :, 1]
    assert not k.is_contiguous()
    out = dit_ops.rmsnorm_qk_bf16(k, dw, eps=1e-6)
    copy = jo.rmsnorm(k.contiguous().reshape(-1, D), dw, 1e-6).reshape(B, L, H, D)
    torch.cuda.synchronize()
    assert out.is_contiguous() and out.shape == (B, L, H, D)
    assert torch.equal(out, copy)
    ref = ops.rmsnorm_f32(qkv[:, :, 1].reshape(-1, D), w, 1e-6)
    assert_within_ulp(out.cpu().reshape(-1, D), ref, torch.bfloat16, what="rmsnorm_qk_bf16")


def test_generic_path_unaligned_head_stride(dev):
    """A head stride that breaks 16-byte row alignment takes the element-wise
    kernel; both roundings still match."""
    import joyomni_ops as jo
    g = torch.Generator().manual_seed(11)
    base = torch.randn(10, 4 * 130 + 3, generator=g).to(torch.bfloat16)
    x = base[:, 3:].unfold(1, 128, 130)  # [10, 4, 128], head stride 130, offset 3
    assert x.stride() == (base.stride(0), 130, 1)
    w = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16)
    dx = base.to(dev)[:, 3:].unfold(1, 128, 130)
    out = jo.rmsnorm_heads(dx, w.to(dev), 1e-6, round_first=True)
    out0 = jo.rmsnorm_heads(dx, w.to(dev), 1e-6, round_first=False)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), ops.rms_norm_module(x.contiguous(), w, 1e-6))
    assert_within_ulp(out0.cpu().reshape(-1, 128), ops.rmsnorm_f32(x.reshape(-1, 128), w, 1e-6),
                      torch.bfloat16, what="generic kernel rounding")


def test_rejects_bad_views(dev):
    import joyomni_ops as jo
    x = torch.zeros(4, 5, 3, 64, dtype=torch.bfloat16, device=dev)
    w = torch.ones(64, dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError, match="one token stride"):
        jo.rmsnorm_heads(x.transpose(0, 1), w, 1e-6)
    with pytest.raises(RuntimeError, match="weight must be 1D"):
        jo.rmsnorm_heads(x, torch.ones(32, dtype=torch.bfloat16, device=dev), 1e-6)
    with pytest.raises(RuntimeError, match="dtype must match"):
        jo.rmsnorm_heads(x, torch.ones(64, device=dev), 1e-6)
