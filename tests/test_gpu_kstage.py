"""GPU parity of the QK ops with the pre-RoPE K stage output (*_kstage).

One pass writes the rotated q and k in place and the pre-RoPE normalized k to
a stage buffer (the DiT's K-cache-before-RoPE branch, dit.py:360-370). Bars:
the stage rows bit-identical to the per-head RMSNorm op on the same k
(rmsnorm_qk_bf16's kernel semantics) and within 1 bf16 ulp of the fp32
oracle (oracle.rmsnorm_f32); q and k bit-identical to the same op without the
stage (itself within 1 bf16 ulp of oracle.qk_norm_rope_f32, checked here
again at the deployment shape); v and everything outside the stage rows
untouched. Every launch shape (the JO_KNOB_QK_SPLIT override) is covered.
"""
from __future__ import annotations

import pytest
import torch

from helpers import assert_bf16_within_ulp
from oracle import ops

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


@pytest.fixture(params=["auto", "1", "2", "4", "6", "8"], autouse=True)
def qk_split(request):
    """The automatic launch shape and one, two, four, six and eight waves per
    token forced: results must not depend on it."""
    from joyomni_ops import _abi
    value = -1 if request.param == "auto" else int(request.param)
    _abi.call("jo_set_launch_override", _abi.JO_KNOB_QK_SPLIT, value)
    yield request.param
    _abi.call("jo_set_launch_override", _abi.JO_KNOB_QK_SPLIT, -1)


def packed_qkv(B, L, H, D, seed):
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn(B, L, 3, H, D, generator=g).to(BF)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(BF)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(BF)
    return qkv, qw, kw


def head_floor(ref):
    return ref.abs().amax(dim=-1, keepdim=True)


def check_stage(stage, k, kw, what, eps=1e-6):
    """stage: the op's pre-RoPE rows [B, L, H, D]; k: the input k [B, L, H, D] (CPU)."""
    import joyomni_ops as jo
    dev = stage.device
    ref_op = jo.rmsnorm_heads(k.to(dev), kw.to(dev), eps, round_first=False)
    torch.cuda.synchronize()
    assert torch.equal(stage.cpu().view(torch.int16), ref_op.cpu().view(torch.int16)), \
        f"{what}: stage differs from the per-head RMSNorm op"
    ref = ops.rmsnorm_f32(k, kw, eps)
    assert_bf16_within_ulp(stage.cpu(), ref, what=f"{what} vs oracle")


@pytest.mark.parametrize("B,L,H,D", [(1, 3120, 32, 128), (2, 37, 6, 128), (1, 9, 3, 64),
                                     (1, 11, 2, 256), (1, 1, 24, 128)])
def test_paired_kstage(dev, B, L, H, D):
    """Table mode on the q / k slices of a packed qkv, stage into a fresh tensor;
    [1, 3120, 32, 128] is the DiT's image stream at 720x1248."""
    import joyomni_ops as jo
    qkv, qw, kw = packed_qkv(B, L, H, D, 1000 + L + H + D)
    ang = torch.rand(L, D // 2, generator=torch.Generator().manual_seed(7)) * 100
    cos, sin = ang.cos().to(BF), ang.sin().to(BF)
    d = qkv.to(dev)
    ref = qkv.to(dev)
    stage = torch.full((B, L, H, D), 7.0, dtype=BF, device=dev)
    qwd, kwd, cd, sd = (t.to(dev) for t in (qw, kw, cos, sin))
    jo.fused_qk_norm_rope_3d_paired_kstage(d[:, :, 0], d[:, :, 1], stage, L, H, 1e-6, qwd, kwd,
                                           cd, sd)
    qr, kr = ref[:, :, 0].contiguous(), ref[:, :, 1].contiguous()
    jo.fused_qk_norm_rope_3d_paired(qr.view(B, L * H, D), kr.view(B, L * H, D), L, H, 1e-6, qwd,
                                    kwd, cd, sd)
    torch.cuda.synchronize()
    out = d.cpu()
    assert torch.equal(out[:, :, 0].view(torch.int16), qr.cpu().view(torch.int16)), "q"
    assert torch.equal(out[:, :, 1].view(torch.int16), kr.cpu().view(torch.int16)), "k"
    assert torch.equal(out[:, :, 2], qkv[:, :, 2]), "v must be untouched"
    check_stage(stage, qkv[:, :, 1].contiguous(), kw, "stage")
    if (B, L, H, D) == (1, 3120, 32, 128):
        for t, w, name in ((0, qw, "q"), (1, kw, "k")):
            x = qkv[:, :, t].contiguous()
            r = ops.qk_norm_rope_f32(x, w, cos, sin, 1e-6)
            assert_bf16_within_ulp(out[:, :, t], r, head_floor(r), what=f"{name} vs oracle")


def test_paired_kstage_into_stage_buffer(dev):
    """The stage rows land in one layer of a [layers, B, T, H, D] buffer (the
    graph runner's pre-RoPE K stage, graph_runner.py:56-59); the other layers
    are not written."""
    import joyomni_ops as jo
    Ly, B, L, H, D = 3, 1, 50, 8, 128
    qkv, qw, kw = packed_qkv(B, L, H, D, 77)
    ang = torch.rand(L, D // 2, generator=torch.Generator().manual_seed(8)) * 10
    cos, sin = ang.cos().to(BF), ang.sin().to(BF)
    d = qkv.to(dev)
    buf = torch.zeros(Ly, B, L, H, D, dtype=BF, device=dev)
    jo.fused_qk_norm_rope_3d_paired_kstage(d[:, :, 0], d[:, :, 1], buf[1], L, H, 1e-6,
                                           qw.to(dev), kw.to(dev), cos.to(dev), sin.to(dev))
    torch.cuda.synchronize()
    check_stage(buf[1], qkv[:, :, 1].contiguous(), kw, "stage layer")
    assert torch.count_nonzero(buf[0]).item() == 0 and torch.count_nonzero(buf[2]).item() == 0


GRID_CASES = [
    # B, frames, gh, gw, H, D, t0, dims, theta, source_id
    (1, 1, 45, 78, 24, 128, 0, (44, 42, 42), 10000.0, 0.0),   # C0 geometry
    (2, 2, 3, 4, 3, 128, 21, (16, 56, 56), 256.0, 1.0),
    (1, 3, 4, 4, 5, 64, 100, (16, 24, 24), 10000.0, 2.0),
]


@pytest.mark.parametrize("case", GRID_CASES)
def test_grid_kstage(dev, case):
    import joyomni_ops as jo
    B, F, gh, gw, H, D, t0, dims, theta, sid = case
    L = F * gh * gw
    qkv, qw, kw = packed_qkv(B, L, H, D, 300 + L)
    freqs = jo.rope_freqs(D, dims, theta, 256.0)
    d, ref = qkv.to(dev), qkv.to(dev)
    stage = torch.empty(B, L, H, D, dtype=BF, device=dev)
    qwd, kwd = qw.to(dev), kw.to(dev)
    jo.fused_qk_norm_rope_3d_grid_kstage(d[:, :, 0], d[:, :, 1], stage, L, H, 1e-6, qwd, kwd,
                                         freqs, dims, (gh, gw), t0, sid)
    jo.fused_qk_norm_rope_3d_grid(ref[:, :, 0], ref[:, :, 1], L, H, 1e-6, qwd, kwd, freqs, dims,
                                  (gh, gw), t0, sid)
    torch.cuda.synchronize()
    assert torch.equal(d.cpu().view(torch.int16), ref.cpu().view(torch.int16)), \
        "q / k / v differ from the op without the stage"
    check_stage(stage, qkv[:, :, 1].contiguous(), kw, "grid stage")


def test_dit_kstage_shim(dev):
    """dit_ops.fused_qk_norm_rope_3d_kstage against the two reference calls it
    replaces (rmsnorm_qk_bf16, then fused_qk_norm_rope_3d), with the DiT's
    fp32 [1, L, D] tables."""
    from joyomni_ops import dit_ops
    B, L, H, D = 1, 96, 4, 128
    qkv, qw, kw = packed_qkv(B, L, H, D, 5)
    cos_full, sin_full = ops.rope_grid_tables(1, 8, 12, 0, (16, 56, 56), 256.0)
    fc = (cos_full.unsqueeze(0).to(dev), sin_full.unsqueeze(0).to(dev))
    d = qkv.to(dev)
    k_for_cache_ref = dit_ops.rmsnorm_qk_bf16(d[:, :, 1], kw.to(dev), eps=1e-6)
    q_ref, k_ref = dit_ops.fused_qk_norm_rope_3d(d[:, :, 0], d[:, :, 1], qw.to(dev), kw.to(dev),
                                                 fc, eps=1e-6)
    q, k, k_for_cache = dit_ops.fused_qk_norm_rope_3d_kstage(d[:, :, 0], d[:, :, 1], qw.to(dev),
                                                             kw.to(dev), fc, eps=1e-6)
    torch.cuda.synchronize()
    for a, b, name in ((q, q_ref, "q"), (k, k_ref, "k"), (k_for_cache, k_for_cache_ref, "stage")):
        assert torch.equal(a.contiguous().cpu().view(torch.int16),
                           b.contiguous().cpu().view(torch.int16)), name


def test_kstage_rejects_bad_stage(dev):
    import joyomni_ops as jo
    B, L, H, D = 1, 4, 2, 128
    qkv, qw, kw = packed_qkv(B, L, H, D, 9)
    d = qkv.to(dev)
    t = torch.ones(L, D // 2, dtype=BF, device=dev)
    with pytest.raises(RuntimeError, match="k_stage"):
        jo.fused_qk_norm_rope_3d_paired_kstage(d[:, :, 0], d[:, :, 1],
                                               torch.empty(B, L, H, 64, dtype=BF, device=dev),
                                               L, H, 1e-6, qw.to(dev), kw.to(dev), t, t)
