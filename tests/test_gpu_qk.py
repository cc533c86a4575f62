"""GPU parity of the QK RMSNorm + RoPE ops through the C ABI and torch ops.

Bar (the benchmark contract): bf16 outputs within 1 bf16 ulp of the fp32-accumulated
oracle (fused_qknorm_rope_3d_kernel.cu:98-142 / test_parity_light.py:77-87
restated in oracle/ops.py), the ulp floored at 2^-10 of the head's largest
|value| to absorb fp32 cancellation in rotated pairs.
"""
from __future__ import annotations

import pytest
import torch

from helpers import assert_bf16_within_ulp
from oracle import ops
from joyomni_ops import workloads as W

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["auto", "1", "2", "4", "6", "8"], autouse=True)
def qk_split(request):
    """Run every QK test with the automatic launch shape and with one, two, four,
    six and eight waves per token forced (the JO_KNOB_QK_SPLIT launch override):
    results must not depend on it."""
    from joyomni_ops import _abi
    value = -1 if request.param == "auto" else int(request.param)
    _abi.call("jo_set_launch_override", _abi.JO_KNOB_QK_SPLIT, value)
    yield request.param
    _abi.call("jo_set_launch_override", _abi.JO_KNOB_QK_SPLIT, -1)


def head_floor(ref):
    return ref.abs().amax(dim=-1, keepdim=True)


def rand_qk(B, L, H, D, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, L * H, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, L * H, D, generator=g).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    return q, k, qw, kw


# Where at least this many elements are checked, at most FLOOR_CAP of them may
# pass only through the 2^-10 head-max floor (the rest within 1 ulp of their
# own value).
FLOOR_CAP = 1e-4
FLOOR_CAP_MIN_ELEMENTS = 1 << 20


def check_qk(out, x, w, cos, sin, B, L, H, D, what, eps=1e-6):
    ref = ops.qk_norm_rope_f32(x.reshape(B, L, H, D), w, cos, sin, eps)
    cap = FLOOR_CAP if ref.numel() >= FLOOR_CAP_MIN_ELEMENTS else None
    return assert_bf16_within_ulp(out.reshape(B, L, H, D), ref, head_floor(ref), what=what,
                                  floor_cap=cap)


# ---------------------------------------------------------------------------
# Table mode (drop-in)
# ---------------------------------------------------------------------------
TABLE_SHAPES = [(1, 128, 8, 128), (2, 7, 3, 64), (1, 5, 2, 256), (1, 33, 30, 128),
                (1, 17, 48, 128), (3, 9, 1, 64), (1, 1560, 32, 128)]


@pytest.mark.parametrize("B,L,H,D", TABLE_SHAPES)
@pytest.mark.parametrize("tables", ["randn", "rope"])
def test_table_mode(abi, dev, stream_handle, B, L, H, D, tables):
    q, k, qw, kw = rand_qk(B, L, H, D, B * 1000 + L * 10 + H + D)
    if tables == "randn":  # what the reference's own tests feed (test_parity_light.py:64-65)
        g = torch.Generator().manual_seed(5)
        cos = torch.randn(L, D // 2, generator=g).to(torch.bfloat16)
        sin = torch.randn(L, D // 2, generator=g).to(torch.bfloat16)
    else:  # the DiT's tables, halved and cast as sgl_fused_ops.py:87-94 does
        dims = {64: (16, 24, 24), 128: (16, 56, 56), 256: (64, 96, 96)}[D]
        c, s = ops.half_tables(*ops.rope_grid_tables(1, 1, L, 3, dims, 256.0))
        cos, sin = c.to(torch.bfloat16), s.to(torch.bfloat16)
    # Device copies are kept in named variables: a temporary's memory would be
    # returned to the caching allocator before the asynchronous kernel runs.
    qd, kd, qwd, kwd, cd, sd = (t.to(dev) for t in (q, k, qw, kw, cos, sin))
    tok = H * D
    abi.call("jo_fused_qk_norm_rope_3d_paired", qd.data_ptr(), kd.data_ptr(), B, L, H, D, L * tok,
             tok, L * tok, tok, 1e-6, qwd.data_ptr(), kwd.data_ptr(), cd.data_ptr(), sd.data_ptr(),
             stream_handle)
    torch.cuda.synchronize()
    check_qk(qd.cpu(), q, qw, cos, sin, B, L, H, D, "q")
    check_qk(kd.cpu(), k, kw, cos, sin, B, L, H, D, "k")


def test_table_mode_strided_qkv_views(abi, dev, stream_handle):
    """q and k as strided views of a packed qkv [B, L, 3, H, D] (token stride 3*H*D)."""
    B, L, H, D = 2, 40, 6, 128
    g = torch.Generator().manual_seed(21)
    qkv = torch.randn(B, L, 3, H, D, generator=g).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    ang = torch.randn(L, D // 2, generator=g)
    cos, sin = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    d, qwd, kwd, cd, sd = (t.to(dev) for t in (qkv, qw, kw, cos, sin))
    abi.call("jo_fused_qk_norm_rope_3d_paired", d[:, :, 0].data_ptr(), d[:, :, 1].data_ptr(), B, L,
             H, D, L * 3 * H * D, 3 * H * D, L * 3 * H * D, 3 * H * D, 1e-6, qwd.data_ptr(),
             kwd.data_ptr(), cd.data_ptr(), sd.data_ptr(), stream_handle)
    torch.cuda.synchronize()
    out = d.cpu()
    check_qk(out[:, :, 0].contiguous(), qkv[:, :, 0].contiguous(), qw, cos, sin, B, L, H, D, "q view")
    check_qk(out[:, :, 1].contiguous(), qkv[:, :, 1].contiguous(), kw, cos, sin, B, L, H, D, "k view")
    assert torch.equal(out[:, :, 2], qkv[:, :, 2]), "v must be untouched"


def test_table_mode_torch_op(dev):
    import joyomni_ops as jo
    B, L, H, D = 1, 128, 8, 128
    q, k, qw, kw = rand_qk(B, L, H, D, 3)
    ang = torch.randn(L, D // 2)
    cos, sin = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    qd, kd = q.to(dev), k.to(dev)
    jo.fused_qk_norm_rope_3d_paired(qd, kd, L, H, 1e-6, qw.to(dev), kw.to(dev), cos.to(dev), sin.to(dev))
    torch.cuda.synchronize()
    check_qk(qd.cpu(), q, qw, cos, sin, B, L, H, D, "q op")
    check_qk(kd.cpu(), k, kw, cos, sin, B, L, H, D, "k op")
    with pytest.raises(RuntimeError, match="head_dim"):
        bad = torch.zeros(1, L * H, 96, dtype=torch.bfloat16, device=dev)
        jo.fused_qk_norm_rope_3d_paired(bad, bad.clone(), L, H, 1e-6, torch.ones(96, dtype=torch.bfloat16, device=dev),
                                        torch.ones(96, dtype=torch.bfloat16, device=dev),
                                        torch.ones(L, 48, dtype=torch.bfloat16, device=dev),
                                        torch.ones(L, 48, dtype=torch.bfloat16, device=dev))


# ---------------------------------------------------------------------------
# Grid mode (in-register angles)
# ---------------------------------------------------------------------------
GRID_CASES = [
    # B, frames, gh, gw, H, D, t0, dims, theta, source_id
    (1, 1, 5, 7, 4, 128, 0, (44, 42, 42), 10000.0, 0.0),
    (2, 2, 3, 4, 3, 128, 21, (16, 56, 56), 256.0, 0.0),
    (1, 1, 30, 52, 2, 128, 7, (16, 56, 56), 256.0, 1.0),
    (1, 3, 4, 4, 5, 64, 100, (16, 24, 24), 10000.0, 2.0),
    (1, 2, 3, 5, 2, 256, 3, (64, 96, 96), 10000.0, 0.0),
    (1, 1, 45, 78, 24, 128, 0, (44, 42, 42), 10000.0, 0.0),   # C0
    # Large angles: many multiples of pi/2 to reduce, and (t0 and source id
    # above 65536) the library-sincos branch, mixed with small angles in a wave.
    (1, 2, 3, 4, 2, 128, 4000, (44, 42, 42), 10000.0, 3.0),
    (1, 1, 4, 6, 2, 128, 70000, (44, 42, 42), 10000.0, 70001.0),
]


def grid_call(abi, stream, qd, kd, B, L, H, D, qw, kw, freqs, dims, gh, gw, t0, sid):
    tok = H * D
    abi.call("jo_fused_qk_norm_rope_3d_grid", qd.data_ptr(), kd.data_ptr(), B, L, H, D, L * tok,
             tok, L * tok, tok, 1e-6, qw.data_ptr(), kw.data_ptr(), freqs.data_ptr(), dims[0] // 2,
             dims[1] // 2, gh, gw, t0, sid, stream)


@pytest.mark.parametrize("case", GRID_CASES)
def test_grid_mode(abi, dev, stream_handle, case):
    import joyomni_ops as jo
    B, F, gh, gw, H, D, t0, dims, theta, sid = case
    L = F * gh * gw
    q, k, qw, kw = rand_qk(B, L, H, D, L + H + D)
    freqs = jo.rope_freqs(D, dims, theta, 256.0)
    qd, kd = q.to(dev), k.to(dev)
    grid_call(abi, stream_handle, qd, kd, B, L, H, D, qw.to(dev), kw.to(dev), freqs, dims, gh, gw, t0, sid)
    torch.cuda.synchronize()
    cos, sin = ops.half_tables(*ops.rope_grid_tables(F, gh, gw, t0, dims, theta, sid, 256.0))
    check_qk(qd.cpu(), q, qw, cos, sin, B, L, H, D, f"grid q {case}")
    check_qk(kd.cpu(), k, kw, cos, sin, B, L, H, D, f"grid k {case}")


def test_grid_mode_torch_op_c0(dev):
    import joyomni_ops as jo
    cfg = W.CONFIGS["C0"]
    d = cfg.dims
    t = W.make_inputs(cfg)
    qd, kd = t["q"].to(dev), t["k"].to(dev)
    freqs = jo.rope_freqs(d["D"], d["rope_dims"], d["theta"])
    jo.fused_qk_norm_rope_3d_grid(qd, kd, d["L"], d["H"], d["eps"], t["q_weight"].to(dev),
                                  t["k_weight"].to(dev), freqs, d["rope_dims"], d["grid"], d["t0"])
    torch.cuda.synchronize()
    cos, sin = ops.half_tables(*ops.rope_grid_tables(1, *d["grid"], d["t0"], d["rope_dims"], d["theta"]))
    check_qk(qd.cpu(), t["q"], t["q_weight"], cos, sin, 1, d["L"], d["H"], d["D"], "C0 q")
    check_qk(kd.cpu(), t["k"], t["k_weight"], cos, sin, 1, d["L"], d["H"], d["D"], "C0 k")


# ---------------------------------------------------------------------------
# Grid mode + K ring cache (C3)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("small", [True, False])
def test_kvcache_mode(abi, dev, stream_handle, small):
    import joyomni_ops as jo
    if small:
        B, F, gh, gw, H, D, t0, slots = 2, 3, 4, 5, 3, 128, 18, 7   # slot_start 6: wraps
        dims, theta = (44, 42, 42), 10000.0
        q, k, qw, kw = rand_qk(B, F * gh * gw, H, D, 77)
    else:
        cfg = W.CONFIGS["C3"]
        d = cfg.dims
        B, F, (gh, gw), H, D, t0, slots = d["B"], d["frames"], d["grid"], d["H"], d["D"], d["t0"], d["cache_slots"]
        dims, theta = d["rope_dims"], d["theta"]
        t = W.make_inputs(cfg)
        q, k, qw, kw = t["q"], t["k"], t["q_weight"], t["k_weight"]
    L = F * gh * gw
    ft = gh * gw
    slot0 = jo.kv_ring_slot(t0, F, slots)
    cache = torch.full((B, slots * ft * H, D), 7.0, dtype=torch.bfloat16, device=dev)
    qd, kd = q.to(dev), k.to(dev)
    freqs = jo.rope_freqs(D, dims, theta)
    jo.fused_qk_norm_rope_3d_kvcache(qd, kd, cache, L, H, 1e-6, qw.to(dev), kw.to(dev), freqs,
                                     dims, (gh, gw), t0, slot0)
    torch.cuda.synchronize()
    cos, sin = ops.half_tables(*ops.rope_grid_tables(F, gh, gw, t0, dims, theta))
    check_qk(qd.cpu(), q, qw, cos, sin, B, L, H, D, "kvcache q")
    assert torch.equal(kd.cpu(), k), "k must not be modified"
    ref_k = ops.qk_norm_rope_f32(k.reshape(B, L, H, D), kw, cos, sin, 1e-6)
    c = cache.cpu().reshape(B, slots, ft, H, D)
    written = set()
    for f, slot in enumerate(ops.ring_slots(F, slots, slot0)):
        written.add(slot)
        r = ref_k[:, f * ft:(f + 1) * ft]
        cap = FLOOR_CAP if r.numel() >= FLOOR_CAP_MIN_ELEMENTS else None
        assert_bf16_within_ulp(c[:, slot], r, head_floor(r), what=f"cache slot {slot}",
                               floor_cap=cap)
    for slot in set(range(slots)) - written:
        assert bool((c[:, slot] == 7.0).all()), f"slot {slot} must be untouched"
