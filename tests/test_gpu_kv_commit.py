"""GPU parity of the KV-pool commit (jo_kv_commit_rope, torch ops kv_commit_rope
and apply_rotary_emb, dit_ops.commit_kv_pool).

Bar: bit-exact. The rotation is apply_rotary_emb as torch evaluates it
(rope.py:21-28: two fp32 products and one fp32 sum per element, one rounding
to the element type), restated in oracle.ops.apply_rotary_emb and fed the same
fp32 tables; V is a copy; pool tokens outside the committed segment keep
their values.
"""
from __future__ import annotations

import pytest
import torch

from oracle import ops

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["auto", "1", "2"], autouse=True)
def kv_split(request):
    """Every commit test with the automatic launch shape and with K and V on
    the same wave (1) or on separate waves (2) forced (the JO_KNOB_KV_SPLIT launch override): results
    must not depend on it."""
    from joyomni_ops import _abi
    value = -1 if request.param == "auto" else int(request.param)
    _abi.call("jo_set_launch_override", _abi.JO_KNOB_KV_SPLIT, value)
    yield request.param
    _abi.call("jo_set_launch_override", _abi.JO_KNOB_KV_SPLIT, -1)


def tables(B, T, D, seed, per_batch=False):
    """fp32 cos/sin [T, D] (or [B, T, D]) from random angles up to 200 rad,
    repeat-interleaved like rope.py:50-51, with a few unequal pair columns so
    both columns of a pair are exercised."""
    g = torch.Generator().manual_seed(seed)
    shape = (B, T, D // 2) if per_batch else (T, D // 2)
    ang = torch.rand(shape, generator=g) * 200
    cos = ang.cos().repeat_interleave(2, -1).contiguous()
    sin = ang.sin().repeat_interleave(2, -1).contiguous()
    cos[..., 1] *= 0.5
    sin[..., -1] *= -1.25
    return cos, sin


def bits_equal(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


CASES = [
    # L, B, T, P, off, H, D, dtype
    (3, 2, 17, 51, 17, 3, 128, torch.bfloat16),   # 384-element rows (partial wave)
    (2, 1, 33, 70, 5, 24, 128, torch.bfloat16),   # 3072: 6 chunks
    (2, 1, 9, 20, 11, 32, 128, torch.bfloat16),   # 4096: 8 chunks (REAL heads)
    (1, 2, 10, 10, 0, 8, 64, torch.float16),
    (2, 1, 7, 9, 1, 4, 256, torch.bfloat16),
    (1, 1, 6, 8, 2, 5, 96, torch.bfloat16),       # 512 % 96 != 0: element-wise kernel
    (1, 1, 5, 5, 0, 40, 128, torch.bfloat16),     # 5120: beyond 8 chunks, element-wise
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("with_v", [True, False])
def test_commit_matches_reference_loop(abi, dev, stream_handle, case, with_v):
    L, B, T, P, off, H, D, dtype = case
    g = torch.Generator().manual_seed(T * 13 + H)
    pool_k = torch.randn(L, B, P, H, D, generator=g).to(dtype)
    pool_v = torch.randn(L, B, P, H, D, generator=g).to(dtype)
    sk = torch.randn(L, B, T, H, D, generator=g).to(dtype)
    sv = torch.randn(L, B, T, H, D, generator=g).to(dtype)
    cos, sin = tables(B, T, D, T)
    pkd, pvd, skd, svd = pool_k.to(dev), pool_v.to(dev), sk.to(dev), sv.to(dev)
    cd, sd = cos.to(dev), sin.to(dev)
    hd = H * D
    abi.call("jo_kv_commit_rope", skd.data_ptr(), svd.data_ptr() if with_v else None,
             pkd.data_ptr(), pvd.data_ptr() if with_v else None, L, B, T, H, D, B * T * hd,
             T * hd, hd, B * P * hd, P * hd, hd, P, off, cd.data_ptr(), sd.data_ptr(), D, 0,
             abi.dtype_code(dtype), stream_handle)
    torch.cuda.synchronize()
    rk, rv = ops.commit_kv(pool_k, pool_v if with_v else None, sk, sv if with_v else None, off,
                           cos, sin)
    assert bits_equal(pkd.cpu(), rk), f"K {case}"
    if with_v:
        assert bits_equal(pvd.cpu(), rv), f"V {case}"
    else:
        assert bits_equal(pvd.cpu(), pool_v), "V touched without a V source"


def test_commit_per_batch_tables_and_strided_source(abi, dev, stream_handle):
    """[B, T, D] tables, and K/V read from strided views of a packed
    [L, B, T, 3, H, D] buffer (token stride 3*H*D)."""
    L, B, T, P, off, H, D = 2, 3, 11, 30, 19, 6, 128
    g = torch.Generator().manual_seed(4)
    packed = torch.randn(L, B, T, 3, H, D, generator=g).to(torch.bfloat16)
    pool_k = torch.zeros(L, B, P, H, D, dtype=torch.bfloat16)
    pool_v = torch.zeros(L, B, P, H, D, dtype=torch.bfloat16)
    cos, sin = tables(B, T, D, 9, per_batch=True)
    pd, pkd, pvd = packed.to(dev), pool_k.to(dev), pool_v.to(dev)
    cd, sd = cos.to(dev), sin.to(dev)
    hd = H * D
    k_view, v_view = pd[:, :, :, 1], pd[:, :, :, 2]
    abi.call("jo_kv_commit_rope", k_view.data_ptr(), v_view.data_ptr(), pkd.data_ptr(),
             pvd.data_ptr(), L, B, T, H, D, k_view.stride(0), k_view.stride(1), k_view.stride(2),
             B * P * hd, P * hd, hd, P, off, cd.data_ptr(), sd.data_ptr(), D, T * D,
             abi.dtype_code(torch.bfloat16), stream_handle)
    torch.cuda.synchronize()
    rk = pool_k.clone()
    rv = pool_v.clone()
    for li in range(L):
        for b in range(B):
            rk[li, b:b + 1, off:off + T] = ops.apply_rotary_emb(
                packed[li, b:b + 1, :, 1], cos[b], sin[b])
            rv[li, b:b + 1, off:off + T] = packed[li, b:b + 1, :, 2]
    assert bits_equal(pkd.cpu(), rk) and bits_equal(pvd.cpu(), rv)


def test_torch_ops_apply_rotary_emb_and_commit(dev):
    import joyomni_ops as jo
    from joyomni_ops import dit_ops
    g = torch.Generator().manual_seed(21)
    # apply_rotary_emb on a strided q view of a packed qkv [B, T, 3, H, D]
    B, T, H, D = 2, 40, 4, 128
    qkv = torch.randn(B, T, 3, H, D, generator=g).to(torch.bfloat16)
    cos, sin = tables(B, T, D, 3)
    x = qkv.to(dev)[:, :, 0]
    out = jo.apply_rotary_emb(x, (cos.unsqueeze(0).to(dev), sin.unsqueeze(0).to(dev)))
    torch.cuda.synchronize()
    assert out.is_contiguous() and out.shape == (B, T, H, D)
    assert bits_equal(out.cpu(), ops.apply_rotary_emb(qkv[:, :, 0], cos, sin))
    # bf16 tables are promoted like x.float() * cos does
    out16 = jo.apply_rotary_emb(x, (cos.to(torch.bfloat16).to(dev), sin.to(torch.bfloat16).to(dev)))
    ref16 = ops.apply_rotary_emb(qkv[:, :, 0], cos.to(torch.bfloat16).float(),
                                 sin.to(torch.bfloat16).float())
    torch.cuda.synchronize()
    assert bits_equal(out16.cpu(), ref16)

    # the graph runner's commit through the DiT shim
    L, T, P, H = 4, 1560, 3120, 32
    sk = torch.randn(L, 1, T, H, D, generator=g).to(torch.bfloat16)
    sv = torch.randn(L, 1, T, H, D, generator=g).to(torch.bfloat16)
    pk = torch.randn(L, 1, P, H, D, generator=g).to(torch.bfloat16)
    pv = torch.randn(L, 1, P, H, D, generator=g).to(torch.bfloat16)
    c, s = ops.rope_grid_tables(1, 30, 52, 7, (16, 56, 56), 256.0)
    c, s = c.unsqueeze(0), s.unsqueeze(0)                     # [1, T, D] like commit_cos
    pkd, pvd = pk.to(dev), pv.to(dev)
    dit_ops.commit_kv_pool(pkd, pvd, sk.to(dev), sv.to(dev), 1560, c.to(dev), s.to(dev))
    torch.cuda.synchronize()
    rk, rv = ops.commit_kv(pk, pv, sk, sv, 1560, c[0], s[0])
    assert bits_equal(pkd.cpu(), rk) and bits_equal(pvd.cpu(), rv)

    with pytest.raises(RuntimeError, match="dst_offset"):
        jo.kv_commit_rope(sk.to(dev), pkd, 2000, c.to(dev), s.to(dev))


def test_commit_abi_rejects_out_of_range_segment(abi, dev, stream_handle):
    x = torch.zeros(1, 1, 4, 1, 8, dtype=torch.bfloat16, device=dev)
    pool = torch.zeros(1, 1, 6, 1, 8, dtype=torch.bfloat16, device=dev)
    c = torch.zeros(4, 8, device=dev)
    with pytest.raises(RuntimeError, match="exceed the destination"):
        abi.call("jo_kv_commit_rope", x.data_ptr(), None, pool.data_ptr(), None, 1, 1, 4, 1, 8,
                 32, 32, 8, 48, 48, 8, 6, 3, c.data_ptr(), c.data_ptr(), 8, 0,
                 abi.dtype_code(torch.bfloat16), stream_handle)


def test_commit_in_captured_graph(dev):
    """The commit runs inside the graph runner's captured graph: capture it
    once, then replay it three times with new stage contents and tables
    written between replays (eager work and synchronization in between), and
    check every replay."""
    import joyomni_ops as jo
    L, B, T, P, H, D = 3, 1, 64, 128, 8, 128
    g = torch.Generator().manual_seed(8)
    sk = torch.zeros(L, B, T, H, D, dtype=torch.bfloat16, device=dev)
    sv = torch.zeros_like(sk)
    pk = torch.zeros(L, B, P, H, D, dtype=torch.bfloat16, device=dev)
    pv = torch.zeros_like(pk)
    cos = torch.zeros(1, T, D, device=dev)
    sin = torch.zeros(1, T, D, device=dev)
    stream = torch.cuda.Stream(dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        jo.kv_commit_rope(sk, pk, T, cos, sin, src_v=sv, dst_v=pv)   # warm-up
    torch.cuda.current_stream(dev).wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        jo.kv_commit_rope(sk, pk, T, cos, sin, src_v=sv, dst_v=pv)
    for rep in range(3):
        hk = torch.randn(L, B, T, H, D, generator=g).to(torch.bfloat16)
        hv = torch.randn(L, B, T, H, D, generator=g).to(torch.bfloat16)
        c, s = tables(B, T, D, 100 + rep)
        p0k, p0v = pk.cpu(), pv.cpu()
        sk.copy_(hk.to(dev))
        sv.copy_(hv.to(dev))
        cos.copy_(c.unsqueeze(0).to(dev))
        sin.copy_(s.unsqueeze(0).to(dev))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        rk, rv = ops.commit_kv(p0k, p0v, hk, hv, T, c, s)
        assert bits_equal(pk.cpu(), rk) and bits_equal(pv.cpu(), rv), f"replay {rep}"
