"""GPU tests of the DiT call shims (joyomni_ops.dit_ops), the counterparts of
deploy/xvideo/models/dit/sgl_fused_ops.py and of Fp8Linear's activation
quantization, against the CPU oracle composed the way the reference composes
those calls. Tolerances as in the op tests (1 output ulp, floored at 2^-10 of
the row/head scale); FP8 bytes and the gated residual bit-exact."""
from __future__ import annotations

import pytest
import torch

from helpers import assert_bf16_within_ulp, assert_within_ulp
from oracle import ops

pytestmark = pytest.mark.gpu


def rowmax(t):
    return t.abs().amax(dim=-1, keepdim=True)


@pytest.mark.parametrize("B,L,D", [(1, 1560, 3072), (2, 33, 512), (1, 1, 256)])
@pytest.mark.parametrize("affine", [False, True])
@pytest.mark.parametrize("mod_shape", ["BD", "B1D", "BLD"])
def test_fused_layernorm_modulate(dev, B, L, D, affine, mod_shape):
    from joyomni_ops import dit_ops
    g = torch.Generator().manual_seed(B * L + D)
    x = torch.randn(B, L, D, generator=g).to(torch.bfloat16)
    shp = {"BD": (B, D), "B1D": (B, 1, D), "BLD": (B, L, D)}[mod_shape]
    shift = (0.2 * torch.randn(shp, generator=g)).to(torch.bfloat16)
    scale = (0.2 * torch.randn(shp, generator=g)).to(torch.bfloat16)
    w = torch.randn(D, generator=g).to(torch.bfloat16) if affine else None
    b = torch.randn(D, generator=g).to(torch.bfloat16) if affine else None
    y = dit_ops.fused_layernorm_modulate(x.to(dev), shift.to(dev), scale.to(dev),
                                         weight=None if w is None else w.to(dev),
                                         bias=None if b is None else b.to(dev), eps=1e-6)
    torch.cuda.synchronize()
    # reference composition: sgl_fused_ops.py:41-54
    sc = scale.unsqueeze(1) if scale.dim() == 2 else scale
    sh = shift.unsqueeze(1) if shift.dim() == 2 else shift
    sc = sc.expand(B, L, D).reshape(-1, D)
    sh = sh.expand(B, L, D).reshape(-1, D)
    ref = ops.norm_scale_shift_f32(x.reshape(-1, D), w, b, sc, sh, 0, 1e-6).reshape(B, L, D)
    assert y.shape == (B, L, D)
    assert_within_ulp(y.cpu(), ref, torch.bfloat16, rowmax(ref), what="layernorm_modulate")


@pytest.mark.parametrize("mod_shape", ["BD", "B1D"])
def test_fused_layernorm_modulate_per_sample_in_place(dev, mod_shape):
    """B = 2 per-sample shift / scale: read in place (the only new allocation is
    the output: no [B*L, D] expanded copies), bit-identical to the reference
    op on the expanded copies the reference caller makes
    (sgl_fused_ops.py:44-51), and within the bar of the oracle."""
    import joyomni_ops as jo
    from joyomni_ops import dit_ops
    B, L, D = 2, 1560, 3072
    g = torch.Generator().manual_seed(31)
    x = torch.randn(B, L, D, generator=g).to(torch.bfloat16)
    shp = (B, D) if mod_shape == "BD" else (B, 1, D)
    shift = (0.2 * torch.randn(shp, generator=g)).to(torch.bfloat16)
    scale = (0.2 * torch.randn(shp, generator=g)).to(torch.bfloat16)
    xd, shd, scd = x.to(dev), shift.to(dev), scale.to(dev)
    dit_ops.fused_layernorm_modulate(xd, shd, scd)  # warm the allocator's pools
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated(dev)
    torch.cuda.reset_peak_memory_stats(dev)
    y = dit_ops.fused_layernorm_modulate(xd, shd, scd)
    torch.cuda.synchronize()
    extra = torch.cuda.max_memory_allocated(dev) - base
    out_bytes = y.numel() * y.element_size()
    assert extra <= out_bytes + 4096, f"{extra} bytes allocated for a {out_bytes}-byte output"
    sc2 = scd.reshape(B, 1, D).expand(B, L, D).reshape(-1, D).contiguous()
    sh2 = shd.reshape(B, 1, D).expand(B, L, D).reshape(-1, D).contiguous()
    y_ref_op = jo.fused_norm_scale_shift(xd.reshape(-1, D), None, None, sc2, sh2, "layer", 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(y.reshape(-1, D), y_ref_op), "differs from the op on expanded copies"
    ref = ops.norm_scale_shift_f32(x.reshape(-1, D), None, None, sc2.cpu(), sh2.cpu(), 0, 1e-6)
    assert_within_ulp(y.cpu().reshape(-1, D), ref, torch.bfloat16, rowmax(ref),
                      what="per-sample layernorm_modulate")


def test_norm_scale_shift_per_sample_op(dev):
    """The per-sample op: [N], [M, N] and [B, N] modulation, LN and RMS, with
    gamma / beta, each bit-identical to the reference op on the expanded rows;
    shapes that do not divide M are refused."""
    import joyomni_ops as jo
    M, N, B = 96, 512, 4
    g = torch.Generator().manual_seed(8)
    x = torch.randn(M, N, generator=g).to(torch.bfloat16).to(dev)
    gam = (1 + 0.1 * torch.randn(N, generator=g)).to(torch.bfloat16).to(dev)
    bet = (0.1 * torch.randn(N, generator=g)).to(torch.bfloat16).to(dev)
    for rows in (1, B, M):
        sc = (0.2 * torch.randn(rows, N, generator=g)).to(torch.bfloat16).to(dev)
        sh = (0.2 * torch.randn(rows, N, generator=g)).to(torch.bfloat16).to(dev)
        sc_in, sh_in = (sc[0], sh[0]) if rows == 1 else (sc, sh)
        full_sc = sc.repeat_interleave(M // rows, dim=0)
        full_sh = sh.repeat_interleave(M // rows, dim=0)
        for nt in ("layer", "rms"):
            for gb in ((None, None), (gam, bet)):
                y = jo.fused_norm_scale_shift_per_sample(x, gb[0], gb[1], sc_in, sh_in, nt, 1e-6)
                r = jo.fused_norm_scale_shift(x, gb[0], gb[1], full_sc, full_sh, nt, 1e-6)
                torch.cuda.synchronize()
                assert torch.equal(y, r), (rows, nt, gb[0] is None)
    bad = torch.zeros(5, N, dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError, match="B dividing M"):
        jo.fused_norm_scale_shift_per_sample(x, None, None, bad, bad, "layer", 1e-6)


def test_fused_qk_norm_rope_3d_dit_tables(dev):
    """Reference contract: q/k views of qkv, fp32 [1, L, D] tables; returns new tensors."""
    from joyomni_ops import dit_ops
    B, L, H, D = 1, 1560, 32, 128
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(B, L, 3, H, D, generator=g).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    cos, sin = ops.rope_grid_tables(1, 30, 52, 4, (16, 56, 56), 256.0, 1.0, 256.0)
    d = qkv.to(dev)
    q2, k2 = dit_ops.fused_qk_norm_rope_3d(d[:, :, 0], d[:, :, 1], qw.to(dev), kw.to(dev),
                                           (cos[None].to(dev), sin[None].to(dev)), eps=1e-6)
    torch.cuda.synchronize()
    assert torch.equal(d.cpu(), qkv), "inputs must not be modified"
    c16, s16 = (t.to(torch.bfloat16) for t in ops.half_tables(cos, sin))
    for out, x, w in ((q2, qkv[:, :, 0], qw), (k2, qkv[:, :, 1], kw)):
        ref = ops.qk_norm_rope_f32(x.contiguous(), w, c16, s16, 1e-6)
        assert_bf16_within_ulp(out.cpu(), ref, rowmax(ref), what="dit qk tables")


@pytest.mark.parametrize("sid", [0.0, 1.0, 2.0])
def test_grid_views_on_packed_qkv(dev, sid):
    """In place on strided views of qkv [B, L, 3, H, D]; v untouched; angles
    from the DiT's grid (30x52, rope dims 16/56/56, theta 256, source id)."""
    from joyomni_ops import dit_ops
    B, L, H, D = 1, 1560, 32, 128
    g = torch.Generator().manual_seed(6)
    qkv = torch.randn(B, L, 3, H, D, generator=g).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    d = qkv.to(dev)
    dit_ops.fused_qk_norm_rope_3d_grid_views(d[:, :, 0], d[:, :, 1], qw.to(dev), kw.to(dev),
                                             grid_hw=(30, 52), t0=9, rope_dims=(16, 56, 56),
                                             theta=256.0, source_id=sid)
    torch.cuda.synchronize()
    out = d.cpu()
    assert torch.equal(out[:, :, 2], qkv[:, :, 2])
    cos, sin = ops.half_tables(*ops.rope_grid_tables(1, 30, 52, 9, (16, 56, 56), 256.0, sid, 256.0))
    for j, w in ((0, qw), (1, kw)):
        ref = ops.qk_norm_rope_f32(qkv[:, :, j].contiguous(), w, cos, sin, 1e-6)
        assert_bf16_within_ulp(out[:, :, j], ref, rowmax(ref), what=f"grid views sid={sid}")


@pytest.mark.parametrize("sid,source_dim", [(1.0, None), (3.0, None), (3.0, 256)])
def test_grid_views_head_dim_256_source_rotation(dev, sid, source_dim):
    """head_dim 256 with a source id: the source rotation covers the first
    min(source_dim, D) dims, source_dim 128 by default (the model's
    source_id_rope_dim, dit.py:792, config.py:35), against the oracle's tables
    built with the same split."""
    from joyomni_ops import dit_ops
    B, L, H, D = 1, 96, 4, 256
    dims = (32, 112, 112)
    g = torch.Generator().manual_seed(60 + int(sid))
    qkv = torch.randn(B, L, 3, H, D, generator=g).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    d = qkv.to(dev)
    kwargs = {} if source_dim is None else {"source_dim": source_dim}
    dit_ops.fused_qk_norm_rope_3d_grid_views(d[:, :, 0], d[:, :, 1], qw.to(dev), kw.to(dev),
                                             grid_hw=(8, 12), t0=5, rope_dims=dims,
                                             theta=256.0, source_id=sid, **kwargs)
    torch.cuda.synchronize()
    out = d.cpu()
    sd = 128 if source_dim is None else source_dim
    cos, sin = ops.half_tables(*ops.rope_grid_tables(1, 8, 12, 5, dims, 256.0, sid, 256.0, sd))
    for j, w in ((0, qw), (1, kw)):
        ref = ops.qk_norm_rope_f32(qkv[:, :, j].contiguous(), w, cos, sin, 1e-6)
        assert_bf16_within_ulp(out[:, :, j], ref, rowmax(ref),
                               what=f"D=256 sid={sid} source_dim={source_dim}")
    if source_dim is None:
        # the full-width source rotation is a different table: the split matters
        c2, s2 = ops.half_tables(*ops.rope_grid_tables(1, 8, 12, 5, dims, 256.0, sid, 256.0, D))
        assert not torch.equal(c2, cos)


def test_rmsnorm_qk_bf16_strided(dev):
    from joyomni_ops import dit_ops
    B, L, H, D = 1, 200, 8, 128
    g = torch.Generator().manual_seed(7)
    qkv = torch.randn(B, L, 3, H, D, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    y = dit_ops.rmsnorm_qk_bf16(qkv.to(dev)[:, :, 1], w.to(dev), eps=1e-6)
    torch.cuda.synchronize()
    ref = ops.rmsnorm_f32(qkv[:, :, 1].reshape(-1, D), w, 1e-6).reshape(B, L, H, D)
    assert_bf16_within_ulp(y.cpu(), ref, rowmax(ref), what="rmsnorm_qk_bf16")


@pytest.mark.parametrize("B", [1, 2])
def test_fused_add_gate_layernorm_modulate(dev, B):
    from joyomni_ops import dit_ops
    L, D = 300, 3072
    g = torch.Generator().manual_seed(8 + B)
    res = torch.randn(B, L, D, generator=g).to(torch.bfloat16)
    x = torch.randn(B, L, D, generator=g).to(torch.bfloat16)
    six = torch.randn(B, 6 * D, generator=g).to(torch.bfloat16)  # modulation vector, chunked views
    shift, scale, gate = six[:, :D], six[:, D:2 * D], six[:, 2 * D:3 * D]
    rd = res.to(dev)
    sd = six.to(dev)
    r2, y = dit_ops.fused_add_gate_layernorm_modulate(rd, x.to(dev), sd[:, 2 * D:3 * D],
                                                      sd[:, :D], sd[:, D:2 * D], eps=1e-6)
    torch.cuda.synchronize()
    # reference: fused_add_gate then fused_layernorm_modulate (dit.py:447-457)
    ref_res = torch.addcmul(res.float(), x.float(), gate.float().unsqueeze(1)).to(torch.bfloat16)
    assert r2.data_ptr() == rd.data_ptr()
    assert torch.equal(rd.cpu(), ref_res), "gated residual not bit-exact"
    ref = torch.stack([ops.norm_scale_shift_f32(ref_res[b], None, None, scale[b].expand(L, D),
                                                shift[b].expand(L, D), 0, 1e-6) for b in range(B)])
    assert_within_ulp(y.cpu(), ref, torch.bfloat16, rowmax(ref), what="add_gate_ln")
    # the unfused shim keeps the reference contract
    assert torch.equal(dit_ops.fused_add_gate(res.to(dev), x.to(dev), gate.to(dev)).cpu(),
                       torch.addcmul(res.to(dev), x.to(dev), gate.to(dev).unsqueeze(1)).cpu())


def test_quantize_activation_fp8(dev):
    from joyomni_ops import dit_ops
    g = torch.Generator().manual_seed(9)
    x = torch.randn(2, 1560, 4096, generator=g).to(torch.bfloat16)
    xq, xs = dit_ops.quantize_activation_fp8(x.to(dev))
    torch.cuda.synchronize()
    qo, so = ops.per_token_quant_fp8(x.reshape(-1, 4096))
    assert xq.shape == (3120, 4096) and xs.shape == (3120, 1)
    assert torch.equal(xq.view(torch.uint8).cpu(), qo) and torch.equal(xs.view(-1).cpu(), so)
