"""GPU test: the image stream of one MMDoubleStreamBlock (dit.py:351-457, FP8
mode, the deployment shape [1, 3120, 4096], 32 heads) composed twice from this
package's ops, with the attention output a fixed input.

`block_reference` makes the reference forward's calls with its caller glue
(sgl_fused_ops.py:30-117: expanded modulation rows, .contiguous() q / k copies,
halved bf16 rotation tables; fp8_linear.py:155-169) through the drop-in ops;
`block_fused` makes them through the fused callers (LayerNorm + AdaLN + FP8 in
one pass, QK norm + RoPE from grid positions in place on the packed qkv, gated
residual + LayerNorm + AdaLN + FP8 in one pass, GELU + FP8 in one pass). With
torch's GELU kept (fuse_gelu=False) the residual stream that leaves the block
must be bit-identical; with the fused GELU it may differ where the two GELU
evaluations round a bf16 activation differently (each within 1 ulp of the
formula, tests/test_gpu_gelu_quant.py), and the residual is held to 1 bf16 ulp
of the reference composition's (floored at 2^-10 of the row maximum). q and k
are each checked against the CPU oracle with the tables their path uses (fp32
grid tables for the fused path, the reference's bf16 tables for the drop-in
path) to 1 bf16 ulp.
"""
from __future__ import annotations

import pytest
import torch

from helpers import assert_bf16_within_ulp
from oracle import ops
from joyomni_ops import workloads as W

pytestmark = pytest.mark.gpu


def head_floor(ref: torch.Tensor) -> torch.Tensor:
    return ref.abs().amax(dim=-1, keepdim=True)


def test_block_fused_matches_reference_composition(dev):
    from joyomni_ops import dit_ops
    d = W.BLOCK
    B, L, D, H, Dh, eps = d["B"], d["L"], d["D"], d["H"], d["Dh"], d["eps"]
    b = W.make_block(dev)
    img0 = b["img"].clone()
    # the pre-norm q / k the block's QK step sees (the qkv GEMM is deterministic)
    x_q, x_s = dit_ops.layernorm_modulate_fp8(img0, b["shift1"], b["scale1"], eps=eps)
    qkv_pre = dit_ops.fp8_linear_quantized(x_q, x_s, *b["qkv"]).view(B, L, 3, H, Dh).cpu()

    r_in = img0.clone()
    r_img, r_q, r_k = W.block_reference(b, r_in)
    u_img, _, _ = W.block_fused(b, img0.clone(), fuse_gelu=False)
    f_in = img0.clone()
    f_img, f_q, f_k = W.block_fused(b, f_in)
    torch.cuda.synchronize()
    print(f"block [{B}, {L}, {D}]: residual max |ref| {r_img.float().abs().max().item():.3f}",
          flush=True)

    assert torch.isfinite(r_img.float()).all()
    assert torch.equal(u_img.cpu(), r_img.cpu()), "residual stream differs between compositions"
    ref = r_img.float().cpu()
    assert_bf16_within_ulp(f_img.cpu(), ref, ref.abs().amax(-1, keepdim=True),
                           what="residual with the fused GELU")
    print(f"fused GELU: {int((f_img != r_img).sum())} of {r_img.numel()} residual values differ",
          flush=True)
    assert torch.equal(r_in.cpu(), img0.cpu()), "block_reference modified its input"

    frames = L // (d["grid"][0] * d["grid"][1])
    cos_f, sin_f = ops.half_tables(*ops.rope_grid_tables(frames, *d["grid"], d["t0"],
                                                         d["rope_dims"], d["theta"]))
    cos_b, sin_b = (t.squeeze(0)[..., ::2].to(torch.bfloat16).cpu() for t in b["freqs_cis"])
    for name, pre, w, fused, ref in (("q", qkv_pre[:, :, 0], b["q_norm"], f_q, r_q),
                                     ("k", qkv_pre[:, :, 1], b["k_norm"], f_k, r_k)):
        w = w.cpu()
        want_f = ops.qk_norm_rope_f32(pre, w, cos_f, sin_f, eps)
        assert_bf16_within_ulp(fused.cpu(), want_f, head_floor(want_f), what=f"fused {name}")
        want_r = ops.qk_norm_rope_f32(pre, w, cos_b, sin_b, eps)
        assert_bf16_within_ulp(ref.cpu(), want_r, head_floor(want_r), what=f"reference {name}")
