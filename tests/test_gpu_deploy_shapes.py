"""The reference-signature ops at the DiT block's deployment shapes (hidden
4096, 32 heads, 3120 tokens per chunk; the bench.py R_* workloads), through
the torch ops the reference's callers use, against the oracle:

  fused_qk_norm_rope_3d_paired  q,k [1, 3120*32, 128], bf16 [3120, 64] tables
                                (sgl_fused_ops.py:57-99 -> fused_qknorm_rope_3d_kernel.cu)
  fused_norm_scale_shift        x [3120, 4096], per-row scale/shift [3120, 4096]
                                (sgl_fused_ops.py:30-54 -> fused_norm_scale_shift.cu)
  sgl_per_token_quant_fp8       x [3120, 4096] and [3120, 16384] (fp8_linear.py:138-169)
  rmsnorm                       pre-RoPE K rows [99840, 128] (sgl_fused_ops.py:102-111)
"""
from __future__ import annotations

import pytest
import torch

from helpers import assert_bf16_within_ulp, assert_within_ulp
from oracle import ops
from joyomni_ops import workloads as W

pytestmark = pytest.mark.gpu


def row_floor(ref):
    return ref.abs().amax(dim=-1, keepdim=True)


def test_deploy_qk_table(dev):
    import joyomni_ops as jo
    cfg = W.CONFIGS["R_qk"]
    d = cfg.dims
    t = W.make_inputs(cfg)
    qd, kd = t["q"].to(dev), t["k"].to(dev)
    jo.fused_qk_norm_rope_3d_paired(qd, kd, d["L"], d["H"], d["eps"], t["q_weight"].to(dev),
                                    t["k_weight"].to(dev), t["cos"].to(dev), t["sin"].to(dev))
    torch.cuda.synchronize()
    for name, out, x, w in (("q", qd, t["q"], t["q_weight"]), ("k", kd, t["k"], t["k_weight"])):
        ref = ops.qk_norm_rope_f32(x.reshape(d["B"], d["L"], d["H"], d["D"]), w, t["cos"], t["sin"],
                                   d["eps"])
        assert_bf16_within_ulp(out.cpu().reshape(ref.shape), ref, row_floor(ref),
                               what=f"R_qk {name}", floor_cap=1e-4)


def test_deploy_norm_scale_shift_rows(dev):
    import joyomni_ops as jo
    cfg = W.CONFIGS["R_ln"]
    t = W.make_inputs(cfg)
    y = jo.fused_norm_scale_shift(t["x"].to(dev), None, None, t["scale"].to(dev),
                                  t["shift"].to(dev), "layer", cfg.dims["eps"])
    torch.cuda.synchronize()
    ref = ops.norm_scale_shift_f32(t["x"], None, None, t["scale"], t["shift"], 0, cfg.dims["eps"])
    assert_within_ulp(y.cpu(), ref, torch.bfloat16, row_floor(ref), what="R_ln")


@pytest.mark.parametrize("name", ["R_q4k", "R_q16k"])
def test_deploy_per_token_quant(dev, name):
    import joyomni_ops as jo
    cfg = W.CONFIGS[name]
    x = W.make_inputs(cfg)["x"]
    M, K = x.shape
    q = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=dev)
    s = torch.empty(M, 1, dtype=torch.float32, device=dev)  # Fp8Linear's [M, 1] scales
    jo.sgl_per_token_quant_fp8(x.to(dev), q, s)
    torch.cuda.synchronize()
    qo, so = ops.per_token_quant_fp8(x)
    nbad = int((q.view(torch.uint8).cpu() != qo).sum())
    assert nbad == 0, f"{name}: {nbad} fp8 bytes differ from the oracle"
    assert torch.equal(s.view(-1).cpu(), so), f"{name}: scales differ"


def test_deploy_rmsnorm_k_rows(dev):
    import joyomni_ops as jo
    cfg = W.CONFIGS["R_rms"]
    t = W.make_inputs(cfg)
    y = jo.rmsnorm(t["x"].to(dev), t["weight"].to(dev), cfg.dims["eps"])
    torch.cuda.synchronize()
    ref = ops.rmsnorm_f32(t["x"], t["weight"], cfg.dims["eps"])
    assert_within_ulp(y.cpu(), ref, torch.bfloat16, row_floor(ref), what="R_rms")
