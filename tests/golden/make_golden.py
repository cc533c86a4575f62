"""Writes tests/golden/fixtures.npz: small seeded inputs of every hot-path op
with the CPU oracle's outputs (the reference ships no golden vectors, so these
are the build's own, pinned by the checks in tests/test_oracle.py).

    python tests/golden/make_golden.py

The file is data only (numpy arrays, no pickles): bf16 tensors are stored as
their uint16 bit patterns, fp8 tensors as uint8 codes. tests/test_golden.py
checks that the oracle still reproduces every output exactly (CPU) and that
the HIP kernels match them (GPU).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import ops  # noqa: E402

OUT = Path(__file__).resolve().parent / "fixtures.npz"


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> uint16 bit patterns."""
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def f32(t: torch.Tensor) -> np.ndarray:
    return t.float().contiguous().numpy()


def with_outliers(x: torch.Tensor, g: torch.Generator) -> torch.Tensor:
    flat = x.reshape(-1)
    idx = torch.randperm(flat.numel(), generator=g)[:round(0.005 * flat.numel())]
    flat[idx] *= 40
    return x


def build() -> dict[str, np.ndarray]:
    fx: dict[str, np.ndarray] = {}

    # Per-token FP8 quant (per_token_quant_fp8.cu:56-82): random rows with
    # outliers plus a zero row, a row with a NaN, one with an inf and one of
    # tiny values whose inverse scale overflows.
    g = torch.Generator().manual_seed(100)
    x = with_outliers(torch.randn(8, 3072, generator=g), g)
    x[0] = 0.0
    x[1, 17] = float("nan")
    x[2, 5] = float("inf")
    x[3] = torch.randn(3072, generator=g) * 2.0 ** -130
    x = x.to(torch.bfloat16)
    q, s = ops.per_token_quant_fp8(x)
    fx.update(quant_x=bits(x), quant_q=q.numpy(), quant_s=f32(s))

    # RMSNorm -> FP8, per token and per 1x128 block.
    g = torch.Generator().manual_seed(101)
    x = with_outliers(torch.randn(6, 3072, generator=g), g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(3072, generator=g)).to(torch.bfloat16)
    qt, st, _ = ops.rmsnorm_quant_fp8(x, w, 1e-6, 0)
    qb, sb, _ = ops.rmsnorm_quant_fp8(x, w, 1e-6, 128)
    fx.update(rmsq_x=bits(x), rmsq_w=bits(w), rmsq_tok_q=qt.numpy(), rmsq_tok_s=f32(st),
              rmsq_blk_q=qb.numpy(), rmsq_blk_s=f32(sb))

    # QK RMSNorm + RoPE, table mode (fused_qknorm_rope_3d_kernel.cu:98-142):
    # q, k [1, L*H, D] with bf16 [L, D/2] tables.
    g = torch.Generator().manual_seed(102)
    L, H, D = 6, 4, 128
    qq = torch.randn(1, L * H, D, generator=g).to(torch.bfloat16)
    kk = torch.randn(1, L * H, D, generator=g).to(torch.bfloat16)
    wq = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    wk = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    ang = torch.rand(L, D // 2, generator=g) * 50
    cos, sin = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    fx.update(qkt_q=bits(qq), qkt_k=bits(kk), qkt_wq=bits(wq), qkt_wk=bits(wk),
              qkt_cos=bits(cos), qkt_sin=bits(sin),
              qkt_q_ref=f32(ops.qk_norm_rope_f32(qq.reshape(1, L, H, D), wq, cos, sin, 1e-6)),
              qkt_k_ref=f32(ops.qk_norm_rope_f32(kk.reshape(1, L, H, D), wk, cos, sin, 1e-6)))

    # Grid mode: 2 frames of a 3 x 5 grid, t0 7, split 44/42/42, theta 1e4,
    # source id 1 (angle addition with theta 256).
    g = torch.Generator().manual_seed(103)
    F, gh, gw, H, D = 2, 3, 5, 2, 128
    L = F * gh * gw
    qq = torch.randn(1, L * H, D, generator=g).to(torch.bfloat16)
    kk = torch.randn(1, L * H, D, generator=g).to(torch.bfloat16)
    wq = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    wk = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    args = (F, gh, gw, 7, (44, 42, 42), 10000.0, 1e-6, 1.0, 256.0)
    fx.update(qkg_q=bits(qq), qkg_k=bits(kk), qkg_wq=bits(wq), qkg_wk=bits(wk),
              qkg_q_ref=f32(ops.qk_norm_rope_grid_f32(qq.reshape(1, L, H, D), wq, *args)),
              qkg_k_ref=f32(ops.qk_norm_rope_grid_f32(kk.reshape(1, L, H, D), wk, *args)))

    # Norm + AdaLN with per-row scale/shift (fused_norm_scale_shift.cu:88-142),
    # LayerNorm with gamma/beta and RMSNorm with gamma.
    g = torch.Generator().manual_seed(104)
    x = (torch.randn(4, 512, generator=g) * 2 + 0.5).to(torch.bfloat16)
    sc = torch.randn(4, 512, generator=g).to(torch.bfloat16)
    sh = torch.randn(4, 512, generator=g).to(torch.bfloat16)
    gm = torch.randn(512, generator=g).to(torch.bfloat16)
    bt = torch.randn(512, generator=g).to(torch.bfloat16)
    fx.update(nss_x=bits(x), nss_scale=bits(sc), nss_shift=bits(sh), nss_gamma=bits(gm),
              nss_beta=bits(bt),
              nss_ln_ref=f32(ops.norm_scale_shift_f32(x, gm, bt, sc, sh, 0, 1e-5)),
              nss_rms_ref=f32(ops.norm_scale_shift_f32(x, gm, None, sc, sh, 1, 1e-5)))

    # RMSNorm (rmsnorm.cu:41-60).
    g = torch.Generator().manual_seed(105)
    x = torch.randn(5, 128, generator=g).to(torch.bfloat16)
    w = torch.randn(128, generator=g).to(torch.bfloat16)
    fx.update(rms_x=bits(x), rms_w=bits(w), rms_ref=f32(ops.rmsnorm_f32(x, w, 1e-6)))

    # Gated residual add + LayerNorm + AdaLN (sgl_fused_ops.py:114-117 then
    # the LayerNorm path) with broadcast modulation rows.
    g = torch.Generator().manual_seed(106)
    x = torch.randn(4, 3072, generator=g).to(torch.bfloat16)
    res = torch.randn(4, 3072, generator=g).to(torch.bfloat16)
    gate = torch.randn(3072, generator=g).to(torch.bfloat16)
    sc = (0.2 * torch.randn(3072, generator=g)).to(torch.bfloat16)
    sh = (0.2 * torch.randn(3072, generator=g)).to(torch.bfloat16)
    new_res, y = ops.add_layernorm_scale_shift(x, res, gate, None, None, sc, sh, 1e-6)
    fx.update(addln_x=bits(x), addln_res=bits(res), addln_gate=bits(gate), addln_scale=bits(sc),
              addln_shift=bits(sh), addln_new_res=bits(new_res), addln_y_ref=f32(y))

    # KV-pool commit (graph_runner.py:137-142 with rope.py:14-28): 2 layers,
    # 3 tokens into a 6-token pool at offset 2.
    g = torch.Generator().manual_seed(107)
    Lr, T, P, H, D = 2, 3, 6, 2, 64
    sk = torch.randn(Lr, 1, T, H, D, generator=g).to(torch.bfloat16)
    sv = torch.randn(Lr, 1, T, H, D, generator=g).to(torch.bfloat16)
    pk = torch.randn(Lr, 1, P, H, D, generator=g).to(torch.bfloat16)
    pv = torch.randn(Lr, 1, P, H, D, generator=g).to(torch.bfloat16)
    ang = torch.rand(T, D // 2, generator=g) * 20
    cos = ang.cos().repeat_interleave(2, 1).contiguous()
    sin = ang.sin().repeat_interleave(2, 1).contiguous()
    nk, nv = ops.commit_kv(pk, pv, sk, sv, 2, cos, sin)
    fx.update(kvc_stage_k=bits(sk), kvc_stage_v=bits(sv), kvc_pool_k=bits(pk), kvc_pool_v=bits(pv),
              kvc_cos=f32(cos), kvc_sin=f32(sin), kvc_new_k=bits(nk), kvc_new_v=bits(nv))

    # Row-wise scaled FP8 GEMM with bias (fp8_gemm.cu:1450-1546, epilogue
    # :99-136): A [16, 128], B^T [32, 128] as e4m3fn codes.
    g = torch.Generator().manual_seed(108)
    a = (torch.randn(16, 128, generator=g) * 3).to(torch.float8_e4m3fn)
    bt8 = (torch.randn(32, 128, generator=g) * 3).to(torch.float8_e4m3fn)
    sa = torch.rand(16, generator=g) * 0.01 + 1e-3
    sbv = torch.rand(32, generator=g) * 0.01 + 1e-3
    bias = torch.randn(32, generator=g).to(torch.bfloat16)
    out, acc, mag = ops.fp8_scaled_mm(a, bt8.t(), sa, sbv, torch.bfloat16, bias)
    exact = acc * sa.double()[:, None] * sbv.double()[None, :] + bias.double()[None, :]
    fx.update(gemm_a=a.view(torch.uint8).numpy(), gemm_bt=bt8.view(torch.uint8).numpy(),
              gemm_sa=f32(sa), gemm_sb=f32(sbv), gemm_bias=bits(bias), gemm_out=bits(out),
              gemm_exact=exact.numpy(), gemm_mag=mag.numpy())

    # The torch RMSNorm module (dit.py:244-249) on per-head rows [T, H, D]:
    # rounded to bf16 before the weight multiply.
    g = torch.Generator().manual_seed(109)
    x = (torch.randn(5, 3, 128, generator=g) * 2).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16)
    fx.update(rmsmod_x=bits(x), rmsmod_w=bits(w), rmsmod_y=bits(ops.rms_norm_module(x, w, 1e-6)))

    # GELU(tanh) + per-token FP8 (dit.py:91-92,433, then fp8_linear.py:140-166):
    # the fp32 activation of the formula, and the oracle's bytes and scales on
    # its bf16 rounding; rows with NaN / +-inf and a deep negative tail.
    g = torch.Generator().manual_seed(110)
    x = with_outliers(3 * torch.randn(6, 4096, generator=g), g)
    x[0, :3] = torch.tensor([float("nan"), float("inf"), float("-inf")])
    x[1, :64] = -20.0
    x = x.to(torch.bfloat16)
    q, s, _ = ops.gelu_tanh_quant_fp8(x)
    fx.update(gelu_x=bits(x), gelu_act=f32(ops.gelu_tanh_f32(x)), gelu_q=q.numpy(),
              gelu_s=f32(s))
    return fx


if __name__ == "__main__":
    fx = build()
    np.savez_compressed(OUT, **fx)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(fx)} arrays)")
