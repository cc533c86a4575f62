"""The ops inside HIP-graph capture, as the reference's graph runner records
them (deploy/xvideo/serving/graph_runner.py:169-171).

One image-stream block of the DiT at a small shape (dit.py:351-476 with the
FP8 linears of fp8_linear.py:138-169, up to the MLP activation quantized for
the down projection) is captured once into a graph; then,
three times, new inputs are copied into the graph's static buffers, the graph
is replayed, and every output is compared bit for bit with the same block run
eagerly on the same inputs (eager work and synchronizations in between, and a
different residual each time, since the block updates it in place).
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

B, F, GH, GW, H, D = 1, 2, 4, 6, 4, 128
L = F * GH * GW
HID = H * D
UP = 2 * HID


def make_inputs(seed: int) -> dict:
    g = torch.Generator().manual_seed(seed)
    bf = torch.bfloat16

    def r(*shape, s=1.0):
        return (torch.randn(*shape, generator=g) * s).to(bf)

    return {
        "img": r(B, L, HID), "res": r(B, L, HID), "txt_qkv": r(B, 16, 3, H, D),
        "shift1": r(B, HID, s=0.2), "scale1": r(B, HID, s=0.2),
        "shift2": r(B, HID, s=0.2), "scale2": r(B, HID, s=0.2), "gate": r(B, HID),
        "qw": (1 + 0.1 * torch.randn(D, generator=g)).to(bf),
        "kw": (1 + 0.1 * torch.randn(D, generator=g)).to(bf),
        "tqw": (1 + 0.1 * torch.randn(D, generator=g)).to(bf),
        "w_qkv": r(3 * HID, HID, s=0.05), "b_qkv": r(3 * HID),
        "w_up": r(UP, HID, s=0.05), "b_up": r(UP),
    }


def prepare(host: dict, dev) -> dict:
    """Device copies, with the linear weights quantized as Fp8Linear.from_linear does."""
    from joyomni_ops import dit_ops
    s = {k: v.to(dev) for k, v in host.items() if not k.startswith("w_")}
    for name in ("qkv", "up"):
        s[f"wq_{name}"], s[f"ws_{name}"] = dit_ops.quantize_weight_per_channel(host[f"w_{name}"].to(dev))
    return s


def block(s: dict, qk: str = "views") -> dict:
    """qk = "views": the pre-RoPE K norm, then grid RoPE in place on the qkv
    views (two ops); "kstage": both in one pass (the *_kstage op)."""
    import joyomni_ops as jo
    from joyomni_ops import dit_ops
    x_q, x_s = dit_ops.layernorm_modulate_fp8(s["img"], s["shift1"], s["scale1"])
    qkv = dit_ops.fp8_linear_quantized(x_q, x_s, s["wq_qkv"], s["ws_qkv"], s["b_qkv"])
    iv = qkv.view(B, L, 3, H, D)
    if qk == "views":
        k_pre = dit_ops.rmsnorm_qk_bf16(iv[:, :, 1], s["kw"])
        q, k = dit_ops.fused_qk_norm_rope_3d_grid_views(
            iv[:, :, 0], iv[:, :, 1], s["qw"], s["kw"], grid_hw=(GH, GW), t0=3,
            rope_dims=(16, 56, 56), theta=256.0, source_id=1.0)
    else:
        k_pre = torch.empty(B, L, H, D, dtype=torch.bfloat16, device=qkv.device)
        freqs = jo.rope_freqs(D, (16, 56, 56), 256.0, 256.0, 128)
        jo.fused_qk_norm_rope_3d_grid_kstage(iv[:, :, 0], iv[:, :, 1], k_pre, L, H, 1e-6,
                                             s["qw"], s["kw"], freqs, (16, 56, 56), (GH, GW), 3,
                                             1.0)
        q = iv[:, :, 0]
    attn = q.reshape(B, L, HID)  # stands in for the attention output
    res, x_q2, x_s2 = dit_ops.fused_add_gate_layernorm_modulate_fp8(
        s["res"], attn, s["gate"], s["shift2"], s["scale2"])
    up = dit_ops.fp8_linear_quantized(x_q2, x_s2, s["wq_up"], s["ws_up"], s["b_up"])
    h_q, h_s = dit_ops.gelu_quantize_activation_fp8(up)  # the MLP activation, quantized
    txt_q = dit_ops.rms_norm_module(s["txt_qkv"][:, :, 0], s["tqw"])
    return {"x_q": x_q, "x_s": x_s, "qkv": qkv, "k_pre": k_pre, "res": res, "x_q2": x_q2,
            "x_s2": x_s2, "up": up, "h_q": h_q, "h_s": h_s, "txt_q": txt_q}


def as_bits(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t


def test_dit_block_graph_replays_match_eager(dev):
    static = prepare(make_inputs(0), dev)
    block(static)  # eager warm-up: the frequency table is cached outside the graph
    torch.cuda.synchronize()
    static = prepare(make_inputs(0), dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = block(static)
    torch.cuda.synchronize()
    for rep in range(1, 4):
        fresh = prepare(make_inputs(rep), dev)
        for k, v in fresh.items():
            static[k].copy_(v)
        graph.replay()
        torch.cuda.synchronize()
        got = {k: v.clone() for k, v in outs.items()}
        want = block(prepare(make_inputs(rep), dev))  # eager, on its own buffers
        torch.cuda.synchronize()
        for k in want:
            assert torch.equal(as_bits(got[k]), as_bits(want[k])), f"replay {rep}: {k} differs"
        assert bool(got["up"].float().abs().sum() > 0), "graph produced nothing"


def test_graph_captured_on_first_use_with_kstage(dev):
    """Nothing runs eagerly before the capture (the grid RoPE frequencies travel
    in the kernel arguments, so the first call needs no device setup): the
    block with the one-pass K stage is captured cold, replayed three times with
    new inputs, and every replay equals, bit for bit, the eager two-op block."""
    import joyomni_ops as jo
    jo._FREQ_CACHE.clear()
    static = prepare(make_inputs(10), dev)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = block(static, "kstage")
    torch.cuda.synchronize()
    for rep in range(11, 14):
        fresh = prepare(make_inputs(rep), dev)
        for k, v in fresh.items():
            static[k].copy_(v)
        graph.replay()
        torch.cuda.synchronize()
        got = {k: v.clone() for k, v in outs.items()}
        want = block(prepare(make_inputs(rep), dev), "views")
        torch.cuda.synchronize()
        for k in want:
            assert torch.equal(as_bits(got[k]), as_bits(want[k])), f"replay {rep}: {k} differs"


@pytest.mark.parametrize("M,N,K,shape", [
    (700, 1000, 640, 3),     # 224-row pair tiles, one round: B three stages in the ring
    (3120, 5120, 256, 3),    # 224-row pair tiles, 280 of them (two rounds): two slots
    (64, 4096, 8192, -1),    # few rows, long K: the split-K partials and their reduction
])
def test_fp8_scaled_mm_graph_replays_match_eager(dev, M, N, K, shape):
    """The FP8 GEMM captured into a graph (its split-K workspace taken from the
    caching allocator during capture), replayed three times with new operands
    copied into the captured buffers, each replay bit-identical to the eager
    call on the same operands."""
    import joyomni_ops as jo
    from joyomni_ops import _abi

    def operands(seed):
        g = torch.Generator().manual_seed(seed)
        a = (torch.randn(M, K, generator=g) * 2).to(torch.float8_e4m3fn)
        w = (torch.randn(N, K, generator=g) * 2).to(torch.float8_e4m3fn)
        sa = torch.rand(M, 1, generator=g) + 0.5
        sb = torch.rand(1, N, generator=g) + 0.5
        bias = torch.randn(N, generator=g).to(torch.bfloat16)
        return [t.to(dev) for t in (a, w, sa, sb, bias)]

    _abi.call("jo_set_launch_override", _abi.JO_KNOB_GEMM_SHAPE, shape)
    try:
        static = operands(100)
        jo.fp8_scaled_mm(static[0], static[1].t(), static[2], static[3], torch.bfloat16, static[4])
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = jo.fp8_scaled_mm(static[0], static[1].t(), static[2], static[3],
                                   torch.bfloat16, static[4])
        torch.cuda.synchronize()
        for rep in range(101, 104):
            fresh = operands(rep)
            for s_t, f_t in zip(static, fresh):
                s_t.copy_(f_t)
            graph.replay()
            torch.cuda.synchronize()
            got = out.clone()
            want = jo.fp8_scaled_mm(fresh[0], fresh[1].t(), fresh[2], fresh[3], torch.bfloat16,
                                    fresh[4])
            torch.cuda.synchronize()
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"replay {rep} differs"
            assert bool(got.float().abs().sum() > 0)
    finally:
        _abi.call("jo_set_launch_override", _abi.JO_KNOB_GEMM_SHAPE, -1)
