"""GPU parity of the row-wise scaled FP8 GEMM (jo_fp8_scaled_mm, torch op
fp8_scaled_mm, dit_ops.fp8_linear).

Bar: every output within 1 ulp of the output dtype of the exact result
scale_a[m] * scale_b[n] * sum_k a*b + bias[n] (float64 from the oracle, whose
accumulation is exact for fp8 operands), plus 2^-13 of the scaled sum of |a*b|
terms for the fp32 accumulation inside the matrix cores (a dropped 16-byte K
chunk or a wrong scale is far outside it). The full deployment shapes are
checked on sampled rows (the last, ragged row tile included).
"""
from __future__ import annotations

import pytest
import torch

from oracle import ops

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["auto", "0", "1", "2", "3", "4", "5", "6", "7", "8", "9", "10", "11"],
                autouse=True)
def gemm_shape(request):
    """Every kernel variant: the default choice, 256x256 (8 waves), 256x128
    (4 waves), the register-staged kernel (also the K % 64 != 0 path), 224x256
    (8 waves, 4 and 3 row blocks), 224x128 (4 waves), and the small-tile
    kernel at 128x128, 64x64, 64x128, 128x192 and 128x96 (4 waves), 128x256
    (8 waves) and 64x96 (2 waves)."""
    from joyomni_ops import _abi
    value = -1 if request.param == "auto" else int(request.param)
    _abi.call("jo_set_launch_override", _abi.JO_KNOB_GEMM_SHAPE, value)
    yield request.param
    _abi.call("jo_set_launch_override", _abi.JO_KNOB_GEMM_SHAPE, -1)


def ulp(x, dtype):
    frac = 7 if dtype == torch.bfloat16 else 10
    e = torch.floor(torch.log2(x.abs().clamp_min(2.0 ** -14)))
    return 2.0 ** (e - frac)


def check(out, a, b, sa, sb, bias, what, rows=None):
    """out [M', N] device result (rows `rows` of the full result if given)."""
    a_r = a if rows is None else a[rows]
    sa_r = sa if rows is None else sa[rows]
    _, acc, mag = ops.fp8_scaled_mm(a_r, b, sa_r, sb, out.dtype, bias)
    ref = acc * sa_r.double().reshape(-1, 1) * sb.double().reshape(1, -1)
    if bias is not None:
        ref = ref + bias.double().reshape(1, -1)
    got = out.cpu().double()
    tol = ulp(ref, out.dtype) + mag * 2.0 ** -13
    err = (got - ref).abs()
    bad = (err > tol).nonzero()
    assert bad.numel() == 0, (f"{what}: {bad.shape[0]} outputs off, first {bad[0].tolist()}: "
                              f"{got[tuple(bad[0])].item()} vs {ref[tuple(bad[0])].item()}")


def operands(M, N, K, seed, dtype=torch.bfloat16, with_bias=True):
    g = torch.Generator().manual_seed(seed)
    a = (torch.randn(M, K, generator=g) * 4).to(torch.float8_e4m3fn)
    w = (torch.randn(N, K, generator=g) * 4).to(torch.float8_e4m3fn)   # weight [N, K]
    sa = torch.rand(M, generator=g) * 0.02 + 1e-3
    sb = torch.rand(N, generator=g) * 0.02 + 1e-3
    bias = torch.randn(N, generator=g).to(dtype) if with_bias else None
    return a, w, sa, sb, bias


SHAPES = [(1, 8, 16), (17, 8, 16), (256, 256, 128), (300, 264, 208), (257, 520, 400),
          (3120, 512, 4096), (129, 1024, 16384), (64, 2048, 4096),
          (448, 256, 64), (225, 520, 192),   # one K stage; 224-row tiles exact / one row over
          (2900, 4104, 128),   # 221 tiles, ragged in both directions, over the XCD tile groups
          (300, 264, 256), (257, 520, 384),   # two and three 128-byte K stages
          (700, 1000, 640)]   # five stages, ragged: a one-round grid's three-slot B ring


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("with_bias", [True, False])
def test_fp8_scaled_mm_matches_oracle(dev, M, N, K, dtype, with_bias):
    import joyomni_ops as jo
    a, w, sa, sb, bias = operands(M, N, K, M + N + K, dtype, with_bias)
    mat_b = w.to(dev).t()                      # [K, N] column-major, as Fp8Linear stores it
    out = jo.fp8_scaled_mm(a.to(dev), mat_b, sa.to(dev), sb.to(dev), dtype,
                           bias.to(dev) if with_bias else None)
    torch.cuda.synchronize()
    assert out.shape == (M, N) and out.dtype == dtype
    check(out, a, w.t(), sa, sb, bias, f"[{M},{N},{K}] {dtype} bias={with_bias}")


def test_fp8_scaled_mm_strided_operands(abi, dev, stream_handle):
    """A and B^T rows padded (lda, ldb > K), an output row stride > N, scales
    given as [M, 1] (Fp8Linear's x_scale)."""
    M, N, K = 200, 136, 320
    a, w, sa, sb, bias = operands(M, N, K, 5)
    ap = torch.zeros(M, K + 48, dtype=torch.uint8)
    ap[:, :K] = a.view(torch.uint8)
    wp = torch.zeros(N, K + 32, dtype=torch.uint8)
    wp[:, :K] = w.view(torch.uint8)
    apd, wpd = ap.to(dev), wp.to(dev)
    out = torch.full((M, N + 24), 7.0, dtype=torch.bfloat16, device=dev)
    sad, sbd, bd = sa.reshape(M, 1).to(dev), sb.to(dev), bias.to(dev)
    abi.call("jo_fp8_scaled_mm", apd.data_ptr(), K + 48, wpd.data_ptr(), K + 32, sad.data_ptr(),
             sbd.data_ptr(), bd.data_ptr(), out.data_ptr(), N + 24, M, N, K,
             abi.dtype_code(torch.bfloat16), stream_handle)
    torch.cuda.synchronize()
    assert (out.cpu()[:, N:] == 7.0).all(), "columns beyond N written"
    check(out[:, :N], a, w.t(), sa, sb, bias, "strided")


def test_fp8_scaled_mm_huge_row_stride(abi, dev, stream_handle):
    """A row stride of 17 MiB: 255 rows of it overflow the 32-bit lane offsets
    of the LDS-pipelined kernels, so the launch must take the 64-bit-addressed
    kernel (a wrapped offset would read other rows and fail the check)."""
    M, N, K = 257, 16, 64
    lda = (1 << 24) + (1 << 20)
    a, w, sa, sb, bias = operands(M, N, K, 9)
    abuf = torch.empty(M * lda, dtype=torch.uint8, device=dev)
    abuf.as_strided((M, K), (lda, 1)).copy_(a.view(torch.uint8).to(dev))
    wd = w.view(torch.uint8).to(dev)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    sad, sbd, bd = sa.to(dev), sb.to(dev), bias.to(dev)
    abi.call("jo_fp8_scaled_mm", abuf.data_ptr(), lda, wd.data_ptr(), K, sad.data_ptr(),
             sbd.data_ptr(), bd.data_ptr(), out.data_ptr(), N, M, N, K,
             abi.dtype_code(torch.bfloat16), stream_handle)
    torch.cuda.synchronize()
    del abuf
    check(out, a, w.t(), sa, sb, bias, "17 MiB row stride")


@pytest.mark.parametrize("N,K", [(12288, 4096), (16384, 4096), (4096, 16384)])
def test_fp8_scaled_mm_deployment_shapes_sampled_rows(dev, N, K):
    """M = 3120 tokens (720x1248 image stream); 40 sampled rows, the ragged
    last row tile included, against the exact oracle."""
    import joyomni_ops as jo
    M = 3120
    a, w, sa, sb, bias = operands(M, N, K, N + K)
    out = jo.fp8_scaled_mm(a.to(dev), w.to(dev).t(), sa.to(dev), sb.to(dev), torch.bfloat16,
                           bias.to(dev))
    torch.cuda.synchronize()
    g = torch.Generator().manual_seed(1)
    rows = torch.cat([torch.randperm(3072, generator=g)[:24], torch.arange(3104, 3120)])
    check(out.cpu()[rows], a, w.t(), sa, sb, bias, f"[{M},{N},{K}] sampled", rows=rows)


_TEXT_ORACLE = {}


@pytest.mark.parametrize("M,N,K", [(77, 12288, 4096), (100, 12288, 4096), (200, 12288, 4096),
                                   (256, 4096, 16384), (512, 16384, 4096), (1000, 4096, 4096)])
def test_fp8_scaled_mm_text_stream_shapes(dev, M, N, K):
    """The text stream's Fp8Linear shapes (a few hundred prompt tokens against
    the hidden 4096 / MLP 16384 weights), where the automatic choice takes the
    small-tile kernel (64x64, 128x128, 64x96 and 128x96 on the qkv projection's
    12288 columns with a ragged last row of tiles, or, at 512 x 16384, 128x256);
    every output against the exact oracle (computed once per shape, reused
    under every launch shape)."""
    import joyomni_ops as jo
    a, w, sa, sb, bias = operands(M, N, K, M * 7 + K)
    out = jo.fp8_scaled_mm(a.to(dev), w.to(dev).t(), sa.to(dev), sb.to(dev), torch.bfloat16,
                           bias.to(dev))
    torch.cuda.synchronize()
    key = (M, N, K)
    if key not in _TEXT_ORACLE:
        _, acc, mag = ops.fp8_scaled_mm(a, w.t(), sa, sb, torch.bfloat16, bias)
        ref = acc * sa.double().reshape(-1, 1) * sb.double().reshape(1, -1) + bias.double().reshape(1, -1)
        _TEXT_ORACLE[key] = (ref, ulp(ref, torch.bfloat16) + mag * 2.0 ** -13)
    ref, tol = _TEXT_ORACLE[key]
    err = (out.cpu().double() - ref).abs()
    bad = (err > tol).nonzero()
    assert bad.numel() == 0, f"[{M},{N},{K}]: {bad.shape[0]} outputs off, first {bad[0].tolist()}"


@pytest.mark.parametrize("split", [2, 4, 8])
@pytest.mark.parametrize("M,N,K", [(100, 520, 1024), (257, 264, 2048), (64, 4096, 8192)])
def test_fp8_scaled_mm_split_k(dev, split, M, N, K):
    """K split over `split` workgroups per tile (fp32 partials in the op's
    workspace, added in a fixed order by the second kernel): taken under the
    forced 128x128 and 64x64 shapes, the others ignore it. Against the exact
    oracle, and bit-identical on a second call."""
    import joyomni_ops as jo
    from joyomni_ops import _abi
    a, w, sa, sb, bias = operands(M, N, K, M + N + K + split)
    args = (a.to(dev), w.to(dev).t(), sa.to(dev), sb.to(dev), torch.bfloat16, bias.to(dev))
    _abi.call("jo_set_launch_override", _abi.JO_KNOB_GEMM_SPLIT, split)
    try:
        out = jo.fp8_scaled_mm(*args)
        again = jo.fp8_scaled_mm(*args)
        torch.cuda.synchronize()
    finally:
        _abi.call("jo_set_launch_override", _abi.JO_KNOB_GEMM_SPLIT, -1)
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))
    check(out, a, w.t(), sa, sb, bias, f"[{M},{N},{K}] split {split}")


def test_fp8_scaled_mm_ws_small_workspace_runs_unsplit(abi, dev, stream_handle):
    """jo_fp8_scaled_mm_ws with less workspace than the split needs (or none)
    runs as jo_fp8_scaled_mm: the same bits."""
    M, N, K = 256, 4096, 16384
    need = abi.lib().jo_fp8_scaled_mm_workspace_bytes(M, N, K)
    a, w, sa, sb, bias = operands(M, N, K, 77)
    ad, wd = a.view(torch.uint8).to(dev), w.view(torch.uint8).to(dev)
    sad, sbd, bd = sa.to(dev), sb.to(dev), bias.to(dev)
    outs = []
    sizes = (0, need - 16, need) if need > 0 else (0, 0, 0)   # forced shapes never split
    for ws_bytes in sizes:
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        abi.call("jo_fp8_scaled_mm_ws", ad.data_ptr(), K, wd.data_ptr(), K, sad.data_ptr(),
                 sbd.data_ptr(), bd.data_ptr(), out.data_ptr(), N, M, N, K,
                 abi.dtype_code(torch.bfloat16), ws.data_ptr() if ws_bytes else None, ws_bytes,
                 stream_handle)
        torch.cuda.synchronize()
        outs.append(out.cpu())
    plain = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    abi.call("jo_fp8_scaled_mm", ad.data_ptr(), K, wd.data_ptr(), K, sad.data_ptr(),
             sbd.data_ptr(), bd.data_ptr(), plain.data_ptr(), N, M, N, K,
             abi.dtype_code(torch.bfloat16), stream_handle)
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int16), plain.cpu().view(torch.int16))
    assert torch.equal(outs[1].view(torch.int16), plain.cpu().view(torch.int16))
    check(outs[2], a, w.t(), sa, sb, bias, "split with the full workspace")


def test_fp8_linear_reference_bench_shape(dev):
    """The reference benchmark's FP8 linear (test_bench.py:160-200): x [4096, 4096]
    bf16 through Fp8Linear's per-token quantization and the GEMM with a
    per-channel quantized [4096, 4096] weight. Sampled rows against the exact
    oracle of the quantized operands; and, as the reference reports it, the
    error against the unquantized product (fp8 e4m3 operands: a few percent)."""
    from joyomni_ops import dit_ops
    g = torch.Generator().manual_seed(4096)
    M = N = K = 4096
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    wq, ws = dit_ops.quantize_weight_per_channel(w.to(dev))
    y = dit_ops.fp8_linear(x.to(dev), wq, ws)
    torch.cuda.synchronize()
    rows = torch.cat([torch.randperm(M, generator=g)[:24], torch.arange(M - 8, M)])
    xq, xs = ops.per_token_quant_fp8(x[rows])
    check(y.cpu()[rows], xq.view(torch.float8_e4m3fn), wq.cpu(), xs, ws.cpu(), None,
          "fp8_linear 4096^3 sampled")
    exact = x[rows].double() @ w.double().t()
    rel = ((y.cpu()[rows].double() - exact).norm() / exact.norm()).item()
    assert rel < 0.08, rel


def test_fp8_linear_shim_and_rejects(dev):
    """dit_ops.fp8_linear == per-token quantization + GEMM (Fp8Linear.forward),
    with the weight prepared like Fp8Linear.from_linear; reference errors."""
    import joyomni_ops as jo
    from joyomni_ops import dit_ops
    g = torch.Generator().manual_seed(3)
    B, L, K, N = 2, 96, 512, 384
    x = torch.randn(B, L, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    wq, ws = dit_ops.quantize_weight_per_channel(w.to(dev))
    assert wq.shape == (K, N) and wq.stride() == (1, K)
    y = dit_ops.fp8_linear(x.to(dev), wq, ws, bias.to(dev))
    torch.cuda.synchronize()
    xq, xs = ops.per_token_quant_fp8(x.reshape(-1, K))
    check(y.reshape(-1, N), xq.view(torch.float8_e4m3fn), wq.cpu(), xs, ws.cpu(), bias, "fp8_linear")
    a = torch.zeros(4, 32, dtype=torch.float8_e4m3fn, device=dev)
    s4, s8 = torch.ones(4, device=dev), torch.ones(8, device=dev)
    with pytest.raises(RuntimeError, match="column major"):
        jo.fp8_scaled_mm(a, torch.zeros(32, 8, dtype=torch.float8_e4m3fn, device=dev), s4, s8,
                         torch.bfloat16)
    with pytest.raises(RuntimeError, match="out_dtype must be Half or BFloat16"):
        jo.fp8_scaled_mm(a, torch.zeros(8, 32, dtype=torch.float8_e4m3fn, device=dev).t(), s4, s8,
                         torch.float32)
