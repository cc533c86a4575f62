"""GPU parity of the FP8 quantization ops through the C ABI (and the torch op).

Bar: bit-exact e4m3fn bytes and bit-exact fp32 scales against the CPU oracle
(per_token_quant_fp8.cu:56-82 restated in oracle/ops.py, itself pinned by the
C brute-force encoder), on random rows with outliers, hand known-answer rows,
every row-shape dispatch class, strided and unaligned views, and the full C1
shape. RMSNorm->FP8 (C4, per token and per 1x128 block) is bit-exact too:
fp8 bytes and fp32 scales equal to the oracle's, whose mean square is the
exactly rounded mean of the exact squares, as the kernel's.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import kat
from oracle import fp8ref, ops
from joyomni_ops import workloads as W
from helpers import f32_ulp

pytestmark = pytest.mark.gpu


def quant_gpu(abi, stream, x_dev, M=None, K=None, in_stride=None):
    M = x_dev.shape[0] if M is None else M
    K = x_dev.shape[1] if K is None else K
    q = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=x_dev.device)
    s = torch.full((M,), -1.0, dtype=torch.float32, device=x_dev.device)
    abi.call("jo_sgl_per_token_quant_fp8", x_dev.data_ptr(), abi.dtype_code(x_dev.dtype), M, K,
             x_dev.stride(0) if in_stride is None else in_stride, q.data_ptr(), K, s.data_ptr(),
             stream)
    torch.cuda.synchronize()
    return q.view(torch.uint8).cpu(), s.cpu()


def assert_quant_equal(q, s, x_cpu, what):
    qo, so = ops.per_token_quant_fp8(x_cpu)
    nbad = int((q != qo).sum())
    assert nbad == 0, f"{what}: {nbad} fp8 bytes differ from the oracle"
    assert torch.equal(s, so) or bool(((s == so) | (torch.isinf(s) & torch.isinf(so))).all()), \
        f"{what}: scales differ"


SHAPES = [(1, 4), (3, 12), (7, 64), (33, 128), (5, 256), (9, 512), (17, 1000), (17, 3072),
          (64, 4096), (8191, 4096), (8192, 4096), (9, 8192), (3, 16384), (2, 32768), (2, 40000),
          (5, 100), (4, 1020), (1, 8)]   # 4096-wide rows: two waves per row below 8192 rows


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,K", SHAPES)
def test_quant_random_rows(abi, dev, stream_handle, dtype, M, K):
    g = torch.Generator().manual_seed(M * 100003 + K)
    x = W.with_outliers(torch.randn(M, K, generator=g), g).to(dtype)
    q, s = quant_gpu(abi, stream_handle, x.to(dev))
    assert_quant_equal(q, s, x, f"{dtype} [{M},{K}]")


def test_quant_known_answer_rows(abi, dev, stream_handle):
    rows = [r for r, _, _ in kat.KAT_ROWS]
    x = torch.tensor(rows, dtype=torch.float32).to(torch.bfloat16)
    for width in (8, 64, 3072):  # replicate each row to hit several kernel shapes
        xr = x.repeat(1, width // 8)
        q, s = quant_gpu(abi, stream_handle, xr.to(dev))
        for i, (_, scale, codes) in enumerate(kat.KAT_ROWS):
            assert q[i].tolist() == codes * (width // 8), f"KAT row {i} width {width}"
            assert s[i].item() == np.float32(scale) or (np.isinf(scale) and np.isinf(s[i].item()))


def inject_nonfinite(x: torch.Tensor, seed: int) -> torch.Tensor:
    """Rows 1, 5, 9, ... get a NaN, rows 2, 6, ... an inf, rows 3, 7, ... a -inf,
    every 4th row is scaled to 2^-127 (1/scale overflows); row 0 stays finite."""
    x = x.clone().float()
    g = torch.Generator().manual_seed(seed)
    M, N = x.shape
    for r in range(1, M):
        j = int(torch.randint(0, N, (1,), generator=g))
        kind = r % 4
        if kind == 1:
            x[r, j] = float("nan")
        elif kind == 2:
            x[r, j] = float("inf")
        elif kind == 3:
            x[r, j] = float("-inf")
        else:
            x[r] = torch.sign(x[r]) * 2.0 ** -127
    return x


@pytest.mark.parametrize("N", [64, 3072, 4096, 16384])
def test_quant_nonfinite_rows(abi, dev, stream_handle, N):
    """Rows with NaN/inf and rows whose inverse scale overflows take the
    clamped path; finite rows sharing their workgroup must be unaffected."""
    g = torch.Generator().manual_seed(N)
    x = inject_nonfinite(torch.randn(13, N, generator=g), N).to(torch.bfloat16)
    q, s = quant_gpu(abi, stream_handle, x.to(dev))
    assert_quant_equal(q, s, x, f"nonfinite [13,{N}]")


def test_quant_strided_and_unaligned_views(abi, dev, stream_handle):
    g = torch.Generator().manual_seed(11)
    big = W.with_outliers(torch.randn(40, 3200, generator=g), g).to(torch.bfloat16)
    bd = big.to(dev)
    # row-strided view (16-byte aligned rows): vector path
    q, s = quant_gpu(abi, stream_handle, bd[:, :3072])
    assert_quant_equal(q, s, big[:, :3072], "strided")
    # view starting 1 element in: unaligned, generic path
    q, s = quant_gpu(abi, stream_handle, bd[:, 1:1 + 3072])
    assert_quant_equal(q, s, big[:, 1:1 + 3072], "unaligned")


def test_quant_full_c1(abi, dev, stream_handle):
    cfg = W.CONFIGS["C1"]
    x = W.make_inputs(cfg)["x"]
    q, s = quant_gpu(abi, stream_handle, x.to(dev))
    assert_quant_equal(q, s, x, "C1 [10530,3072]")
    # cross-check with the C restatement as well
    qc, sc = fp8ref.per_token_quant(x[:512].float().numpy())
    assert (q[:512].numpy() == qc).all() and (s[:512].numpy() == sc).all()


def test_quant_torch_op_matches_abi(dev):
    import joyomni_ops as jo
    g = torch.Generator().manual_seed(12)
    x = W.with_outliers(torch.randn(300, 4096, generator=g), g).to(torch.bfloat16)
    xq = torch.empty(300, 4096, dtype=torch.float8_e4m3fn, device=dev)
    xs = torch.empty(300, 1, dtype=torch.float32, device=dev)  # Fp8Linear's [M, 1] scales
    jo.sgl_per_token_quant_fp8(x.to(dev), xq, xs)
    torch.cuda.synchronize()
    assert_quant_equal(xq.view(torch.uint8).cpu(), xs.view(-1).cpu(), x, "torch op")
    with pytest.raises(RuntimeError):
        jo.sgl_per_token_quant_fp8(x.to(dev), torch.empty(300, 4096, dtype=torch.uint8, device=dev), xs)


# ---------------------------------------------------------------------------
# RMSNorm -> FP8
# ---------------------------------------------------------------------------
def rms_quant_gpu(abi, stream, x_dev, w_dev, eps, group):
    M, N = x_dev.shape
    q = torch.empty(M, N, dtype=torch.float8_e4m3fn, device=x_dev.device)
    s = torch.empty((M,) if group == 0 else (M, N // group), dtype=torch.float32,
                    device=x_dev.device)
    abi.call("jo_rmsnorm_quant_fp8", x_dev.data_ptr(), x_dev.stride(0), w_dev.data_ptr(),
             q.data_ptr(), N, s.data_ptr(), M, N, abi.dtype_code(x_dev.dtype), eps, group, stream)
    torch.cuda.synchronize()
    return q.view(torch.uint8).cpu(), s.cpu()


def check_rms_quant(q, s, x, w, eps, group, what):
    """Scales and e4m3fn bytes bit-exact against the oracle (the kernels' fixed
    fp32 summation order of the squares, IEEE sqrt/div, (x*r)*w, then the
    per_token_quant_fp8 rule per row/block)."""
    qo, so, _ = ops.rmsnorm_quant_fp8(x, w, eps, group)
    ds = (s - so).abs()
    assert torch.equal(s, so), \
        f"{what}: {int((s != so).sum())} scales differ, max {float((ds / f32_ulp(so)).max())} ulp"
    n = int((q != qo).sum())
    assert n == 0, f"{what}: {n} fp8 bytes differ"


@pytest.mark.parametrize("group", [0, 128])
@pytest.mark.parametrize("M,N", [(1, 128), (7, 256), (33, 1024), (17, 3072), (5, 4096),
                                 (3, 16384), (2, 24576),
                                 # one-wave rows that do not fill the last chunk
                                 # (lane masks; the LDS-shared weight row below
                                 # 8192 rows, x kept in fp32 above), and a row
                                 # width that is not a whole number of blocks
                                 (9, 2688), (9, 2176), (8200, 2688), (9, 2696)])
def test_rmsnorm_quant_random(abi, dev, stream_handle, group, M, N):
    g = torch.Generator().manual_seed(M * 7 + N + group)
    if group and N % group:
        # per-block scales need whole blocks: refused before any launch
        x = torch.zeros(M, N, dtype=torch.bfloat16, device=dev)
        q = torch.empty(M, N, dtype=torch.uint8, device=dev)
        s = torch.empty(M * (N // group + 1), dtype=torch.float32, device=dev)
        st = abi.lib().jo_rmsnorm_quant_fp8(x.data_ptr(), N, x.data_ptr(), q.data_ptr(), N,
                                            s.data_ptr(), M, N, abi.JO_DTYPE_BF16, 1e-6, group,
                                            stream_handle)
        assert st == abi.JO_ERR_INVALID and "divisible by 128" in abi.last_error()
        return
    x = W.with_outliers(torch.randn(M, N, generator=g), g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(N, generator=g)).to(torch.bfloat16)
    q, s = rms_quant_gpu(abi, stream_handle, x.to(dev), w.to(dev), 1e-6, group)
    check_rms_quant(q, s, x, w, 1e-6, group, f"[{M},{N}] g{group}")


ROW_SHAPE_CASES = [(N, 0) for N in (8, 40, 64, 512, 1536, 2048, 6144, 8192, 32768)] + \
    [(N, 128) for N in (512, 1536, 2048, 6144, 8192, 32768)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("N,group", ROW_SHAPE_CASES)
def test_rmsnorm_quant_every_row_shape(abi, dev, stream_handle, dtype, N, group):
    """Every row shape of the fixed-order sum (8-, 16-, 32- and 64-lane rows
    with 1 to 16 chunks per lane, 256-lane rows of four waves), bf16 and fp16,
    a ragged row count: bit-exact against the oracle's restatement."""
    M = 11
    g = torch.Generator().manual_seed(N * 3 + group + (dtype == torch.float16))
    x = W.with_outliers(torch.randn(M, N, generator=g), g).to(dtype)
    w = (1 + 0.1 * torch.randn(N, generator=g)).to(dtype)
    q, s = rms_quant_gpu(abi, stream_handle, x.to(dev), w.to(dev), 1e-6, group)
    check_rms_quant(q, s, x, w, 1e-6, group, f"[{M},{N}] {dtype} g{group}")


@pytest.mark.parametrize("group", [0, 128])
@pytest.mark.parametrize("N", [128, 3072, 16384])
@pytest.mark.parametrize("where", ["x", "w"])
def test_rmsnorm_quant_nonfinite(abi, dev, stream_handle, group, N, where):
    """NaN/inf in a row, in the weight, or rows so small that 1/scale overflows."""
    g = torch.Generator().manual_seed(N + group)
    x = torch.randn(13, N, generator=g)
    w = 1 + 0.1 * torch.randn(N, generator=g)
    if where == "x":
        x = inject_nonfinite(x, N)
    else:
        w[N // 3] = float("nan")
        w[N // 2] = float("inf")
        x[5] = 2.0 ** -127
    x, w = x.to(torch.bfloat16), w.to(torch.bfloat16)
    q, s = rms_quant_gpu(abi, stream_handle, x.to(dev), w.to(dev), 1e-6, group)
    check_rms_quant(q, s, x, w, 1e-6, group, f"nonfinite {where} [13,{N}] g{group}")


def test_rmsnorm_quant_nonfinite_many_rows(abi, dev, stream_handle):
    """Per-token mode from 8192 rows on takes its non-finite decision per wave:
    NaN/inf rows and rows whose 1/scale overflows, spread over 8200 rows."""
    g = torch.Generator().manual_seed(8200)
    M, N = 8200, 3072
    x = torch.randn(M, N, generator=g)
    for r in (0, 4099, 8187):
        x[r:r + 13] = inject_nonfinite(x[r:r + 13].clone(), N)
    w = 1 + 0.1 * torch.randn(N, generator=g)
    x, w = x.to(torch.bfloat16), w.to(torch.bfloat16)
    q, s = rms_quant_gpu(abi, stream_handle, x.to(dev), w.to(dev), 1e-6, 0)
    check_rms_quant(q, s, x, w, 1e-6, 0, "nonfinite [8200,3072] per token")


@pytest.mark.parametrize("name", ["C4_4725_tok", "C4_4725_blk", "C4_10530_tok", "C4_10530_blk"])
def test_rmsnorm_quant_full_c4(abi, dev, stream_handle, name):
    cfg = W.CONFIGS[name]
    t = W.make_inputs(cfg)
    q, s = rms_quant_gpu(abi, stream_handle, t["x"].to(dev), t["weight"].to(dev),
                         cfg.dims["eps"], cfg.dims["group"])
    check_rms_quant(q, s, t["x"], t["weight"], cfg.dims["eps"], cfg.dims["group"], name)


def test_rmsnorm_quant_torch_op(dev):
    import joyomni_ops as jo
    g = torch.Generator().manual_seed(13)
    x = torch.randn(64, 3072, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(3072, generator=g)).to(torch.bfloat16)
    q = torch.empty(64, 3072, dtype=torch.float8_e4m3fn, device=dev)
    s = torch.empty(64, 24, dtype=torch.float32, device=dev)
    jo.rmsnorm_quant_fp8(x.to(dev), w.to(dev), 1e-6, q, s, 128)
    torch.cuda.synchronize()
    check_rms_quant(q.view(torch.uint8).cpu(), s.cpu(), x, w, 1e-6, 128, "torch op")
