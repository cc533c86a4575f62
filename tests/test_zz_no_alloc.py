"""The allocation-free FP8 GEMM entry point (jo_fp8_scaled_mm_noalloc)
against jo_fp8_scaled_mm_ws with a torch workspace of the size the library
asks for: the same plan, so the same bits; two calls in a row, the second
with a smaller input (the static scratch keeps the first call's partials,
which the second must not read); a shape whose partials exceed the static
scratch is refused before any launch."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

SCRATCH = 32 << 20


def operands(M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    a = (torch.randn(M, K, generator=g) * 4).to(torch.float8_e4m3fn)
    w = (torch.randn(N, K, generator=g) * 4).to(torch.float8_e4m3fn)
    sa = torch.rand(M, generator=g) * 0.02 + 1e-3
    sb = torch.rand(N, generator=g) * 0.02 + 1e-3
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    return a, w, sa, sb, bias


def test_noalloc_matches_workspace_entry_point(abi, dev, stream_handle):
    lib = abi.lib()
    bf = abi.dtype_code(torch.bfloat16)
    for M, N, K in [(256, 4096, 16384), (64, 1024, 8192)]:   # split plans, the second smaller
        need = lib.jo_fp8_scaled_mm_workspace_bytes(M, N, K)
        assert 0 < need <= SCRATCH, (M, N, K, need)
        a, w, sa, sb, bias = operands(M, N, K, M + N)
        ad, wd = a.view(torch.uint8).to(dev), w.view(torch.uint8).to(dev)
        sad, sbd, bd = sa.to(dev), sb.to(dev), bias.to(dev)
        got = torch.full((M, N), 3.0, dtype=torch.bfloat16, device=dev)
        print(f"noalloc [{M},{N}] x {K}: {need} bytes of scratch", flush=True)
        abi.call("jo_fp8_scaled_mm_noalloc", ad.data_ptr(), K, wd.data_ptr(), K, sad.data_ptr(),
                 sbd.data_ptr(), bd.data_ptr(), got.data_ptr(), N, M, N, K, bf, stream_handle)
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        want = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        abi.call("jo_fp8_scaled_mm_ws", ad.data_ptr(), K, wd.data_ptr(), K, sad.data_ptr(),
                 sbd.data_ptr(), bd.data_ptr(), want.data_ptr(), N, M, N, K, bf, ws.data_ptr(),
                 need, stream_handle)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu().view(torch.int16), want.cpu().view(torch.int16)), (M, N, K)
        assert want.abs().amax().item() > 0


def test_noalloc_unsplit_shape_and_refusal(abi, dev, stream_handle):
    """An image-stream shape needs no scratch (the plain kernels, no split);
    a forced split whose partials exceed the scratch is refused."""
    lib = abi.lib()
    bf = abi.dtype_code(torch.bfloat16)
    M, N, K = 448, 512, 1024
    assert lib.jo_fp8_scaled_mm_workspace_bytes(M, N, K) == 0
    a, w, sa, sb, bias = operands(M, N, K, 5)
    ad, wd = a.view(torch.uint8).to(dev), w.view(torch.uint8).to(dev)
    sad, sbd, bd = sa.to(dev), sb.to(dev), bias.to(dev)
    got = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    want = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    abi.call("jo_fp8_scaled_mm_noalloc", ad.data_ptr(), K, wd.data_ptr(), K, sad.data_ptr(),
             sbd.data_ptr(), bd.data_ptr(), got.data_ptr(), N, M, N, K, bf, stream_handle)
    abi.call("jo_fp8_scaled_mm", ad.data_ptr(), K, wd.data_ptr(), K, sad.data_ptr(),
             sbd.data_ptr(), bd.data_ptr(), want.data_ptr(), N, M, N, K, bf, stream_handle)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu().view(torch.int16), want.cpu().view(torch.int16))
    try:
        abi.call("jo_set_launch_override", abi.JO_KNOB_GEMM_SHAPE, 6)
        abi.call("jo_set_launch_override", abi.JO_KNOB_GEMM_SPLIT, 8)
        Mb, Nb, Kb = 1024, 4096, 1024                # 8 x 1024 x 4096 x 4 bytes = 128 MiB
        assert lib.jo_fp8_scaled_mm_workspace_bytes(Mb, Nb, Kb) == 8 * Mb * Nb * 4
        status = lib.jo_fp8_scaled_mm_noalloc(ad.data_ptr(), Kb, wd.data_ptr(), Kb,
                                              sad.data_ptr(), sbd.data_ptr(), bd.data_ptr(),
                                              got.data_ptr(), Nb, Mb, Nb, Kb, bf, stream_handle)
        assert status == abi.JO_ERR_INVALID
        assert "static scratch" in abi.last_error()
    finally:
        abi.call("jo_set_launch_override", abi.JO_KNOB_GEMM_SHAPE, -1)
        abi.call("jo_set_launch_override", abi.JO_KNOB_GEMM_SPLIT, -1)
