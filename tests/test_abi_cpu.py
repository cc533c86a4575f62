"""CPU tests of the boundary: the C ABI library loads and exports every entry
point of include/joyomni_hip.h, the ctypes binding matches the header, the
validation errors come back as status codes without touching a GPU, and the
torch op library registers the reference's schemas byte-for-byte."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "joyomni_hip.h"
PKG = ROOT / "joyai-video-edit_amd"


def header_functions() -> dict[str, int]:
    """name -> number of parameters, for every function declared in the header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:int|int64_t|const char\*)\s+(jo_\w+)\s*\(([^)]*)\)\s*;", text):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else len(params.split(","))
    return out


def test_header_declares_all_entry_points():
    fns = header_functions()
    for name in ("jo_last_error", "jo_abi_version", "jo_sgl_per_token_quant_fp8",
                 "jo_fused_qk_norm_rope_3d_paired", "jo_fused_qk_norm_rope_3d_grid",
                 "jo_fused_qk_norm_rope_3d_kvcache", "jo_fused_norm_scale_shift", "jo_rmsnorm",
                 "jo_fused_add_layernorm_scale_shift", "jo_rmsnorm_quant_fp8",
                 "jo_rmsnorm_heads", "jo_norm_scale_shift_quant_fp8", "jo_fp8_scaled_mm",
                 "jo_kv_commit_rope", "jo_fused_norm_scale_shift_per_sample",
                 "jo_fp8_scaled_mm_ws", "jo_fp8_scaled_mm_workspace_bytes"):
        assert name in fns, name


def test_library_exports_every_header_symbol(abi):
    lib = abi.lib()
    for name in header_functions():
        assert hasattr(lib, name), f"{name} not exported by {abi.lib_path()}"
    nm = subprocess.run(["nm", "-D", "--defined-only", abi.lib_path()], capture_output=True,
                        text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in nm.splitlines() if " T " in ln}
    assert set(header_functions()) <= exported


def test_ctypes_signatures_match_header(abi):
    fns = header_functions()
    for name, argtypes in abi.SIGNATURES.items():
        assert fns[name] == len(argtypes), name
    assert set(abi.SIGNATURES) == set(fns) - {"jo_last_error", "jo_abi_version"}


def test_abi_version(abi):
    assert abi.lib().jo_abi_version() == 4


# Launch-size bounds of the entry points (work items of one launch < 2^32).
QK_MAX_TOKENS = (2**32 - 1) // (8 * 64)
KV_MAX_ROWS = (2**32 - 1) // (2 * 64)
MAX_ROWS = (2**32 - 1) // 256

# Validation paths return before any HIP call, so they run without a GPU.
BAD_CALLS = [
    ("jo_sgl_per_token_quant_fp8", (8, 0, 4, 8, 8, 8, 8, 8, None), "bf16 or fp16"),
    ("jo_sgl_per_token_quant_fp8", (8, 2, 4, 6, 6, 8, 6, 8, None), "divisible by 4"),
    ("jo_sgl_per_token_quant_fp8", (None, 2, 4, 8, 8, 8, 8, 8, None), "null pointer"),
    ("jo_sgl_per_token_quant_fp8", (8, 2, 4, 8, 4, 8, 8, 8, None), "row stride"),
    ("jo_gelu_tanh_quant_fp8", (8, 0, 4, 8, 8, 8, 8, 8, None, 0, None), "bf16 or fp16"),
    ("jo_gelu_tanh_quant_fp8", (8, 2, 4, 6, 6, 8, 6, 8, None, 0, None), "divisible by 4"),
    ("jo_gelu_tanh_quant_fp8", (None, 2, 4, 8, 8, 8, 8, 8, None, 0, None), "null pointer"),
    ("jo_gelu_tanh_quant_fp8", (8, 2, 4, 8, 4, 8, 8, 8, None, 0, None), "row stride"),
    ("jo_gelu_tanh_quant_fp8", (8, 2, 4, 8, 8, 8, 8, 8, 8, 4, None), "activation row stride"),
    # input rows span bytes [4096, 4160): an activation at the same address or
    # starting inside that span is refused
    ("jo_gelu_tanh_quant_fp8", (4096, 2, 4, 8, 8, 8192, 8, 16384, 4096, 8, None),
     "must not overlap"),
    ("jo_gelu_tanh_quant_fp8", (4096, 2, 4, 8, 8, 8192, 8, 16384, 4158, 8, None),
     "must not overlap"),
    ("jo_gelu_tanh_quant_fp8", (4096, 2, 4, 8, 8, 8192, 8, 16384, 4040, 8, None),
     "must not overlap"),
    ("jo_fused_qk_norm_rope_3d_paired",
     (16, 16, 1, 4, 2, 96, 768, 192, 768, 192, 1e-6, 16, 16, 16, 16, None), "head_dim"),
    ("jo_fused_qk_norm_rope_3d_paired",
     (16, 16, 1, 4, 2, 128, 1024, 256, 1024, 256, 1e-6, 16, 16, None, 16, None), "cos/sin"),
    ("jo_fused_qk_norm_rope_3d_paired",
     (16, 16, 1, 4, 2, 128, 1024, 250, 1024, 256, 1e-6, 16, 16, 16, 16, None), "token stride"),
    ("jo_fused_qk_norm_rope_3d_grid",
     (16, 16, 1, 10, 2, 128, 2560, 256, 2560, 256, 1e-6, 16, 16, 16, 11, 21, 3, 3, 0, 0.0, None),
     "whole number"),
    ("jo_fused_qk_norm_rope_3d_grid",
     (16, 16, 1, 9, 2, 128, 2304, 256, 2304, 256, 1e-6, 16, 16, 16, 40, 30, 3, 3, 0, 0.0, None),
     "pairs_t"),
    ("jo_fused_qk_norm_rope_3d_kvcache",
     (16, 16, 16, 1, 9, 2, 128, 2304, 256, 2304, 256, 4608, 256, 1, 0, 1e-6, 16, 16, 16, 22, 21,
      3, 3, 0, 0.0, None), None),  # 1 frame, 1 slot: valid geometry, but null-free pointers -> ok check below
    ("jo_fused_qk_norm_rope_3d_kvcache",
     (16, 16, 16, 1, 18, 2, 128, 4608, 256, 4608, 256, 4608, 256, 1, 0, 1e-6, 16, 16, 16, 22, 21,
      3, 3, 0, 0.0, None), "more frames"),
    ("jo_fused_qk_norm_rope_3d_kvcache",
     (16, 16, 16, 1, 9, 2, 128, 2304, 256, 2304, 256, 4608, 256, 2, 2, 1e-6, 16, 16, 16, 22, 21,
      3, 3, 0, 0.0, None), "slot_start"),
    ("jo_fused_norm_scale_shift", (16, 8, None, None, 16, 8, 16, 8, 16, 8, 4, 8, 2, 2, 1e-6, None),
     "norm_type"),
    ("jo_fused_norm_scale_shift", (16, 6, None, None, 16, 6, 16, 6, 16, 6, 4, 6, 2, 0, 1e-6, None),
     "divisible by 4"),
    ("jo_fused_norm_scale_shift", (16, 8, None, None, 16, 8, 16, 8, 16, 8, 4, 8, 7, 0, 1e-6, None),
     "dtype"),
    ("jo_fused_norm_scale_shift_per_sample",
     (16, 8, None, None, 16, 8, 16, 8, 0, 16, 8, 4, 8, 2, 0, 1e-6, None), "mod_rows"),
    ("jo_fused_norm_scale_shift_per_sample",
     (16, 8, None, None, 16, 8, 16, 8, 2, 16, 8, 4, 8, 2, 2, 1e-6, None), "norm_type"),
    ("jo_fused_norm_scale_shift_per_sample",
     (None, 8, None, None, 16, 8, 16, 8, 2, 16, 8, 4, 8, 2, 0, 1e-6, None), "null pointer"),
    # launch-size bounds: a launch's work-item count must stay below 2^32 (up to 8 waves of
    # 64 lanes per QK token, 2 waves per KV-pool row, one 256-thread workgroup per row)
    ("jo_fused_qk_norm_rope_3d_paired",
     (16, 16, 2, 1 << 28, 2, 128, 256 << 28, 256, 256 << 28, 256, 1e-6, 16, 16, 16, 16, None),
     "shape too large"),
    ("jo_fused_qk_norm_rope_3d_paired",
     (16, 16, 1, QK_MAX_TOKENS + 1, 2, 128, 256 * (QK_MAX_TOKENS + 1), 256,
      256 * (QK_MAX_TOKENS + 1), 256, 1e-6, 16, 16, 16, 16, None), "shape too large"),
    ("jo_fused_qk_norm_rope_3d_paired",  # at the bound: passes the shape check, stops at the pointer
     (None, 16, 1, QK_MAX_TOKENS, 2, 128, 256 * QK_MAX_TOKENS, 256, 256 * QK_MAX_TOKENS, 256,
      1e-6, 16, 16, 16, 16, None), "null pointer"),
    ("jo_kv_commit_rope",
     (16, None, 16, None, 1, 1, KV_MAX_ROWS + 1, 2, 128, 256 * (KV_MAX_ROWS + 1),
      256 * (KV_MAX_ROWS + 1), 256, 256 * (KV_MAX_ROWS + 1), 256 * (KV_MAX_ROWS + 1), 256,
      KV_MAX_ROWS + 1, 0, 16, 16, 128, 0, 2, None), "too many rows"),
    ("jo_kv_commit_rope",
     (None, None, 16, None, 1, 1, KV_MAX_ROWS, 2, 128, 256 * KV_MAX_ROWS, 256 * KV_MAX_ROWS, 256,
      256 * KV_MAX_ROWS, 256 * KV_MAX_ROWS, 256, KV_MAX_ROWS, 0, 16, 16, 128, 0, 2, None),
     "null pointer"),
    ("jo_rmsnorm", (16, 8, 16, 16, 8, MAX_ROWS + 1, 8, 2, 1e-6, None), "bad shape"),
    ("jo_rmsnorm", (None, 8, 16, 16, 8, MAX_ROWS, 8, 2, 1e-6, None), "null pointer"),
    ("jo_sgl_per_token_quant_fp8", (16, 2, MAX_ROWS + 1, 8, 8, 16, 8, 16, None), "shape too large"),
    ("jo_gelu_tanh_quant_fp8", (16, 2, MAX_ROWS + 1, 8, 8, 16, 8, 16, None, 0, None),
     "shape too large"),
    ("jo_rmsnorm_quant_fp8", (16, 256, 16, 16, 256, 16, MAX_ROWS + 1, 256, 2, 1e-6, 0, None),
     "bad shape"),
    ("jo_rmsnorm_heads", (16, 1152, 128, 16, 16, 128, MAX_ROWS // 3 + 1, 3, 128, 2, 1e-6, 0, None),
     "bad shape"),
    # zero-width rows would leave scales with nothing to take them from
    ("jo_norm_scale_shift_quant_fp8",
     (16, 8, None, 8, None, 0, None, None, 16, 0, 16, 0, 1, 16, 8, 16, 4, 0, 2, 0, 1e-6, None),
     "bad shape"),
    ("jo_norm_scale_shift_quant_fp8",
     (16, 8, None, 8, None, 0, None, None, 16, 8, 16, 8, 0, 16, 8, 16, 4, 8, 2, 0, 1e-6, None),
     "mod_rows"),
    ("jo_fused_add_layernorm_scale_shift",
     (16, 8, 16, 8, None, 0, None, None, 16, 8, 16, 8, 0, 16, 8, 4, 8, 2, 1e-6, None),
     "mod_rows"),
    ("jo_rmsnorm", (16, 8, 16, None, 8, 4, 8, 2, 1e-6, None), "null pointer"),
    ("jo_rmsnorm_heads", (16, 1152, 128, 16, 16, 128, 4, 3, 128, 2, 1e-6, 2, None), "round_first"),
    ("jo_rmsnorm_heads", (16, 1152, 128, 16, 16, 128, 4, 0, 128, 2, 1e-6, 0, None), "bad shape"),
    ("jo_rmsnorm_heads", (16, 1152, 64, 16, 16, 128, 4, 3, 128, 2, 1e-6, 0, None), "bad strides"),
    ("jo_rmsnorm_heads", (16, 1152, 128, None, 16, 128, 4, 3, 128, 2, 1e-6, 1, None), "null pointer"),
    ("jo_rmsnorm_heads", (16, 1152, 128, 16, 16, 128, 4, 3, 128, 9, 1e-6, 1, None), "dtype"),
    ("jo_fused_add_layernorm_scale_shift",
     (16, 12, 16, 12, None, 0, None, None, 16, 0, 16, 0, 1, 16, 8, 4, 12, 2, 1e-6, None),
     "bad row stride"),
    ("jo_rmsnorm_quant_fp8", (16, 256, 16, 16, 256, 16, 4, 256, 2, 1e-6, 64, None), "group_size"),
    ("jo_rmsnorm_quant_fp8", (16, 200, 16, 16, 200, 16, 4, 200, 2, 1e-6, 128, None), "divisible by 128"),
    ("jo_rmsnorm_quant_fp8", (16, 256, 16, 16, 256, 16, 4, 256, 0, 1e-6, 0, None), "bf16 or fp16"),
]


@pytest.mark.parametrize("name,args,msg", [b for b in BAD_CALLS if b[2] is not None])
def test_validation_errors_without_gpu(abi, name, args, msg):
    status = getattr(abi.lib(), name)(*args)
    assert status == abi.JO_ERR_INVALID
    assert msg in abi.last_error()


def test_launch_override(abi):
    lib = abi.lib()
    accepted = {abi.JO_KNOB_QK_SPLIT: {1, 2, 4, 6, 8}, abi.JO_KNOB_KV_SPLIT: {1, 2},
                abi.JO_KNOB_GEMM_SHAPE: set(range(12)),
                abi.JO_KNOB_GEMM_SPLIT: {1, 2, 4, 8}}
    for knob, ok in accepted.items():
        for v in range(-3, 66):
            want = abi.JO_OK if (v == -1 or v in ok) else abi.JO_ERR_INVALID
            assert lib.jo_set_launch_override(knob, v) == want, (knob, v)
            if want != abi.JO_OK:
                assert "not one knob" in abi.last_error()
        assert lib.jo_set_launch_override(knob, -1) == abi.JO_OK
    assert lib.jo_set_launch_override(4, 1) == abi.JO_ERR_INVALID
    assert "unknown knob" in abi.last_error()


def test_gemm_workspace_bytes(abi):
    """The split-K workspace the FP8 GEMM asks for (a host computation, the
    same with or without a GPU: 256 CUs assumed when none is visible): none
    for the image stream's shapes, S x M x N x 4 bytes for few rows and a long
    K, and what a forced split asks for (taken only by the small tiles)."""
    lib = abi.lib()
    wb = lib.jo_fp8_scaled_mm_workspace_bytes
    for M, N, K in [(3120, 12288, 4096), (3120, 4096, 16384), (256, 12288, 4096),
                    (1024, 4096, 16384)]:
        assert wb(M, N, K) == 0, (M, N, K)
    assert wb(256, 4096, 16384) == 4 * 256 * 4096 * 4   # 128x128 tiles, K in four
    assert wb(64, 4096, 16384) == 4 * 64 * 4096 * 4     # 64x64 tiles, K in four
    assert wb(0, 4096, 4096) == 0 and wb(256, 4096, 0) == 0
    try:
        assert lib.jo_set_launch_override(abi.JO_KNOB_GEMM_SHAPE, 6) == abi.JO_OK
        assert lib.jo_set_launch_override(abi.JO_KNOB_GEMM_SPLIT, 8) == abi.JO_OK
        assert wb(100, 520, 1024) == 8 * 100 * 520 * 4
        assert wb(100, 520, 896) == 0          # K % (128 x 8) != 0: no split
        assert lib.jo_set_launch_override(abi.JO_KNOB_GEMM_SHAPE, 3) == abi.JO_OK
        assert wb(100, 520, 1024) == 0         # the 224-row tiles never split
    finally:
        lib.jo_set_launch_override(abi.JO_KNOB_GEMM_SHAPE, -1)
        lib.jo_set_launch_override(abi.JO_KNOB_GEMM_SPLIT, -1)


def test_launch_override_env_values_are_checked(tmp_path):
    """An environment override the knob does not accept is ignored with a
    message (a fresh process, since the variables are read at load)."""
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, %r)\n"
            "from joyomni_ops import _abi\n"
            "lib = _abi.lib()\n"
            "assert lib.jo_set_launch_override(_abi.JO_KNOB_QK_SPLIT, -1) == 0\n"
            "print('loaded')\n" % str(PKG))
    env = dict(os.environ, JO_QK_SPLIT="3", JO_KV_SPLIT="2", JO_GEMM_SHAPE="7x",
               JO_GEMM_SPLIT="3")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env,
                       timeout=300)
    assert r.returncode == 0 and "loaded" in r.stdout, r.stderr
    assert "ignoring JO_QK_SPLIT=3" in r.stderr and "ignoring JO_GEMM_SHAPE=7x" in r.stderr
    assert "ignoring JO_GEMM_SPLIT=3" in r.stderr
    assert "JO_KV_SPLIT" not in r.stderr


def test_empty_inputs_are_noops(abi):
    lib = abi.lib()
    # zero rows / zero tokens: valid, nothing to launch
    assert lib.jo_sgl_per_token_quant_fp8(None, 2, 0, 8, 8, None, 8, None, None) == abi.JO_OK
    assert lib.jo_gelu_tanh_quant_fp8(None, 2, 0, 8, 8, None, 8, None, None, 0, None) == abi.JO_OK
    assert lib.jo_rmsnorm(None, 8, None, None, 8, 0, 8, 2, 1e-6, None) == abi.JO_OK
    assert lib.jo_rmsnorm_heads(None, 1152, 128, None, None, 128, 0, 3, 128, 2, 1e-6, 1,
                                None) == abi.JO_OK
    assert lib.jo_fused_norm_scale_shift(None, 8, None, None, None, 0, None, 0, None, 8, 0, 8, 2,
                                         0, 1e-6, None) == abi.JO_OK
    assert lib.jo_fused_norm_scale_shift_per_sample(None, 8, None, None, None, 0, None, 0, 4,
                                                    None, 8, 0, 8, 2, 0, 1e-6, None) == abi.JO_OK
    assert lib.jo_fused_qk_norm_rope_3d_paired(None, None, 1, 0, 2, 128, 0, 256, 0, 256, 1e-6,
                                               None, None, None, None, None) == abi.JO_OK
    assert lib.jo_fused_add_layernorm_scale_shift(None, 8, None, 8, None, 0, None, None, None, 0,
                                                  None, 0, 1, None, 8, 0, 8, 2, 1e-6,
                                                  None) == abi.JO_OK
    assert lib.jo_rmsnorm_quant_fp8(None, 8, None, None, 8, None, 0, 8, 2, 1e-6, 0,
                                    None) == abi.JO_OK
    assert lib.jo_norm_scale_shift_quant_fp8(None, 8, None, 8, None, 0, None, None, None, 0, None,
                                             0, 1, None, 8, None, 0, 8, 2, 0, 1e-6,
                                             None) == abi.JO_OK
    assert lib.jo_fp8_scaled_mm(None, 16, None, 16, None, None, None, None, 8, 0, 8, 16, 2,
                                None) == abi.JO_OK
    assert lib.jo_kv_commit_rope(None, None, None, None, 1, 1, 0, 2, 128, 0, 0, 256, 0, 0, 256, 4,
                                 0, None, None, 128, 0, 2, None) == abi.JO_OK
    # the grid modes check their pointers first (the frequency table is always read), then
    # return at zero tokens; host addresses stand in, as nothing is dereferenced
    buf = ctypes.create_string_buffer(64)
    p = ctypes.addressof(buf)
    assert lib.jo_fused_qk_norm_rope_3d_grid(p, p, 1, 0, 2, 128, 0, 256, 0, 256, 1e-6, p, p, p,
                                             22, 21, 4, 4, 0, 0.0, None) == abi.JO_OK
    assert lib.jo_fused_qk_norm_rope_3d_kvcache(p, p, p, 1, 0, 2, 128, 0, 256, 0, 256, 0, 256, 2,
                                                0, 1e-6, p, p, p, 22, 21, 4, 4, 0, 0.0,
                                                None) == abi.JO_OK


REFERENCE_SCHEMAS = {
    # deploy/joyomni_ops/csrc/pybind.cpp:35-43, verbatim.
    "fused_qk_norm_rope_3d_paired":
        "fused_qk_norm_rope_3d_paired(Tensor! q, Tensor! k, int seq_len, int num_heads, float eps, "
        "Tensor q_weight, Tensor k_weight, Tensor cos, Tensor sin) -> ()",
    "fused_norm_scale_shift":
        "fused_norm_scale_shift(Tensor x, Tensor? gamma_opt, Tensor? beta_opt, "
        "Tensor scale, Tensor shift, int norm_type, float eps) -> Tensor",
    "rmsnorm": "rmsnorm(Tensor x, Tensor weight, float eps) -> Tensor",
    "sgl_per_token_quant_fp8":
        "sgl_per_token_quant_fp8(Tensor input, Tensor! output_q, Tensor! output_s) -> ()",
    # pybind.cpp:44-46
    "fp8_scaled_mm":
        "fp8_scaled_mm(Tensor mat_a, Tensor mat_b, Tensor scales_a, Tensor scales_b, "
        "ScalarType out_dtype, Tensor? bias) -> Tensor",
}


def test_torch_ops_register_reference_schemas():
    import joyomni_ops as jo  # noqa: F401  (loads _C.so)
    for name, schema in REFERENCE_SCHEMAS.items():
        expected = torch._C.parse_schema("joyomni_ops::" + schema)
        assert getattr(torch.ops.joyomni_ops, name).default._schema == expected, name
    for name in ("fused_qk_norm_rope_3d_grid", "fused_qk_norm_rope_3d_kvcache",
                 "fused_add_layernorm_scale_shift", "rmsnorm_quant_fp8",
                 "norm_scale_shift_quant_fp8", "kv_commit_rope", "apply_rotary_emb",
                 "fused_norm_scale_shift_per_sample"):
        assert hasattr(torch.ops.joyomni_ops, name)
    assert jo.has_fp8()


def test_ops_have_no_cpu_kernel():
    """The product has no CPU path: CPU tensors are rejected by the dispatcher."""
    import joyomni_ops as jo
    x = torch.randn(4, 8, dtype=torch.bfloat16)
    with pytest.raises((NotImplementedError, RuntimeError)):
        jo.rmsnorm(x, torch.ones(8, dtype=torch.bfloat16))
    with pytest.raises((NotImplementedError, RuntimeError)):
        jo.sgl_per_token_quant_fp8(x, torch.empty(4, 8, dtype=torch.float8_e4m3fn),
                                   torch.empty(4))


def test_wrapper_norm_type_mapping_matches_reference():
    """'layer'->0, 'rms'->1, anything else -> -1 (rejected), __init__.py:38-41."""
    import inspect

    import joyomni_ops as jo
    src = inspect.getsource(jo.fused_norm_scale_shift)
    assert '0 if norm_type == "layer" else 1 if norm_type == "rms" else -1' in src
    sig = inspect.signature(jo.fused_norm_scale_shift)
    assert sig.parameters["eps"].default == 1e-5
    assert inspect.signature(jo.rmsnorm).parameters["eps"].default == 1e-6
