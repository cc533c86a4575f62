"""ctypes binding of the C ABI declared in include/joyomni_hip.h.

This is the reference-side binding a Python host would add for the C ABI
(the torch op shim `_C.so` is the other one). `lib()` loads
libjoyomni_hip.so from this package directory; every entry point returns a
status code and `check()` turns a non-zero status into a RuntimeError
carrying jo_last_error().
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_char_p, c_float, c_int, c_int32, c_int64, c_void_p

LIB_NAME = "libjoyomni_hip.so"

# The header's JO_ABI_VERSION this binding's SIGNATURES follow; a library
# reporting another version is refused at load.
JO_ABI_VERSION = 4

JO_OK = 0
JO_ERR_INVALID = 1
JO_ERR_UNSUPPORTED = 2
JO_ERR_HIP = 3

JO_DTYPE_F32 = 0
JO_DTYPE_F16 = 1
JO_DTYPE_BF16 = 2

JO_NORM_LAYER = 0
JO_NORM_RMS = 1

JO_KNOB_QK_SPLIT = 0
JO_KNOB_KV_SPLIT = 1
JO_KNOB_GEMM_SHAPE = 2
JO_KNOB_GEMM_SPLIT = 3

_P = c_void_p
_I64 = c_int64
_F = c_float

# Entry points that return something other than an int status.
RESTYPES = {"jo_fp8_scaled_mm_workspace_bytes": _I64}

# name -> argument types, in header order.
SIGNATURES: dict[str, list] = {
    "jo_set_launch_override": [c_int, c_int],
    "jo_sgl_per_token_quant_fp8": [_P, c_int, _I64, _I64, _I64, _P, _I64, _P, _P],
    "jo_gelu_tanh_quant_fp8": [_P, c_int, _I64, _I64, _I64, _P, _I64, _P, _P, _I64, _P],
    "jo_fused_qk_norm_rope_3d_paired": [
        _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P, _P, _P, _P, _P],
    "jo_fused_qk_norm_rope_3d_grid": [
        _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P, _P, _P,
        c_int32, c_int32, c_int32, c_int32, c_int32, _F, _P],
    "jo_fused_qk_norm_rope_3d_paired_kstage": [
        _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P, _P, _P,
        _P, _P],
    "jo_fused_qk_norm_rope_3d_grid_kstage": [
        _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P, _P, _P,
        c_int32, c_int32, c_int32, c_int32, c_int32, _F, _P],
    "jo_fused_qk_norm_rope_3d_kvcache": [
        _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
        _F, _P, _P, _P, c_int32, c_int32, c_int32, c_int32, c_int32, _F, _P],
    "jo_fused_norm_scale_shift": [
        _P, _I64, _P, _P, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, c_int, c_int, _F, _P],
    "jo_fused_norm_scale_shift_per_sample": [
        _P, _I64, _P, _P, _P, _I64, _P, _I64, _I64, _P, _I64, _I64, _I64, c_int, c_int, _F, _P],
    "jo_rmsnorm": [_P, _I64, _P, _P, _I64, _I64, _I64, c_int, _F, _P],
    "jo_rmsnorm_heads": [_P, _I64, _I64, _P, _P, _I64, _I64, _I64, _I64, c_int, _F, c_int, _P],
    "jo_fused_add_layernorm_scale_shift": [
        _P, _I64, _P, _I64, _P, _I64, _P, _P, _P, _I64, _P, _I64, _I64, _P, _I64, _I64, _I64,
        c_int, _F, _P],
    "jo_rmsnorm_quant_fp8": [_P, _I64, _P, _P, _I64, _P, _I64, _I64, c_int, _F, _I64, _P],
    "jo_norm_scale_shift_quant_fp8": [
        _P, _I64, _P, _I64, _P, _I64, _P, _P, _P, _I64, _P, _I64, _I64, _P, _I64, _P, _I64, _I64,
        c_int, c_int, _F, _P],
    "jo_fp8_scaled_mm": [_P, _I64, _P, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _I64, c_int, _P],
    "jo_fp8_scaled_mm_ws": [_P, _I64, _P, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _I64, c_int, _P,
                            _I64, _P],
    "jo_fp8_scaled_mm_workspace_bytes": [_I64, _I64, _I64],
    "jo_fp8_scaled_mm_noalloc": [_P, _I64, _P, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _I64, c_int,
                                 _P],
    "jo_kv_commit_rope": [
        _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
        _I64, _P, _P, _I64, _I64, c_int, _P],
}

_lib = None


def lib_path() -> str:
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)


def lib() -> ctypes.CDLL:
    """Load libjoyomni_hip.so (raises ImportError if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    path = lib_path()
    if not os.path.exists(path):
        raise ImportError(
            f"{LIB_NAME} not found at {path}; build it first "
            "(python joyai-video-edit_amd/build.py)")
    # torch's HIP runtime has the same SONAME as the one this library links;
    # importing torch first makes both share one runtime instance.
    import torch  # noqa: F401
    handle = ctypes.CDLL(path)
    handle.jo_last_error.restype = c_char_p
    handle.jo_last_error.argtypes = []
    handle.jo_abi_version.restype = c_int
    handle.jo_abi_version.argtypes = []
    found = handle.jo_abi_version()
    if found != JO_ABI_VERSION:
        raise ImportError(
            f"{path} has ABI version {found}, this binding expects {JO_ABI_VERSION}; "
            "rebuild it (python joyai-video-edit_amd/build.py)")
    for name, argtypes in SIGNATURES.items():
        fn = getattr(handle, name, None)
        if fn is None:  # reported by the export test; call() raises on use
            continue
        fn.restype = RESTYPES.get(name, c_int)
        fn.argtypes = argtypes
    _lib = handle
    return _lib


def last_error() -> str:
    return lib().jo_last_error().decode()


def check(status: int, op: str = "") -> None:
    if status != JO_OK:
        raise RuntimeError(f"{op or 'joyomni'}: status {status}: {last_error()}")


def call(name: str, *args) -> None:
    """Call entry point `name` and raise RuntimeError on a non-zero status."""
    check(getattr(lib(), name)(*args), name)


def dtype_code(dtype) -> int:
    import torch
    codes = {torch.float32: JO_DTYPE_F32, torch.float16: JO_DTYPE_F16,
             torch.bfloat16: JO_DTYPE_BF16}
    if dtype not in codes:
        raise TypeError(f"unsupported dtype {dtype}")
    return codes[dtype]
