"""Build the gfx950 kernel library and the torch op shim in-tree.

Outputs (next to the Python package, so they travel with the source tree):
  joyomni_ops/libjoyomni_hip.so     HIP kernels + the C ABI of include/joyomni_hip.h
  joyomni_ops/_C.so                 TORCH_LIBRARY(joyomni_ops) registration over the C ABI
  joyomni_ops/libjoyomni_stream.so  bare row streams that bench.py times as the
                                    HBM ceiling of each kernel's access shape
                                    (csrc/bench/; not part of the op library)

The library is compiled with hipcc for gfx950 only. The shim is plain C++
compiled with g++ against torch's ROCm headers; it holds no device code.

Usage:  python joyai-video-edit_amd/build.py [--jobs N] [--only lib|shim]
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent          # joyai-video-edit_amd/
REPO_ROOT = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
OUT_DIR = PKG_ROOT / "joyomni_ops"
BUILD_DIR = PKG_ROOT / "_build"
INCLUDE = REPO_ROOT / "include"

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = "gfx950"

LIB_NAME = "libjoyomni_hip.so"
SHIM_NAME = "_C.so"
STREAM_NAME = "libjoyomni_stream.so"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed fp32 VALU forms are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # The first 16 kernel-argument dwords arrive in SGPRs at wave launch (gfx950
    # kernarg preload), so a row kernel's first loads do not wait on an s_load of
    # its argument struct: 1-3 % on the RMSNorm->FP8 kernels, level elsewhere.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout)
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}")
    out = "\n".join(
        ln for ln in res.stdout.splitlines()
        if "packed-fp32-ops" not in ln and ln.strip() and "warning generated" not in ln
    )
    if out:
        sys.stderr.write(out + "\n")


def hip_sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build_lib(jobs: int) -> Path:
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    objs = []
    cmds = []
    for src in hip_sources():
        obj = BUILD_DIR / (src.stem + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)])
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(_run, cmds))
    out = OUT_DIR / LIB_NAME
    tmp = out.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          *map(str, objs), f"-Wl,-soname,{LIB_NAME}"])
    os.replace(tmp, out)
    return out


def build_stream() -> Path:
    out = OUT_DIR / STREAM_NAME
    tmp = out.with_suffix(".so.tmp")
    _run([HIPCC, *HIP_FLAGS, "-shared", str(CSRC / "bench" / "stream_ceiling.hip"), "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build_shim() -> Path:
    import torch
    from torch.utils import cpp_extension

    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    py_inc = sysconfig.get_paths()["include"]
    out = OUT_DIR / SHIM_NAME
    tmp = out.with_suffix(".so.tmp")
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        "-DTORCH_EXTENSION_NAME=_C",
        *[f"-I{p}" for p in cpp_extension.include_paths()],
        f"-I{py_inc}", f"-I{ROCM / 'include'}", f"-I{INCLUDE}",
        str(CSRC / "torch_shim.cpp"),
        "-o", str(tmp),
        f"-L{torch_lib}", f"-L{OUT_DIR}",
        "-l:" + LIB_NAME,
        "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
        f"-L{ROCM / 'lib'}", "-lamdhip64",
        "-Wl,-rpath,$ORIGIN",
        f"-Wl,-rpath,{torch_lib}",
    ]
    _run(cmd)
    os.replace(tmp, out)
    return out


def build(jobs: int | None = None, only: str | None = None) -> None:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    jobs = jobs or min(8, os.cpu_count() or 1)
    if only in (None, "lib"):
        build_lib(jobs)
        build_stream()
    if only in (None, "shim"):
        if (CSRC / "torch_shim.cpp").exists():
            build_shim()


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--only", choices=["lib", "shim"], default=None)
    args = ap.parse_args()
    build(args.jobs, args.only)
    print("built", OUT_DIR / LIB_NAME, "and", OUT_DIR / SHIM_NAME)


if __name__ == "__main__":
    main()
