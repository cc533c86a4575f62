"""Build the C part of the oracle (TEST INFRASTRUCTURE): oracle/_build/libfp8ref.so.

The reference's own kernels are CUDA and cannot be compiled in this image
(no nvcc), so there is no oracle/_ref build. The reference ships no golden
vectors or known-answer tests for this path either, so the restatement in
oracle/ is pinned by independent checks (tests/test_oracle.py): a brute-force
e4m3fn encoder, hand-derived known-answer rows, library routines
(F.layer_norm, F.rms_norm, complex multiplication), float64 closed forms,
invariants, and planted mistakes that must be caught.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

ORACLE = Path(__file__).resolve().parent
BUILD = ORACLE / "_build"
LIB = BUILD / "libfp8ref.so"


def build() -> Path:
    BUILD.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    subprocess.run(
        ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
         "-Wall", "-o", str(tmp), str(ORACLE / "fp8_ref.c"), "-lm"],
        check=True)
    tmp.replace(LIB)
    return LIB


if __name__ == "__main__":
    print(build())
