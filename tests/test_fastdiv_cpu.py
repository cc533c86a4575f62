"""CPU test of the multiply-high division (FastDiv / make_fastdiv / fdiv in
csrc/jo_device.hpp) that the QK, KV-commit and per-head RMSNorm kernels use for
their token / head / frame / slot index arithmetic.

A host-only program compiled from the same header checks fdiv(n, d) == n / d:
exhaustively over every 32-bit n for two divisors of the deployment shapes, and
for edge and random numerators over small, deployment-shape, power-of-two and
near-2^32 divisors; a planted slip (the final shift one too large) must be
caught. fdiv compiles to the same device code (v_mul_hi_u32) as the kernels use.
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "joyai-video-edit_amd" / "csrc"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

CHECK = r"""
#include <cstdio>
#include <cstdint>
#include <random>
#include "jo_device.hpp"

static int slip = 0;

static uint32_t div_under_test(uint32_t n, const jo::FastDiv& f) {
  jo::FastDiv g = f;
  g.s2 += slip;
  return jo::fdiv(n, g);
}

static long check(uint32_t n, uint32_t d, const jo::FastDiv& f) {
  if (div_under_test(n, f) != n / d) {
    if (!slip) std::printf("mismatch n=%u d=%u got=%u\n", n, d, div_under_test(n, f));
    return 1;
  }
  return 0;
}

int main(int argc, char** argv) {
  slip = argc > 1;
  long bad = 0;
  // every numerator for a grid-frame size and a token count of the deployment shapes
  if (!slip) {
    for (uint32_t d : {1560u, 4725u}) {
      const jo::FastDiv f = jo::make_fastdiv(d);
      uint32_t n = 0;
      do { bad += check(n, d, f); } while (++n != 0);
    }
  }
  std::mt19937_64 rng(7);
  std::vector<uint32_t> ds = {1u, 2u, 3u, 5u, 7u, 24u, 32u, 52u, 128u, 3120u, 10530u, 99840u,
                              (1u << 31) - 1, 1u << 31, (1u << 31) + 1, 0xFFFFFFFEu, 0xFFFFFFFFu};
  for (int k = 0; k < 32; ++k) ds.push_back(1u << k);
  for (int i = 0; i < 4000; ++i) {
    const int bits = 1 + static_cast<int>(rng() % 32);
    uint32_t d = static_cast<uint32_t>(rng() >> (64 - bits));
    ds.push_back(d ? d : 1u);
  }
  for (uint32_t d : ds) {
    const jo::FastDiv f = jo::make_fastdiv(d);
    const uint32_t edges[] = {0u, 1u, d - 1, d, d + 1, 2 * d - 1, 2 * d, 0xFFFFFFFFu, 0xFFFFFFFEu,
                              (0xFFFFFFFFu / d) * d, (0xFFFFFFFFu / d) * d - 1};
    for (uint32_t n : edges) bad += check(n, d, f);
    for (int i = 0; i < 2000; ++i) {
      bad += check(static_cast<uint32_t>(rng()), d, f);
      const uint64_t q = rng() % (0xFFFFFFFFull / d + 1);
      bad += check(static_cast<uint32_t>(q * d), d, f);
      if (q) bad += check(static_cast<uint32_t>(q * d - 1), d, f);
    }
  }
  std::printf("divisors %zu mismatches %ld\n", ds.size(), bad);
  return bad ? 1 : 0;
}
"""


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if not Path(HIPCC).exists():
        pytest.skip("hipcc not found")
    d = tmp_path_factory.mktemp("fastdiv")
    src = d / "fastdiv_check.hip"
    src.write_text(CHECK)
    exe = d / "fastdiv_check"
    r = subprocess.run([HIPCC, "-x", "hip", "--cuda-host-only", "-O2", "-std=c++17",
                        f"-I{ROOT / 'include'}", f"-I{CSRC}", str(src), "-o", str(exe)],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    return exe


def test_fdiv_equals_integer_division(checker):
    r = subprocess.run([str(checker)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-2000:]
    assert "mismatches 0" in r.stdout


def test_fdiv_check_catches_a_wrong_shift(checker):
    r = subprocess.run([str(checker), "slip"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 1 and "mismatches 0" not in r.stdout, r.stdout[-500:]
