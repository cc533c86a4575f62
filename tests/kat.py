"""Hand-derived known-answer rows for the per-token FP8 rule
(deploy/joyomni_ops/csrc/per_token_quant_fp8.cu:56-82).

Each entry: (row values, expected scale, expected e4m3fn bytes). The
expectations were worked out by hand from the rule
  scale = amax/448, inv = scale==0 ? 0 : 1/scale, q = rne(clamp(x*inv, +-448))
and the e4m3fn code table (bias 7, 3 mantissa bits, 0x7e = 448, subnormals
m * 2^-9); they do not come from any implementation.
"""
from __future__ import annotations

import math

NAN = float("nan")
INF = float("inf")

# Codes: 1.0 = 0x38, 1.125 = 0x39, 1.25 = 0x3a, 2.0 = 0x40, 448 = 0x7e,
# 2^-9 (smallest subnormal) = 0x01, sign bit 0x80.
KAT_ROWS = [
    # all-zero row: scale 0, inv 0, every code +0.
    ([0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0], 0.0, [0x00] * 8),
    # amax 448 -> scale 1, inv 1. 1.0625 is the 1.0/1.125 midpoint (even: 0x38);
    # 1.1875 is the 1.125/1.25 midpoint (even: 0x3a); signs mirror.
    ([448.0, 1.0625, 1.1875, -1.0625, -1.1875, 1.0, -448.0, 2.0], 1.0,
     [0x7e, 0x38, 0x3a, 0xb8, 0xba, 0x38, 0xfe, 0x40]),
    # NaN is skipped by the max: amax 2 -> scale 2/448, inv 224. 2*224 = 448;
    # NaN*224 = NaN and fminf(NaN, 448) = 448 -> 0x7e; 1*224 = 224 = 0x76.
    ([NAN, 2.0, 1.0, -2.0, 0.0, NAN, 0.5, -1.0], 2.0 / 448.0,
     [0x7e, 0x7e, 0x76, 0xfe, 0x00, 0x7e, 0x6e, 0xf6]),
    # +inf: scale inf, inv 1/inf = 0; inf*0 = NaN -> 448; finite*0 = +-0.
    ([INF, 1.0, -1.0, 0.0, 3.0, -3.0, 0.5, -0.5], INF,
     [0x7e, 0x00, 0x80, 0x00, 0x00, 0x80, 0x00, 0x80]),
    # -inf behaves the same: |-inf| = inf; -inf*0 = NaN -> +448 (0x7e).
    ([-INF, 1.0, -1.0, 0.0, 2.0, -2.0, 4.0, -4.0], INF,
     [0x7e, 0x00, 0x80, 0x00, 0x00, 0x80, 0x00, 0x80]),
    # Subnormal boundary with scale 1: 2^-10 is the 0 / 2^-9 midpoint (even: 0);
    # 1.5*2^-10 rounds up to 2^-9 (0x01); 3*2^-10 is the 2^-9 / 2^-8 midpoint
    # (even: 2^-8 = 0x02); 2^-7 = 0x04 exactly.
    ([448.0, 2.0 ** -10, 1.5 * 2.0 ** -10, 3 * 2.0 ** -10, 2.0 ** -7, -(2.0 ** -10),
      -(1.5 * 2.0 ** -10), 0.0], 1.0,
     [0x7e, 0x00, 0x01, 0x02, 0x04, 0x80, 0x81, 0x00]),
    # Tiny row: amax 2^-126 -> scale = 2^-126/448 = 2^-132/7, a denormal that
    # rounds to 18725 * 2^-149; 1/scale overflows to inf. Nonzero x*inf = +-inf
    # clamps to +-448; +-0 * inf = NaN -> 448.
    ([2.0 ** -127, -(2.0 ** -127), 0.0, 2.0 ** -128, -0.0, 2.0 ** -127, 2.0 ** -126,
      -(2.0 ** -126)], 18725 * 2.0 ** -149,
     [0x7e, 0xfe, 0x7e, 0x7e, 0x7e, 0x7e, 0x7e, 0xfe]),
    # amax 7 -> scale 7/448 = 1/64 exactly, inv 64: x*64 exact; 7*64 = 448;
    # 3.5*64 = 224 = 0x76; 0.0078125*64 = 0.5 = 0x30; 5*64 = 320 = 0x7a;
    # 1*64 = 64 = 0x68; 0.25*64 = 16 = 0x58.
    ([7.0, 3.5, 0.0078125, 5.0, -7.0, -3.5, 1.0, 0.25], 1.0 / 64.0,
     [0x7e, 0x76, 0x30, 0x7a, 0xfe, 0xf6, 0x68, 0x58]),
]


def check_table() -> None:
    """Self-check of the hand table against the e4m3fn value of each code."""
    def dec(c):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 7
        return s * (m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7))
    assert dec(0x7e) == 448 and dec(0x38) == 1 and dec(0x76) == 224 and dec(0x6e) == 112
    assert dec(0x7a) == 320 and dec(0x68) == 64 and dec(0x58) == 16 and dec(0x30) == 0.5
    assert dec(0x01) == 2.0 ** -9 and dec(0x02) == 2.0 ** -8 and dec(0x04) == 2.0 ** -7
    assert math.isclose(dec(0x40), 2.0) and dec(0xfe) == -448
