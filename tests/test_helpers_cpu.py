"""CPU tests of the parity helpers' bf16 bar: the 2^-10 head-max floor is
counted (elements that pass only through it), capped when asked, and a
result beyond the floored ulp still fails."""
from __future__ import annotations

import pytest
import torch

from helpers import assert_bf16_within_ulp


def test_floor_only_elements_are_counted_and_capped():
    ref = torch.tensor([[1.0, 0.5, 2.0 ** -12, -3.0]])
    floor = ref.abs().amax(dim=-1, keepdim=True)            # 3.0: floored ulp = ulp(3 * 2^-10)
    out = ref.clone()
    out[0, 1] += 2.0 ** -9                                  # exactly 1 ulp of 0.5: passes on its own
    out[0, 2] += 2.0 ** -16                                 # 8 ulps of 2^-12: 1 floored ulp
    st = assert_bf16_within_ulp(out.to(torch.bfloat16).float(), ref, floor, what="t")
    assert st["floor_only"] == 1 and st["elements"] == 4
    assert st["floor_only_max_ulps"] == pytest.approx(8.0)
    assert_bf16_within_ulp(out, ref, floor, what="t", floor_cap=0.25)
    with pytest.raises(AssertionError, match="only through the 2\\^-10 floor"):
        assert_bf16_within_ulp(out, ref, floor, what="t", floor_cap=0.2)


def test_beyond_the_floored_ulp_fails():
    ref = torch.tensor([[1.0, 2.0 ** -12, -3.0]])
    out = ref.clone()
    out[0, 1] += 2.0 ** -15                                 # 2 floored ulps (2^-16 each)
    with pytest.raises(AssertionError, match="beyond 1.0 bf16 ulp"):
        assert_bf16_within_ulp(out, ref, ref.abs().amax(dim=-1, keepdim=True), what="t")
