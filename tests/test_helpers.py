"""CPU: the parity bar itself. bf16_ulp against the bit-level successor of bfloat16 values, and
the elementwise bar accepting a 1-ulp difference but rejecting a planted 2-ulp one."""
from __future__ import annotations

import pytest
import torch

from helpers import NEAR_ZERO_SLACK, assert_parity, bf16_ulp


def test_bf16_ulp_is_the_spacing_of_bfloat16():
    torch.manual_seed(0)
    mags = torch.cat([torch.randn(4000) * 10.0 ** torch.randint(-30, 30, (4000,)).float(),
                      torch.tensor([1.0, 2.0, 0.5, 3.0, 1e-38, 2.0 ** -126])])
    x = mags.abs().to(torch.bfloat16)
    x = x[(x > 0) & torch.isfinite(x)]
    # the next bfloat16 above a positive x: its bit pattern plus one
    step = (x.view(torch.int16) + 1).view(torch.bfloat16)
    assert torch.equal(bf16_ulp(x.float()), step.double() - x.double())


def test_elementwise_bar_accepts_one_ulp_and_rejects_two():
    torch.manual_seed(1)
    ref = torch.randn(1000).to(torch.bfloat16)
    one = (ref.view(torch.int16) + 1).view(torch.bfloat16)  # one ulp away (sign-magnitude)
    assert_parity(one, ref, torch.bfloat16, what="one ulp")
    two = ref.clone()
    two.view(torch.int16)[17] += 2  # a planted two-ulp error in one element
    with pytest.raises(AssertionError, match="beyond 1 ulp"):
        assert_parity(two, ref, torch.bfloat16, what="two ulp")
    # the scaled bar of reductions and chains accepts it
    assert_parity(two, ref, torch.bfloat16, what="two ulp scaled", kind="reduced")


def test_near_zero_slack_is_relative_to_the_largest_value():
    ref = torch.tensor([4.0, 1e-6, -3.0], dtype=torch.float64)
    got = ref.clone()
    got[1] += 0.9 * NEAR_ZERO_SLACK * 4.0  # far beyond 1 ulp of 1e-6, within the slack
    assert_parity(got, ref, torch.bfloat16, what="near zero")
    got[1] = ref[1] + 2 * NEAR_ZERO_SLACK * 4.0
    with pytest.raises(AssertionError):
        assert_parity(got, ref, torch.bfloat16, what="near zero too far")
