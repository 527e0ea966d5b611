"""GPU: workspace-mode gradients whose event lanes are padded to whole 4-wave blocks.

The LDS-tile gradient kernel runs (channel-group lanes) x (event lanes) blocks; where a
few idle event lanes make the block a whole number of 4-wave groups, they are added and
only help stage the gradient tile. 512 channels with 3 updates (64 x 3 -> 64 x 4 lanes)
and 128 channels with 13 updates (16 x 13 -> 16 x 16) take the padded shape; 136
channels with 3 updates (no padding within the limit) is the control. Token counts
leave short reduction chunks.
"""
from __future__ import annotations

import pytest
import torch

from helpers import announce, assert_parity
from oracle import sihc_oracle as O
from sihc_hip import launch

pytestmark = pytest.mark.gpu

CASES = [(3, 512), (13, 128), (3, 136)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("active,channels", CASES, ids=[f"a{a}-c{c}" for a, c in CASES])
def test_padded_event_lanes(active, channels, dtype):
    announce(f"padded event lanes A={active} C={channels} dtype={dtype}")
    torch.manual_seed(41 + active + channels)
    rows = 3 * 13 * 13  # 507 tokens
    grad = torch.randn(1, rows, channels, device="cuda").to(dtype)
    ups = [torch.randn(1, rows, channels, device="cuda").to(dtype) for _ in range(active)]
    gamma = torch.randn(active, channels, device="cuda")
    ddz, dg = launch.triangular_backward(grad, ups, gamma, out_dtype=torch.float32)
    rdz, rdg = O.triangular_backward(grad.cpu(), [u.cpu() for u in ups], gamma.cpu())
    for j in range(active):
        assert torch.equal(ddz[j].cpu(), rdz[j]), f"update gradient {j} not bit-exact"
    wdt = torch.float32 if dtype == torch.float32 else dtype
    assert_parity(dg, rdg, wdt, what="dgamma (fused)", kind="reduced")
    gg = launch.triangular_gamma_grad(grad, ups, gamma, out_dtype=torch.float32)
    assert_parity(gg, O.triangular_gamma_grad(grad.cpu(), [u.cpu() for u in ups]), wdt, what="dgamma", kind="reduced")
    assert torch.equal(gg, launch.triangular_gamma_grad(grad, ups, gamma, out_dtype=torch.float32))
