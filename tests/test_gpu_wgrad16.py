"""GPU: the 16-slot weight gradient over every launch shape of its bf16 kernels.

bf16 carriers with rows of whole 16-byte vectors and 8..24 events take the pipelined
kernel (3 or 4 events per lane, 2..8 event waves); other event counts, channel counts
that are not multiples of 8 and fp32 take the one-channel-per-lane kernel. Products of
bf16 values are exact in fp32 and the sums are fp32, so the fp32 bar applies against the
oracle's float64 sums of the same bf16 inputs. Token tails (grids of 5x5 cells), channel
tails (136 = 2 x 64 + 8 channels) and per-batch state permutations are covered.
"""
from __future__ import annotations

import pytest
import torch

from helpers import announce, assert_parity
from oracle import sihc_oracle as O
from sihc_hip import launch

pytestmark = pytest.mark.gpu

# event counts hitting each (events per lane, waves) shape: 8 -> 4x2, 9 -> 4x3,
# 12 -> 3x4, 16 -> 4x4, 20 -> 4x5, 21 -> 4x6, 24 -> 3x8; 4 and 25 use the other kernel
EVENTS = [4, 8, 9, 12, 16, 20, 21, 24, 25]


@pytest.mark.parametrize("events", EVENTS)
@pytest.mark.parametrize("geom", [(2, 16, 64, False), (3, 5, 136, True), (1, 16, 1152, True)],
                         ids=["b2-g16-c64", "b3-g5-c136-index", "b1-g16-c1152-index"])
def test_weight_grad_16_slots_bf16(events, geom):
    b, g, c, with_index = geom
    announce(f"wgrad16 b={b} g={g} c={c} events={events} index={with_index}")
    torch.manual_seed(7 * events + c)
    x = torch.randn(b, 4 * g, 4 * g, c, device="cuda").to(torch.bfloat16)
    ups = [torch.randn(b, g * g, c, device="cuda").to(torch.bfloat16) for _ in range(events)]
    w = torch.randn(events, c, 16, device="cuda").to(torch.bfloat16)
    index = None
    if with_index:
        gen = torch.Generator().manual_seed(events)
        index = torch.stack([torch.randperm(g * g, generator=gen) for _ in range(b)]).to(torch.int32)
    got = launch.weight_grad(x, ups, w, index=None if index is None else index.cuda(), out_dtype=torch.float32)
    xp = x.cpu() if index is None else O.cells_to_high(O.gather_cells(x.cpu(), index, 16))
    exp = O.weight_grad(xp, [u.cpu() for u in ups], 16)
    assert_parity(got, exp, torch.float32, what=f"wgrad16 events={events}")
    # deterministic: a second call gives the same bits
    assert torch.equal(got, launch.weight_grad(x, ups, w, index=None if index is None else index.cuda(),
                                               out_dtype=torch.float32))
