"""GPU: the carrier weight gradient over every launch shape of its bf16 kernels.

bf16 carriers with rows of whole 16-byte vectors and up to 24 events take the pipelined
kernel (one channel per lane, EPL events per lane, 2..8 event waves; under 8 events 4
waves of 1 or 2 events, or 2 waves of 4 at 16 slots); other event counts (4 slots: 1
event, and counts with no balanced shape), channel counts that are not multiples of 8
and fp32 take the other kernels.
Products of bf16 values are exact in fp32 and the sums are fp32, so the fp32 bar applies
against the oracle's float64 sums of the same bf16 inputs. Token tails (grids of 5x5
cells), channel tails (136 = 2 x 64 + 8 channels; 24 channels in one 64-lane slice) and
per-batch state permutations are covered.
"""
from __future__ import annotations

import pytest
import torch

from helpers import announce, assert_parity
from oracle import sihc_oracle as O
from sihc_hip import launch

pytestmark = pytest.mark.gpu

# (slots, events): events per lane x waves of the pipelined kernel, or the other kernel
CASES = [
    (4, 1),    # the direct kernel
    (4, 2),    # 1 x 4 (two waves stage only)
    (4, 4),    # 1 x 4
    (4, 5),    # 2 x 4 (last wave partly empty)
    (4, 6),    # 2 x 4
    (4, 7),    # 2 x 4
    (4, 8),    # 2 x 4
    (4, 9),    # no balanced shape: the LDS-tile kernel
    (4, 12),   # 3 x 4
    (4, 16),   # 4 x 4
    (4, 17),   # the LDS-tile kernel
    (4, 20),   # 6 x 4 (last wave partly empty)
    (4, 24),   # 6 x 4
    (16, 1),   # 1 x 4 (three waves stage only)
    (16, 3),   # 1 x 4
    (16, 4),   # 1 x 4
    (16, 5),   # 4 x 2 (last wave partly empty)
    (16, 7),   # 4 x 2
    (16, 8),   # 4 x 2
    (16, 9),   # 4 x 3
    (16, 12),  # 3 x 4
    (16, 16),  # 4 x 4
    (16, 20),  # 4 x 5
    (16, 21),  # 4 x 6
    (16, 24),  # 3 x 8
    (16, 25),  # the one-channel-per-lane kernel
]
GEOMS = [(2, 16, 64, False), (3, 5, 136, True), (1, 16, 1152, True), (2, 4, 24, False)]


@pytest.mark.parametrize("slots,events", CASES, ids=[f"s{s}-e{e}" for s, e in CASES])
@pytest.mark.parametrize("geom", GEOMS, ids=["b2-g16-c64", "b3-g5-c136-index", "b1-g16-c1152-index", "b2-g4-c24"])
def test_carrier_weight_grad_bf16(slots, events, geom):
    b, g, c, with_index = geom
    k = O.cell_edge(slots)
    announce(f"wgrad slots={slots} b={b} g={g} c={c} events={events} index={with_index}")
    torch.manual_seed(7 * events + c + slots)
    x = torch.randn(b, k * g, k * g, c, device="cuda").to(torch.bfloat16)
    ups = [torch.randn(b, g * g, c, device="cuda").to(torch.bfloat16) for _ in range(events)]
    w = torch.randn(events, c, slots, device="cuda").to(torch.bfloat16)
    index = None
    if with_index:
        gen = torch.Generator().manual_seed(events)
        index = torch.stack([torch.randperm(g * g, generator=gen) for _ in range(b)]).to(torch.int32)
    idx = None if index is None else index.cuda()
    got = launch.weight_grad(x, ups, w, index=idx, out_dtype=torch.float32)
    xp = x.cpu() if index is None else O.cells_to_high(O.gather_cells(x.cpu(), index, slots))
    exp = O.weight_grad(xp, [u.cpu() for u in ups], slots)
    assert_parity(got, exp, torch.float32, what=f"wgrad slots={slots} events={events}")
    # deterministic: a second call gives the same bits
    assert torch.equal(got, launch.weight_grad(x, ups, w, index=idx, out_dtype=torch.float32))
