"""GPU: the 16-slot bf16 read and write whose sums run in bf16 pairs (v_dot2c_f32_bf16:
slot pairs for the read, event pairs for the write). They take every 16-slot bf16 call with
an even channel count and word-aligned tensors; the other tests of those ops use odd channel
counts or fp32 in places, so this file covers the paired paths on purpose: token tails
(grids of 5x5 and 7x7 cells), channel tails (72 = 64 + 8 channels in a 64-channel slice,
6 channels), odd event counts (the write's last pair has a zero half), 1..32 events and a
per-batch state permutation. Each pair sum adds exact bf16 products in fp32, so the outputs
meet the elementwise bar (1 bf16 ulp of the oracle) as the unpaired kernels do.
"""
from __future__ import annotations

import pytest
import torch

from helpers import announce, assert_parity
from oracle import sihc_oracle as O
from sihc_hip import launch

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16
EVENTS = [1, 2, 3, 8, 13, 24, 32]
GEOMS = [(3, 5, 72, False), (2, 7, 72, True), (2, 4, 6, False), (1, 16, 1152, True)]
GEOM_IDS = ["b3-g5-c72", "b2-g7-c72-index", "b2-g4-c6", "b1-g16-c1152-index"]


def _case(b, g, c, with_index, events, seed):
    torch.manual_seed(seed)
    x = torch.randn(b, 4 * g, 4 * g, c, device="cuda").to(BF16)
    alpha = (0.25 + 0.02 * torch.randn(events, c, 16, device="cuda")).to(BF16)
    beta = (1.0 + 0.02 * torch.randn(events, c, 16, device="cuda")).to(BF16)
    ups = [torch.randn(b, g * g, c, device="cuda").to(BF16) for _ in range(events)]
    index = None
    if with_index:
        gen = torch.Generator().manual_seed(events + c)
        index = torch.stack([torch.randperm(g * g, generator=gen) for _ in range(b)]).to(torch.int32)
    return x, alpha, beta, ups, index


def _cells_view(x, index):
    """The carrier as the oracle sees the indexed kernels' cells (gather through the index)."""
    return x.cpu() if index is None else O.cells_to_high(O.gather_cells(x.cpu(), index, 16))


@pytest.mark.parametrize("events", EVENTS)
@pytest.mark.parametrize("geom", GEOMS, ids=GEOM_IDS)
def test_read_slot_pairs(events, geom):
    b, g, c, with_index = geom
    announce(f"dot2 read b={b} g={g} c={c} events={events} index={with_index}")
    x, alpha, _, _, index = _case(b, g, c, with_index, events, seed=11 * events + c)
    got = launch.read(x, alpha, index=None if index is None else index.cuda())
    exp = O.read(_cells_view(x, index), alpha.cpu())
    for e in range(events):
        assert_parity(got[e], exp[e], BF16, what=f"read event {e}")


@pytest.mark.parametrize("add_x", [True, False])
@pytest.mark.parametrize("events", EVENTS)
@pytest.mark.parametrize("geom", GEOMS, ids=GEOM_IDS)
def test_write_event_pairs(events, geom, add_x):
    b, g, c, with_index = geom
    announce(f"dot2 write b={b} g={g} c={c} events={events} add_x={add_x} index={with_index}")
    x, _, beta, ups, index = _case(b, g, c, with_index, events, seed=13 * events + c)
    idx = None if index is None else index.cuda()
    got = launch.write(x, ups, beta, add_x=add_x, index=idx)
    if index is None:
        exp = O.write(x.cpu(), [u.cpu() for u in ups], beta.cpu(), add_x=add_x)
        assert_parity(got, exp, BF16, what="write")
    else:
        # through a permutation the kernel writes the cell of state index[m]: compare the
        # gathered cells with the oracle's write of the gathered carrier
        cells = _cells_view(x, index)
        exp = O.write(cells, [u.cpu() for u in ups], beta.cpu(), add_x=add_x)
        got_cells = O.cells_to_high(O.gather_cells(got.cpu(), index, 16))
        assert_parity(got_cells, exp, BF16, what="write (gathered cells)")
    # a second call gives the same bits
    assert torch.equal(got, launch.write(x, ups, beta, add_x=add_x, index=idx))


# 4-slot bf16 reads with 8+ events and 16-byte lanes (C % 8 == 0): the one-array-per-wave
# kernel that stages the cell tile as slot-pair words (token tails: 5x5 and 7x7 grids;
# channel tails: 136 = 128 + 8)
GEOMS4 = [(3, 5, 136, False), (2, 7, 136, True), (1, 16, 1152, True)]


@pytest.mark.parametrize("events", [8, 13, 24, 32])
@pytest.mark.parametrize("geom", GEOMS4, ids=["b3-g5-c136", "b2-g7-c136-index", "b1-g16-c1152-index"])
def test_read_4slot_wave_per_event(events, geom):
    b, g, c, with_index = geom
    announce(f"4-slot wave read b={b} g={g} c={c} events={events} index={with_index}")
    torch.manual_seed(17 * events + c)
    x = torch.randn(b, 2 * g, 2 * g, c, device="cuda").to(BF16)
    alpha = (0.25 + 0.02 * torch.randn(events, c, 4, device="cuda")).to(BF16)
    index = None
    if with_index:
        gen = torch.Generator().manual_seed(events + c)
        index = torch.stack([torch.randperm(g * g, generator=gen) for _ in range(b)]).to(torch.int32)
    got = launch.read(x, alpha, index=None if index is None else index.cuda())
    xs = x.cpu() if index is None else O.cells_to_high(O.gather_cells(x.cpu(), index, 4))
    exp = O.read(xs, alpha.cpu())
    for e in range(events):
        assert_parity(got[e], exp[e], BF16, what=f"read event {e}")
