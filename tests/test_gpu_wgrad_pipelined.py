"""GPU: the carrier weight gradient over every launch shape of its bf16 kernels.

bf16 carriers with rows of whole 16-byte vectors and up to 32 events take the pipelined
kernels (one channel per lane, EPL events per lane, 2..8 event waves chosen per event
count) or, at 4 slots for most event counts, 16-byte row lanes (8 channels x 4 slots x
1-4 events per thread, 2, 4 or 8 event groups); one event at 4 slots, channel counts that
are not multiples of 8 and fp32 take the other kernels.
Products of bf16 values are exact in fp32 and the sums are fp32, so the fp32 bar applies
against the oracle's float64 sums of the same bf16 inputs. Token tails (grids of 5x5
cells), channel tails (136 = 2 x 64 + 8 channels; 24 channels in one 64-lane slice) and
per-batch state permutations are covered. The gamma gradient (one-slot workspace rows)
runs on the pipelined kernel for 2 updates and on 16-byte row lanes for 3..32 (136
channels: a second 128-channel slice holding one lane; 24: three lanes of one slice).
"""
from __future__ import annotations

import pytest
import torch

from helpers import announce, assert_parity
from oracle import sihc_oracle as O
from sihc_hip import launch

pytestmark = pytest.mark.gpu

CASES = [  # (slots, events): the kernel and its shape
    (4, 1),    # the direct kernel
    (4, 2),    # row lanes, 2 groups x 1 event
    (4, 3),    # pipelined 4 waves x 1 (one wave stages only)
    (4, 4),    # pipelined 4 x 1
    (4, 5),    # row lanes 2 x 3 (the last group repeats an event)
    (4, 6),    # row lanes 2 x 3
    (4, 7),    # row lanes 4 x 2 (one repeated event)
    (4, 12),   # row lanes 4 x 3
    (4, 13),   # row lanes 4 x 4 (three repeated)
    (4, 16),   # row lanes 4 x 4
    (4, 17),   # pipelined 6 waves x 3
    (4, 18),   # pipelined 6 x 3
    (4, 19),   # row lanes 8 x 3 (five repeated)
    (4, 24),   # row lanes 8 x 3
    (4, 25),   # row lanes 8 x 4
    (4, 32),   # row lanes 8 x 4
    # 16 slots: waves x events per lane of the pipelined dot2 kernel
    (16, 1),   # 4 x 1 (three waves stage only)
    (16, 4),   # 4 x 1
    (16, 5),   # 2 x 4
    (16, 8),   # 2 x 4
    (16, 9),   # 3 x 3
    (16, 12),  # 4 x 3
    (16, 13),  # 4 x 4
    (16, 16),  # 4 x 4
    (16, 17),  # 8 x 3
    (16, 21),  # 8 x 3
    (16, 24),  # 8 x 3
    (16, 25),  # 8 x 4
    (16, 32),  # 8 x 4
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


# 2: the pipelined kernel (1 wave x 2 updates); 3..32: row lanes, update groups x updates per
# lane 4 x 1 (3, 4: the last group repeats an update), 1 x A (5..10), 2 x 6..11 (11..22, odd
# counts half-filled), 4 x 6..8 (23..32)
GAMMA_CASES = [2, 3, 4, 5, 7, 10, 11, 12, 17, 22, 23, 25, 32]


@pytest.mark.parametrize("active", GAMMA_CASES)
@pytest.mark.parametrize("rows,channels", [(3 * 13 * 13, 136), (4096, 1152), (77, 24)],
                         ids=["r507-c136", "r4096-c1152", "r77-c24"])
def test_gamma_grad_bf16(active, rows, channels):
    # the gamma gradient of the triangular op over bf16 workspace rows: sum over rows of
    # grad * update_j (the pipelined kernel for 2 updates, row lanes for 3..32)
    announce(f"gamma grad bf16 A={active} rows={rows} C={channels}")
    torch.manual_seed(5 * active + channels)
    grad = torch.randn(1, rows, channels, device="cuda").to(torch.bfloat16)
    ups = [torch.randn(1, rows, channels, device="cuda").to(torch.bfloat16) for _ in range(active)]
    gamma = 0.05 * torch.randn(active, channels, device="cuda")
    got = launch.triangular_gamma_grad(grad, ups, gamma, out_dtype=torch.float32)
    exp = O.triangular_gamma_grad(grad.cpu(), [u.cpu() for u in ups])
    assert_parity(got, exp, torch.float32, what=f"dgamma A={active}")
    assert torch.equal(got, launch.triangular_gamma_grad(grad, ups, gamma, out_dtype=torch.float32))
