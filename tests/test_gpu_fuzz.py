"""GPU: seeded random geometries through every C-ABI entry point, against the oracle.

Each case draws a batch, a workspace grid (not only 16x16), a cell size (4 or 16
slots), a channel count (odd counts force the scalar path, multiples of 8 the vector
paths), an event count in 1..32, a dtype and, for half the cases, a per-batch state
permutation. For an index, the expected values come from the oracle applied to the
carrier gathered through that index (and scattered back for carrier outputs), the
definition of the indexed variant. The tier's parity bar applies throughout.
"""
from __future__ import annotations

import random

import pytest
import torch

from helpers import announce, assert_parity
from oracle import sihc_oracle as O
from sihc_hip import launch

pytestmark = pytest.mark.gpu

CHANNELS = [1, 3, 7, 8, 16, 24, 37, 64, 67, 130, 256]


def _case(seed):
    r = random.Random(seed)
    k = r.choice([2, 4])
    return dict(seed=seed, k=k, s=k * k, g=r.choice([1, 2, 3, 5, 16]), b=r.choice([1, 2, 3]),
                c=r.choice(CHANNELS), e=r.randint(1, 32), dtype=r.choice([torch.float32, torch.bfloat16]),
                index=r.random() < 0.5)


CASES = [_case(1000 + i) for i in range(40)]


def _ids(c):
    return f"s{c['s']}-g{c['g']}-b{c['b']}-c{c['c']}-e{c['e']}-{str(c['dtype'])[6:]}-{'idx' if c['index'] else 'plain'}"


class _View:
    """Oracle-side view of a carrier through a per-batch state permutation."""

    def __init__(self, index, slots):
        self.index, self.slots = index, slots

    def gather(self, x):  # carrier whose cell n is the input's cell index[b, n]
        return x if self.index is None else O.cells_to_high(O.gather_cells(x, self.index, self.slots))

    def scatter(self, x):  # inverse of gather for a carrier output
        return x if self.index is None else O.scatter_cells(O.high_to_cells(x, self.slots), self.index)


@pytest.mark.parametrize("case", CASES, ids=_ids)
def test_random_geometry_all_entry_points(case):
    announce(f"fuzz {_ids(case)}")
    torch.manual_seed(case["seed"])
    b, g, k, s, c, e, dt = case["b"], case["g"], case["k"], case["s"], case["c"], case["e"], case["dtype"]
    dev = "cuda"
    gk = g * k
    x = torch.randn(b, gk, gk, c, device=dev).to(dt)
    alpha = (1.0 / s + 0.05 * torch.randn(e, c, s, device=dev)).to(dt)
    beta = (1.0 + 0.05 * torch.randn(e, c, s, device=dev)).to(dt)
    ups = [torch.randn(b, g * g, c, device=dev).to(dt) for _ in range(e)]
    idx = None
    if case["index"]:
        idx = torch.stack([torch.randperm(g * g, generator=torch.Generator().manual_seed(case["seed"] + i))
                           for i in range(b)]).to(torch.int32).to(dev)
    view = _View(None if idx is None else idx.cpu(), s)
    xc, ac, bc = x.cpu(), alpha.cpu(), beta.cpu()
    uc = [u.cpu() for u in ups]
    xp = view.gather(xc)

    # read / write (with and without the carrier) / weight gradient
    for i, (got, exp) in enumerate(zip(launch.read(x, alpha, index=idx), O.read(xp, ac))):
        assert_parity(got, exp, dt, what=f"read {i}")
    for add_x in (True, False):
        got = launch.write(x, ups, beta, add_x=add_x, index=idx)
        # under a permutation every cell is written once, so the scatter is complete
        exp = view.scatter(O.write(xp, uc, bc, add_x=add_x))
        assert_parity(got, exp, dt, what=f"write add_x={add_x}")
    got = launch.weight_grad(x, ups, alpha, index=idx, out_dtype=torch.float32)
    assert_parity(got, O.weight_grad(xp, uc, s), torch.float32 if dt == torch.float32 else dt, what="weight grad", kind="reduced")

    # triangular (an active prefix of the updates) and its fused backward
    a = max(1, min(e - 1, 1 + case["seed"] % 7)) if e > 1 else 1
    base, prefix = ups[0], ups[1:1 + a] if e > 1 else [ups[0]]
    a = len(prefix)
    gamma = torch.randn(a, c, device=dev) * 0.5
    if dt == torch.bfloat16 and case["seed"] % 2:
        gamma = gamma.to(dt)
    got = launch.triangular(base, prefix, gamma)
    assert_parity(got, O.triangular_torch(base.cpu(), [p.cpu() for p in prefix], gamma.cpu()), dt,
                  what="triangular")
    ddz, dg = launch.triangular_backward(base, prefix, gamma, out_dtype=torch.float32)
    rdz, rdg = O.triangular_backward(base.cpu(), [p.cpu() for p in prefix], gamma.cpu())
    for j in range(a):
        assert torch.equal(ddz[j].cpu(), rdz[j]), f"triangular backward d{j} not bit-exact"
    assert_parity(dg, rdg, torch.float32 if dt == torch.float32 else dt, what="triangular dgamma", kind="reduced")

    # per-event forward and its backward in every mode
    b0, a1 = beta[0].contiguous(), alpha[min(1, e - 1)].contiguous()
    xo, zo = launch.event_forward(x, ups[0], b0, a1, index=idx)
    rxo, rzo = O.event_forward(xp, uc[0], b0.cpu(), a1.cpu())
    assert_parity(xo, view.scatter(rxo), dt, what="event x_out")
    assert_parity(zo, rzo, dt, what="event z_out")
    h = (1e-2 * torch.randn(x.shape, device=dev)).to(dt)
    gz = (1e-2 * torch.randn(b, g * g, c, device=dev)).to(dt)
    hp, xop = view.gather(h.cpu()), view.gather(xo.cpu())
    wdt = torch.float32 if dt == torch.float32 else dt
    for mode in ("full", "write-only", "read-only"):
        args = dict(full=(h, gz, xo, ups[0], b0, a1), **{"write-only": (h, None, None, ups[0], b0, None),
                                                        "read-only": (h, gz, xo, None, None, a1)})[mode]
        gx, gdz, gb, ga = launch.event_backward(*args, index=idx, carrier_like=x)
        ref = O.event_backward(hp, None if args[1] is None else gz.cpu(), xop, uc[0], b0.cpu(),
                               None if args[5] is None else a1.cpu())
        if mode != "write-only":
            assert_parity(gx, view.scatter(ref[0]).to(dt), dt, what=f"event bwd {mode} grad_x")
        if mode != "read-only":
            assert_parity(gdz, ref[1].to(dt), dt, what=f"event bwd {mode} grad_dz")
            assert_parity(gb, ref[2].to(wdt), wdt, what=f"event bwd {mode} grad_beta", kind="reduced")
        if mode != "write-only":
            assert_parity(ga, ref[3].to(wdt), wdt, what=f"event bwd {mode} grad_alpha", kind="reduced")

    # bit-exact cell copies
    cells = launch.gather_cells(x, idx, s)
    assert torch.equal(cells.cpu(), O.gather_cells(xc, view.index, s))
    if idx is not None:
        assert torch.equal(launch.scatter_cells(cells, idx), x)
