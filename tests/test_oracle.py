"""CPU: pin the oracle before trusting it (no GPU, no product code).

Each check is chosen so that a plausible oracle mistake (swapped slot order, a
transposed weight, a dropped term, a wrong adjoint) fails at least one of them.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import sihc_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    return dict(np.load(GOLDEN / f"{name}.npz", allow_pickle=False))


def test_known_answer_slot_order_and_round_trip():
    # Reference known answer: research/tests/test_reference_variants.py:85-94.
    high = torch.arange(32 * 32, dtype=torch.float32).reshape(1, 32, 32, 1)
    cells = O.high_to_cells(high, 4)
    assert cells.shape == (1, 256, 4, 1)
    assert cells[0, 0, :, 0].tolist() == [0.0, 1.0, 32.0, 33.0]
    assert torch.equal(O.cells_to_high(cells), high)
    # p4 (16 slots): first cell is rows 0..3, cols 0..3 of a 64-wide carrier.
    high4 = torch.arange(64 * 64, dtype=torch.float32).reshape(1, 64, 64, 1)
    c4 = O.high_to_cells(high4, 16)
    assert c4[0, 0, :, 0].tolist() == [r * 64 + c for r in range(4) for c in range(4)]
    assert torch.equal(O.cells_to_high(c4), high4)


def test_carrier_offset_matches_cell_layout():
    # The brute-force index map agrees with the reshape/permute layout on every element.
    x = torch.arange(2 * 6 * 6 * 3, dtype=torch.float64).reshape(2, 6, 6, 3)
    cells = O.high_to_cells(x, 4)
    for m in range(2 * 9):
        for s in range(4):
            for c in range(3):
                assert O.carrier_offset(m, s, c, 3, 3, 2) == int(cells[m // 9, m % 9, s, c])


@pytest.mark.parametrize("name", ["p8_small", "p4_small"])
def test_torch_restatement_matches_brute_force_fixtures(name):
    f = _load(name)
    x = torch.from_numpy(f["x"]).double()
    alpha = torch.from_numpy(f["alpha"]).double()
    beta = torch.from_numpy(f["beta"]).double()
    updates = [torch.from_numpy(u).double() for u in f["updates"]]
    slots = alpha.shape[2]
    got = torch.stack(O.read(x, alpha))
    torch.testing.assert_close(got, torch.from_numpy(f["read"]), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(O.write(x, updates, beta), torch.from_numpy(f["write"]), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(O.write(x, updates, beta, add_x=False), torch.from_numpy(f["write_noadd"]),
                               rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(O.weight_grad(x, updates, slots).double(), torch.from_numpy(f["weight_grad"]),
                               rtol=1e-6, atol=1e-6)
    gamma = torch.from_numpy(f["gamma"]).double()
    torch.testing.assert_close(O.triangular_torch(updates[0], updates[1:], gamma[1:]),
                               torch.from_numpy(f["triangular"]), rtol=1e-12, atol=1e-12)
    index = torch.from_numpy(f["index"])
    assert torch.equal(O.gather_cells(torch.from_numpy(f["x"]), index, slots), torch.from_numpy(f["gather"]))


@pytest.mark.parametrize("slots", [4, 16])
def test_read_write_are_adjoint(slots):
    torch.manual_seed(1)
    k = O.cell_edge(slots)
    x = torch.randn(2, 5 * k, 5 * k, 7, dtype=torch.float64)
    alpha = torch.randn(3, 7, slots, dtype=torch.float64)
    g = [torch.randn(2, 25, 7, dtype=torch.float64) for _ in range(3)]
    lhs = sum((z * gi).sum() for z, gi in zip(O.read(x, alpha), g))
    rhs = (x * O.write(x, g, alpha, add_x=False)).sum()
    torch.testing.assert_close(lhs, rhs, rtol=1e-12, atol=1e-12)


def test_identity_initialised_stage_is_the_residual_recurrence():
    # Reference: research/tests/test_reference_variants.py:97-123.
    torch.manual_seed(0)
    high = torch.randn(2, 32, 32, 5, dtype=torch.float64)
    alpha = torch.full((3, 5, 4), 0.25, dtype=torch.float64)
    beta = torch.ones(3, 5, 4, dtype=torch.float64)
    fns = [lambda z, s=s: torch.tanh(z * s) for s in (0.1, 0.2, 0.3)]
    actual = O.fused_stage(high, alpha, beta, fns)
    cells = O.high_to_cells(high, 4)
    z = cells.mean(dim=2)
    ups = []
    for fn in fns:
        u = fn(z)
        ups.append(u)
        z = z + u
    expected = O.cells_to_high(cells + torch.stack(ups).sum(0).unsqueeze(2))
    torch.testing.assert_close(actual, expected)


@pytest.mark.parametrize("slots", [4, 16])
def test_literal_recurrence_equals_fused_stage(slots):
    # Late materialisation (README.md:36-51) is exact algebra: check it in float64.
    torch.manual_seed(5)
    k = O.cell_edge(slots)
    x = torch.randn(2, 4 * k, 4 * k, 6, dtype=torch.float64)
    alpha = 0.3 * torch.randn(6, 6, slots, dtype=torch.float64)
    beta = 0.3 * torch.randn(6, 6, slots, dtype=torch.float64)
    fns = [lambda z, i=i: torch.tanh((i + 1) * 0.1 * z) for i in range(6)]
    torch.testing.assert_close(O.literal_stage(x, alpha, beta, fns), O.fused_stage(x, alpha, beta, fns),
                               rtol=1e-10, atol=1e-10)


def test_weight_gradients_match_autograd():
    torch.manual_seed(2)
    x = torch.randn(2, 8, 8, 3, dtype=torch.float64, requires_grad=True)
    alpha = torch.randn(2, 3, 4, dtype=torch.float64, requires_grad=True)
    g = [torch.randn(2, 16, 3, dtype=torch.float64) for _ in range(2)]
    loss = sum((z * gi).sum() for z, gi in zip(O.read(x, alpha), g))
    dx, da = torch.autograd.grad(loss, (x, alpha))
    torch.testing.assert_close(O.weight_grad(x.detach(), g, 4).double(), da, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(O.write(x.detach(), g, alpha.detach(), add_x=False), dx)
    # triangular gamma gradient == autograd of triangular_torch
    base = torch.randn(2, 16, 3, dtype=torch.float64)
    ups = [torch.randn(2, 16, 3, dtype=torch.float64) for _ in range(3)]
    gamma = torch.randn(3, 3, dtype=torch.float64, requires_grad=True)
    go = torch.randn(2, 16, 3, dtype=torch.float64)
    (dg,) = torch.autograd.grad((O.triangular_torch(base, ups, gamma) * go).sum(), (gamma,))
    torch.testing.assert_close(O.triangular_gamma_grad(go, ups).double(), dg, rtol=1e-6, atol=1e-6)


def test_triangular_backward_matches_autograd():
    torch.manual_seed(5)
    base = torch.randn(2, 16, 3, dtype=torch.float64, requires_grad=True)
    ups = [torch.randn(2, 16, 3, dtype=torch.float64, requires_grad=True) for _ in range(4)]
    gamma = torch.randn(4, 3, dtype=torch.float64, requires_grad=True)
    go = torch.randn(2, 16, 3, dtype=torch.float64)
    grads = torch.autograd.grad((O.triangular_torch(base, ups, gamma) * go).sum(), (base, *ups, gamma))
    torch.testing.assert_close(grads[0], go)
    ddz, dg = O.triangular_backward(go, [u.detach() for u in ups], gamma.detach())
    for a, b in zip(ddz, grads[1:5]):
        torch.testing.assert_close(a, b)
    torch.testing.assert_close(dg.double(), grads[5], rtol=1e-6, atol=1e-6)


def test_cell_mean_is_average_pooling_over_cells():
    # Pinned by torch's 4x4 average pooling of the NCHW carrier: a wrong cell map (rows
    # and columns swapped, a 2x2 cell) or a wrong scale fails it.
    torch.manual_seed(6)
    x = torch.randn(2, 64, 64, 5, dtype=torch.float64)
    pooled = torch.nn.functional.avg_pool2d(x.permute(0, 3, 1, 2), 4)         # [B,C,16,16]
    expected = pooled.permute(0, 2, 3, 1).reshape(2, 256, 5)
    torch.testing.assert_close(O.cell_mean(x), expected)
    # fp32: the fp32 slot-order sum times 1/16 (exact scaling) equals the fp64 mean
    # rounded once only up to the sum's rounding
    x32 = x.float()
    torch.testing.assert_close(O.cell_mean(x32).double(), expected, rtol=1e-6, atol=1e-6)
    assert O.cell_mean(x32.bfloat16()).dtype == torch.bfloat16


def test_event_backward_matches_autograd():
    torch.manual_seed(3)
    x = torch.randn(2, 6, 6, 4, dtype=torch.float64, requires_grad=True)
    dz = torch.randn(2, 9, 4, dtype=torch.float64, requires_grad=True)
    beta = torch.randn(4, 4, dtype=torch.float64, requires_grad=True)
    alpha = torch.randn(4, 4, dtype=torch.float64, requires_grad=True)
    x_out, z_out = O.event_forward(x, dz, beta, alpha)
    h = torch.randn_like(x_out)
    g = torch.randn_like(z_out)
    grads = torch.autograd.grad((x_out * h).sum() + (z_out * g).sum(), (x, dz, beta, alpha))
    mine = O.event_backward(h, g, x_out.detach(), dz.detach(), beta.detach(), alpha.detach())
    for a, b in zip(mine, grads):
        torch.testing.assert_close(a, b)


def test_gather_scatter_round_trip_and_identity():
    torch.manual_seed(4)
    x = torch.randn(3, 8, 8, 5)
    idx = torch.stack([torch.randperm(16) for _ in range(3)]).to(torch.int32)
    cells = O.gather_cells(x, idx, 4)
    assert torch.equal(O.scatter_cells(cells, idx), x)
    ident = torch.arange(16, dtype=torch.int32).expand(3, 16).contiguous()
    assert torch.equal(O.gather_cells(x, ident, 4), O.high_to_cells(x, 4))


def test_scatter_add_is_the_adjoint_of_the_gather():
    """Pins oracle.scatter_add_cells: (1) small integers make every fp32 sum exact in any
    order, so it must equal torch's index_add_ (a library scatter-add) bit for bit; (2)
    <gather(x), g> == <x, scatter_add(g)> (the adjoint identity) in float64; (3) for a
    permutation it equals the scatter copy, -0.0 included; (4) unselected states are +0."""
    torch.manual_seed(11)
    b, g, c = 3, 4, 6
    idx = torch.randint(0, g * g, (b, g * g), dtype=torch.int32)
    idx[:, :3] = 5  # a state selected three times in every row
    grad = torch.randint(-8, 9, (b, g * g, 4, c)).float()
    got = O.high_to_cells(O.scatter_add_cells(grad, idx), 4)
    want = torch.zeros(b, g * g, 4, c)
    for r in range(b):
        want[r].index_add_(0, idx[r].long(), grad[r])
    assert torch.equal(got, want)
    x = torch.randn(b, 2 * g, 2 * g, c, dtype=torch.float64)
    gg = torch.randn(b, g * g, 4, c, dtype=torch.float64)
    lhs = (O.gather_cells(x, idx, 4) * gg).sum()
    rhs = (x * O.scatter_add_cells(gg.float(), idx).double()).sum()
    assert abs(float(lhs - rhs)) <= 1e-5 * float(gg.abs().sum())
    perm = torch.stack([torch.randperm(g * g) for _ in range(b)]).to(torch.int32)
    cells = torch.randn(b, g * g, 4, c).to(torch.bfloat16)
    cells[0, 0, 0, 0] = -0.0
    assert torch.equal(O.scatter_add_cells(cells, perm).view(torch.int16),
                       O.scatter_cells(cells, perm).view(torch.int16))
    unselected = torch.ones(g * g, dtype=torch.bool)
    unselected[idx[0].long()] = False
    out0 = O.high_to_cells(O.scatter_add_cells(grad, idx), 4)[0]
    assert unselected.any() and (out0[unselected] == 0).all()
    assert not torch.signbit(out0[unselected]).any()


def test_planted_slot_swap_is_caught(monkeypatch):
    """A mistake planted in the oracle (slots ux/uy transposed) must fail the pins."""
    def swapped(x, slots):
        b, h, w, c = x.shape
        k = O.cell_edge(slots)
        g = h // k
        return x.reshape(b, g, k, g, k, c).permute(0, 1, 3, 4, 2, 5).reshape(b, g * g, k * k, c)

    monkeypatch.setattr(O, "high_to_cells", swapped)
    with pytest.raises(AssertionError):
        test_known_answer_slot_order_and_round_trip()
    # ... and the weight-gradient fixture (weights indexed by slot) disagrees too.
    f = _load("p8_small")
    x = torch.from_numpy(f["x"]).double()
    ups = [torch.from_numpy(u).double() for u in f["updates"]]
    with pytest.raises(AssertionError):
        torch.testing.assert_close(O.weight_grad(x, ups, 4).double(), torch.from_numpy(f["weight_grad"]),
                                   rtol=1e-6, atol=1e-6)
