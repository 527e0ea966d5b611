"""GPU parity of the spatially indexed variant: bit-exact gathers/scatters and
indexed read/write against torch advanced indexing on the CPU oracle."""
from __future__ import annotations

import pytest
import torch

from helpers import announce, assert_parity
from oracle import sihc_oracle as O
from sihc_hip import launch
from sihc_hip.indexed import gather_cells, group_index, indexed_read, indexed_write, scatter_cells
from sihc_hip.sublayer_kernels import sublayer_read, sublayer_write

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("slots,channels", [(4, 67), (4, 64), (16, 24)])
def test_gather_scatter_bit_exact(dtype, slots, channels):
    announce(f"gather/scatter dtype={dtype} slots={slots} C={channels}")
    torch.manual_seed(5)
    k = O.cell_edge(slots)
    x = torch.randn(3, 16 * k, 16 * k, channels, device="cuda", dtype=dtype)
    idx = group_index(3, 16, 5, seed=9).cuda()
    cells = gather_cells(x, idx, slots)
    assert torch.equal(cells.cpu(), O.gather_cells(x.cpu(), idx.cpu(), slots))
    back = scatter_cells(cells, idx)
    assert torch.equal(back, x)  # round trip, bit for bit
    # NaN/Inf payloads are copied untouched
    x2 = x.clone()
    x2.view(-1)[::97] = float("nan")
    x2.view(-1)[5::101] = float("inf")
    c2 = gather_cells(x2, idx, slots)
    assert torch.equal(c2.cpu().view(torch.int16 if dtype == torch.bfloat16 else torch.int32),
                       O.gather_cells(x2.cpu(), idx.cpu(), slots).view(torch.int16 if dtype == torch.bfloat16
                                                                       else torch.int32))


def test_gather_accepts_shared_states_and_rejects_bad_indices():
    announce("gather shared/bad indices")
    x = torch.randn(2, 32, 32, 16, device="cuda")
    idx = torch.randint(0, 256, (2, 256), device="cuda", dtype=torch.int32)  # repeats allowed
    assert torch.equal(gather_cells(x, idx).cpu(), O.gather_cells(x.cpu(), idx.cpu(), 4))
    with pytest.raises(ValueError, match="permutations"):
        scatter_cells(gather_cells(x, idx), idx)
    bad = idx.clone()
    bad[0, 0] = 256
    with pytest.raises(ValueError, match=r"\[0, 256\)"):
        gather_cells(x, bad)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("slots,channels", [(4, 67), (4, 64), (16, 24)])
def test_gather_backward_sums_repeated_states(dtype, slots, channels):
    # The gather accepts repeated indices; its adjoint adds the gradient rows of every
    # token that selected a state (fp32, ascending token order, one rounding) and leaves
    # unselected states at zero. Same summation order as the oracle: bit for bit.
    announce(f"gather backward repeated index dtype={dtype} slots={slots} C={channels}")
    torch.manual_seed(12)
    k = O.cell_edge(slots)
    x = torch.randn(3, 16 * k, 16 * k, channels, device="cuda", dtype=dtype).requires_grad_()
    idx = torch.randint(0, 256, (3, 256), device="cuda", dtype=torch.int32)
    idx[:, 10:20] = 7  # one state selected at least ten times per row
    cells = gather_cells(x, idx, slots)
    g = torch.randn_like(cells)
    (gx,) = torch.autograd.grad(cells, x, g)
    want = O.scatter_add_cells(g.cpu(), idx.cpu())
    assert torch.equal(gx.cpu(), want)
    # cells no token selected receive exactly zero
    unselected = torch.ones(3, 256, dtype=torch.bool)
    unselected[torch.arange(3)[:, None], idx.cpu().long()] = False
    assert unselected.any()
    assert (O.high_to_cells(gx.detach().cpu(), slots)[unselected] == 0).all()
    # a permutation index: the adjoint is the scatter copy, bit for bit
    perm = group_index(3, 16, 5, seed=4).cuda()
    (gp,) = torch.autograd.grad(gather_cells(x, perm, slots), x, g)
    assert torch.equal(gp, scatter_cells(g, perm))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_identity_index_is_bit_identical_to_plain_ops(dtype):
    announce(f"identity index dtype={dtype}")
    torch.manual_seed(6)
    x = torch.randn(2, 32, 32, 64, device="cuda", dtype=dtype)
    a = (0.25 + 0.02 * torch.randn(3, 64, 4, device="cuda")).to(dtype)
    ups = [torch.randn(2, 256, 64, device="cuda", dtype=dtype) for _ in range(3)]
    ident = torch.arange(256, device="cuda", dtype=torch.int32).expand(2, 256).contiguous()
    for z, r in zip(indexed_read(x, a, ident), sublayer_read(x, a)):
        assert torch.equal(z, r)
    assert torch.equal(indexed_write(x, ups, a, ident), sublayer_write(x, ups, a))
    assert torch.equal(launch.weight_grad(x, ups, a, index=ident), launch.weight_grad(x, ups, a))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_indexed_read_write_match_gather_apply_scatter(dtype):
    # Spec: gather each token's state, apply read/write, scatter back.
    announce(f"indexed read/write dtype={dtype}")
    torch.manual_seed(8)
    b, c, events = 4, 72, 2
    x = torch.randn(b, 32, 32, c, device="cuda", dtype=dtype).requires_grad_()
    a = (0.25 + 0.02 * torch.randn(events, c, 4, device="cuda")).to(dtype).requires_grad_()
    beta = (1.0 + 0.02 * torch.randn(events, c, 4, device="cuda")).to(dtype).requires_grad_()
    dz = [torch.randn(b, 256, c, device="cuda", dtype=dtype).requires_grad_() for _ in range(events)]
    idx = group_index(b, 16, 5, seed=3).cuda()
    z = indexed_read(x, a, idx)
    xo = indexed_write(x, dz, beta, idx)
    loss = sum((zi * (i + 1)).sum() for i, zi in enumerate(z)) + (xo * 1e-2 * torch.ones_like(xo)).sum()
    grads = torch.autograd.grad(loss, (x, a, beta, *dz))

    xc, ac, bc = (t.detach().cpu().clone().requires_grad_() for t in (x, a, beta))
    dzc = [t.detach().cpu().clone().requires_grad_() for t in dz]
    ic = idx.cpu()
    cells = O.gather_cells(xc, ic, 4)                 # [B,N,S,C] states in token order
    as_carrier = O.cells_to_high(cells)               # token-ordered carrier
    zr = O.read(as_carrier, ac)
    xr = O.scatter_cells(O.high_to_cells(O.write(as_carrier, dzc, bc), 4), ic)
    rloss = sum((zi * (i + 1)).sum() for i, zi in enumerate(zr)) + (xr * 1e-2).sum()
    rgrads = torch.autograd.grad(rloss, (xc, ac, bc, *dzc))
    for e in range(events):
        assert_parity(z[e], zr[e], dtype, what=f"z[{e}]")
    assert_parity(xo, xr, dtype, what="carrier")
    # grads: x (two events' adjoints added by autograd in bf16 on both sides), alpha and
    # beta (token reductions), the updates (one read each)
    for i, (g, r) in enumerate(zip(grads, rgrads)):
        kind = "chained" if i == 0 else ("reduced" if i in (1, 2) else "elementwise")
        assert_parity(g, r, dtype, what=f"grad[{i}]", kind=kind)
