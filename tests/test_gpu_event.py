"""GPU parity of the per-event fused write+read (literal schedule) and its adjoint."""
from __future__ import annotations

import pytest
import torch

from helpers import announce, assert_parity
from oracle import sihc_oracle as O
from sihc_hip import launch
from sihc_hip.event_ops import event_write_read, literal_stage

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.bfloat16]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("slots", [4, 16])
@pytest.mark.parametrize("channels", [67, 64])
def test_event_forward_matches_write_then_read(dtype, slots, channels):
    announce(f"event fwd dtype={dtype} slots={slots} C={channels}")
    torch.manual_seed(11)
    k = O.cell_edge(slots)
    x = torch.randn(3, 7 * k, 7 * k, channels, device="cuda", dtype=dtype)
    dz = torch.randn(3, 49, channels, device="cuda", dtype=dtype)
    beta = (1.0 + 0.02 * torch.randn(channels, slots, device="cuda")).to(dtype)
    alpha = (0.25 + 0.02 * torch.randn(channels, slots, device="cuda")).to(dtype)
    x_out, z_out = launch.event_forward(x, dz, beta, alpha)
    rx, rz = O.event_forward(x.cpu(), dz.cpu(), beta.cpu(), alpha.cpu())
    assert_parity(x_out, rx, dtype, what="x_out")
    assert_parity(z_out, rz, dtype, what="z_out")
    # the write half is the E=1 stage write, bit for bit
    assert torch.equal(x_out, launch.write(x, [dz], beta[None]))
    x_only, none = launch.event_forward(x, dz, beta, None)
    assert none is None and torch.equal(x_only, x_out)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("slots", [4, 16])
@pytest.mark.parametrize("has_h,has_g", [(True, True), (False, True), (True, False)])
def test_event_backward_matches_adjoint(dtype, slots, has_h, has_g):
    announce(f"event bwd dtype={dtype} slots={slots} h={has_h} g={has_g}")
    torch.manual_seed(12)
    k = O.cell_edge(slots)
    c = 72
    x_out = torch.randn(4, 9 * k, 9 * k, c, device="cuda", dtype=dtype)
    dz = torch.randn(4, 81, c, device="cuda", dtype=dtype)
    beta = (1.0 + 0.02 * torch.randn(c, slots, device="cuda")).to(dtype)
    alpha = (0.25 + 0.02 * torch.randn(c, slots, device="cuda")).to(dtype)
    h = (1e-2 * torch.randn_like(x_out)) if has_h else None
    g = (1e-2 * torch.randn_like(dz)) if has_g else None
    gx, gdz, gb, ga = launch.event_backward(h, g, x_out, dz, beta, alpha)
    ref = O.event_backward(None if h is None else h.cpu(), None if g is None else g.cpu(), x_out.cpu(),
                           dz.cpu(), beta.cpu(), alpha.cpu())
    assert_parity(gx, ref[0], dtype, what="grad_x")
    assert_parity(gdz, ref[1], dtype, what="grad_dz")
    assert_parity(gb, ref[2], dtype, what="grad_beta", kind="reduced")
    if has_g:
        assert_parity(ga, ref[3], dtype, what="grad_alpha_next", kind="reduced")
    else:
        assert torch.count_nonzero(ga) == 0
    # deterministic reductions
    again = launch.event_backward(h, g, x_out, dz, beta, alpha)
    for a, b in zip((gx, gdz, gb, ga), again):
        assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("slots,batch,grid", [(4, 37, 15), (16, 9, 13)])
def test_event_backward_many_interleaved_chunks(dtype, slots, batch, grid):
    # Tens of reduction chunks, each taking every chunks-th group of 64 tokens; the token
    # count (8325 and 1521) leaves a short last group and the 136 channels a short last
    # channel slice, with a per-batch state permutation.
    announce(f"event bwd chunks dtype={dtype} slots={slots} b={batch} g={grid}")
    torch.manual_seed(31)
    k = O.cell_edge(slots)
    c = 136
    x_out = torch.randn(batch, grid * k, grid * k, c, device="cuda", dtype=dtype)
    dz = torch.randn(batch, grid * grid, c, device="cuda", dtype=dtype)
    beta = (1.0 + 0.02 * torch.randn(c, slots, device="cuda")).to(dtype)
    alpha = (1.0 / slots + 0.02 * torch.randn(c, slots, device="cuda")).to(dtype)
    h = 1e-2 * torch.randn_like(x_out)
    g = 1e-2 * torch.randn_like(dz)
    gen = torch.Generator().manual_seed(5)
    index = torch.stack([torch.randperm(grid * grid, generator=gen) for _ in range(batch)]).to(torch.int32)
    got = launch.event_backward(h, g, x_out, dz, beta, alpha, index=index.cuda())
    cells = lambda t: O.cells_to_high(O.gather_cells(t.cpu(), index, slots))
    ref = O.event_backward(cells(h), g.cpu(), cells(x_out), dz.cpu(), beta.cpu(), alpha.cpu())
    assert_parity(O.cells_to_high(O.gather_cells(got[0].cpu(), index, slots)), ref[0], dtype, what="grad_x")
    for name, a, b in zip(("grad_dz", "grad_beta", "grad_alpha_next"), got[1:], ref[1:]):
        assert_parity(a, b, dtype, what=name, kind="elementwise" if name == "grad_dz" else "reduced")
    again = launch.event_backward(h, g, x_out, dz, beta, alpha, index=index.cuda())
    for a, b in zip(got, again):
        assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("slots", [4, 16])
def test_literal_stage_forward_and_gradients(dtype, slots):
    # Literal per-event schedule on HIP vs the oracle's literal schedule
    # (fusion_controls.py:41-85, "literal") with autograd through both.
    announce(f"literal stage dtype={dtype} slots={slots}")
    torch.manual_seed(21)
    k = O.cell_edge(slots)
    events, c = 6, 40
    x = torch.randn(2, 5 * k, 5 * k, c, device="cuda", dtype=dtype).requires_grad_()
    alpha = (0.25 + 0.05 * torch.randn(events, c, slots, device="cuda")).to(dtype).requires_grad_()
    beta = (1.0 + 0.05 * torch.randn(events, c, slots, device="cuda")).to(dtype).requires_grad_()
    fns = [lambda z, i=i: 0.1 * torch.tanh((1 + 0.1 * i) * z) for i in range(events)]
    out = literal_stage(x, alpha, beta, fns)
    go = torch.randn_like(out) * 0.1
    grads = torch.autograd.grad(out, (x, alpha, beta), go)
    xc, ac, bc = (t.detach().cpu().clone().requires_grad_() for t in (x, alpha, beta))
    ref = O.literal_stage(xc, ac, bc, fns)
    rgrads = torch.autograd.grad(ref, (xc, ac, bc), go.cpu())
    # six events deep: every event's carrier is rounded on both sides, so neighbouring
    # ulps compound
    assert_parity(out, ref, dtype, what="carrier", kind="chained")
    for name, a, b in zip(("dX", "dalpha", "dbeta"), grads, rgrads):
        assert_parity(a, b, dtype, what=name, kind="chained")


def test_event_op_handles_unused_outputs():
    announce("event op unused outputs")
    torch.manual_seed(3)
    x = torch.randn(2, 8, 8, 32, device="cuda", requires_grad=True)
    dz = torch.randn(2, 16, 32, device="cuda", requires_grad=True)
    beta = torch.randn(32, 4, device="cuda", requires_grad=True)
    alpha = torch.randn(32, 4, device="cuda", requires_grad=True)
    x_out, z_out = event_write_read(x, dz, beta, alpha)
    gx, gdz, gb, ga = torch.autograd.grad(z_out.sum(), (x, dz, beta, alpha), retain_graph=True)
    ref = O.event_backward(None, torch.ones(2, 16, 32), x_out.detach().cpu(), dz.detach().cpu(),
                           beta.detach().cpu(), alpha.detach().cpu())
    for a, b in zip((gx, gdz, gb, ga), ref):
        assert_parity(a, b, torch.float32)
    gx2, = torch.autograd.grad(x_out.sum(), (x,))
    assert torch.equal(gx2, torch.ones_like(gx2))


def test_deferred_finalize_matches_per_call_finalize():
    # sihc_event_backward_partial over a chain of 35 events (full, write-only and read-only
    # modes), then one sihc_event_finalize (two launches: 32 + 3 events): every output
    # bit-identical to sihc_event_backward's own finalize.
    import ctypes

    from sihc_hip import _lib

    announce("deferred event finalize, 35 events")
    torch.manual_seed(41)
    L = _lib.lib()
    b, c, slots = 3, 136, 4
    x_out = torch.randn(b, 32, 32, c, device="cuda").to(torch.bfloat16)
    dz = torch.randn(b, 256, c, device="cuda").to(torch.bfloat16)
    h = (1e-2 * torch.randn_like(x_out))
    g = (1e-2 * torch.randn_like(dz))
    nws = L.sihc_event_backward_workspace_size(b, 16, 2, c)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    n = 35
    info = (ctypes.c_int * (2 * n))()
    slot = lambda i: ctypes.cast(ctypes.addressof(info) + 8 * i, ctypes.POINTER(ctypes.c_int))  # noqa: E731
    works, got, ref = [], [], []
    for i in range(n):
        beta = (1.0 + 0.05 * torch.randn(c, slots, device="cuda")).to(torch.bfloat16)
        alpha = (0.25 + 0.05 * torch.randn(c, slots, device="cuda")).to(torch.bfloat16)
        mode = ("full", "write", "read")[i % 3]
        args = dict(full=(h, g, x_out, dz, beta, alpha), write=(h, None, None, dz, beta, None),
                    read=(h, g, x_out, None, None, alpha))[mode]
        ref.append(launch.event_backward(*args, carrier_like=x_out))
        outs = [torch.full_like(t, float("nan")) if t is not None else None for t in ref[-1]]
        gx = outs[0] if mode != "write" else torch.full_like(x_out, float("nan"))
        work = torch.empty(nws // 4 + 16, device="cuda", dtype=torch.float32)
        works.append(work)
        hh, gz, xo, d, bt, al = args
        _lib.check(L.sihc_event_backward_partial(p(hh), p(gz), p(xo), p(d), p(bt), p(al), p(gx), p(outs[1]),
                                                 p(outs[2]), p(outs[3]), b, 16, 2, c, None, 1, 1, p(work),
                                                 work.numel() * 4, slot(i), st))
        got.append((gx, *outs[1:]))
    vp = lambda ts: _lib.ptr_array(None if t is None else t.data_ptr() for t in ts)  # noqa: E731
    _lib.check(L.sihc_event_finalize(n, vp(works), info, vp([o[2] for o in got]), vp([o[3] for o in got]),
                                     2, c, 1, st))
    torch.cuda.synchronize()
    for i, (a, r) in enumerate(zip(got, ref)):
        for k in range(4):
            if r[k] is None:
                continue
            assert torch.equal(a[k], r[k]), f"event {i} output {k} differs"
