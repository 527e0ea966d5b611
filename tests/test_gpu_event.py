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


def _offset_copy(t: torch.Tensor) -> torch.Tensor:
    """The same values, stored one element past a 16-byte boundary."""
    buf = torch.empty(t.numel() + 1, device=t.device, dtype=t.dtype)
    out = buf[1:].view(t.shape)
    out.copy_(t)
    return out


@pytest.mark.parametrize("channels,batch,grid", [(8, 3, 7), (1152, 2, 9), (1160, 2, 5), (5776, 1, 3)])
def test_event_forward_whole_row_blocks(channels, batch, grid):
    # 4-slot bf16 cells with 16-byte aligned rows run on whole-row blocks of C/8 lanes and
    # max(1, 720 // (C/8)) tokens: 1 lane x 720 tokens (C=8), 144 x 5 and 145 x 4 with a
    # partial last block (162 and 50 tokens), 722 lanes x 1 token (C=5776). The same call
    # on rows one element off a 16-byte boundary takes the general kernel: same bits.
    announce(f"event fwd whole rows C={channels} batch={batch} grid={grid}")
    torch.manual_seed(channels + grid)
    dt = torch.bfloat16
    x = torch.randn(batch, 2 * grid, 2 * grid, channels, device="cuda", dtype=dt)
    dz = torch.randn(batch, grid * grid, channels, device="cuda", dtype=dt)
    beta = (1.0 + 0.02 * torch.randn(channels, 4, device="cuda")).to(dt)
    alpha = (0.25 + 0.02 * torch.randn(channels, 4, device="cuda")).to(dt)
    x_out, z_out = launch.event_forward(x, dz, beta, alpha)
    rx, rz = O.event_forward(x.cpu(), dz.cpu(), beta.cpu(), alpha.cpu())
    assert_parity(x_out, rx, dt, what="x_out")
    assert_parity(z_out, rz, dt, what="z_out")
    xg, zg = launch.event_forward(_offset_copy(x), _offset_copy(dz), beta, alpha)
    assert torch.equal(xg, x_out) and torch.equal(zg, z_out)
    # a per-image permutation of the grid's cells: every carrier cell is written
    idx = torch.stack([torch.randperm(grid * grid) for _ in range(batch)]).to(torch.int32).cuda()
    xi, zi = launch.event_forward(x, dz, beta, alpha, index=idx)
    xgi, zgi = launch.event_forward(_offset_copy(x), _offset_copy(dz), beta, alpha, index=idx)
    assert torch.equal(xi, xgi) and torch.equal(zi, zgi)


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


def _finalize_chain_case(dtype, slots, n, seed):
    """n per-event backward calls (full, write-only and read-only modes in turn; call
    n // 2 has no tokens) with their per-call results from sihc_event_backward."""
    torch.manual_seed(seed)
    b, c = 3, 136
    k = O.cell_edge(slots)
    x_out = torch.randn(b, 16 * k, 16 * k, c, device="cuda").to(dtype)
    dz = torch.randn(b, 256, c, device="cuda").to(dtype)
    h = 1e-2 * torch.randn_like(x_out)
    g = 1e-2 * torch.randn_like(dz)
    empty = [t[:0] for t in (x_out, dz, h, g)]
    cases = []
    for i in range(n):
        beta = (1.0 + 0.05 * torch.randn(c, slots, device="cuda")).to(dtype)
        alpha = (0.25 + 0.05 * torch.randn(c, slots, device="cuda")).to(dtype)
        xo, d, hh, gg = empty if i == n // 2 else (x_out, dz, h, g)
        mode = ("full", "write", "read")[i % 3]
        args = dict(full=(hh, gg, xo, d, beta, alpha), write=(hh, None, None, d, beta, None),
                    read=(hh, gg, xo, None, None, alpha))[mode]
        ref = launch.event_backward(*args, carrier_like=xo)
        cases.append((mode, xo.shape[0], args, ref))
    return cases, c, k


def _run_partial(L, entry, case, c, k, code, work, info_slot, prev, st, reuse=None):
    import ctypes

    p = lambda t: None if t is None or t.numel() == 0 else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    mode, b, args, ref = case
    outs = [torch.full_like(t, float("nan")) if t is not None else None for t in ref]
    if reuse is not None:  # this call's weight gradients in the given tensors
        outs[2], outs[3] = reuse[2], reuse[3]
    gx = outs[0] if mode != "write" else torch.full_like(ref[0], float("nan"))
    hh, gz, xo, d, bt, al = args
    call = (p(hh), p(gz), p(xo), p(d), p(bt), p(al), p(gx), p(outs[1]), p(outs[2]), p(outs[3]), b, 16, k, c, None,
            code, code, ctypes.c_void_p(work.data_ptr()), work.numel() * 4, info_slot)
    if entry == "chain":
        _lib_check(L.sihc_event_backward_chain(*call, *prev, st))
    else:
        _lib_check(L.sihc_event_backward_partial(*call, st))
    return (gx, *outs[1:])


def _lib_check(rc):
    from sihc_hip import _lib

    _lib.check(rc)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("slots", [4, 16])
def test_deferred_finalize_matches_per_call_finalize(dtype, slots):
    # sihc_event_backward_partial over a chain of 35 events (full, write-only and read-only
    # modes; one event without tokens), then one sihc_event_finalize (two launches: 32 + 3
    # events): every output bit-identical to sihc_event_backward's own finalize.
    import ctypes

    from sihc_hip import _lib

    announce(f"deferred event finalize, 35 events, {dtype}, {slots} slots")
    L = _lib.lib()
    n = 35
    cases, c, k = _finalize_chain_case(dtype, slots, n, seed=41)
    code = _lib.DTYPE_F32 if dtype == torch.float32 else _lib.DTYPE_BF16
    nws = L.sihc_event_backward_workspace_size(3, 16, k, c)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    info = (ctypes.c_int * (2 * n))()
    slot = lambda i: ctypes.cast(ctypes.addressof(info) + 8 * i, ctypes.POINTER(ctypes.c_int))  # noqa: E731
    works, got = [], []
    for i, case in enumerate(cases):
        works.append(torch.empty(nws // 4 + 16, device="cuda", dtype=torch.float32))
        got.append(_run_partial(L, "partial", case, c, k, code, works[-1], slot(i), None, st))
    assert info[2 * (n // 2)] == 0, "the call without tokens leaves no partial rows"
    vp = lambda ts: _lib.ptr_array(None if t is None else t.data_ptr() for t in ts)  # noqa: E731
    _lib.check(L.sihc_event_finalize(n, vp(works), _lib.size_array(w.numel() * 4 for w in works), info,
                                     vp([o[2] for o in got]), vp([o[3] for o in got]), k, c, code, st))
    torch.cuda.synchronize()
    for i, (a, case) in enumerate(zip(got, cases)):
        for j in range(4):
            if case[3][j] is None:
                continue
            assert torch.equal(a[j], case[3][j]), f"event {i} output {j} differs"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("slots", [4, 16])
def test_chained_finalize_matches_per_call_finalize(dtype, slots):
    # sihc_event_backward_chain over a chain of 13 events with two workspaces used in turn:
    # each launch finalizes the previous call's partial rows in its trailing blocks (the
    # call without tokens finalizes its predecessor with a launch of its own), and one
    # sihc_event_finalize ends the chain. Every output bit-identical to sihc_event_backward.
    import ctypes

    from sihc_hip import _lib

    announce(f"chained event finalize, 13 events, {dtype}, {slots} slots")
    L = _lib.lib()
    n = 13
    cases, c, k = _finalize_chain_case(dtype, slots, n, seed=43)
    code = _lib.DTYPE_F32 if dtype == torch.float32 else _lib.DTYPE_BF16
    nws = L.sihc_event_backward_workspace_size(3, 16, k, c)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    info = (ctypes.c_int * (2 * n))()
    slot = lambda i: ctypes.cast(ctypes.addressof(info) + 8 * i, ctypes.POINTER(ctypes.c_int))  # noqa: E731
    works = [torch.full((nws // 4 + 16,), float("nan"), device="cuda") for _ in range(2)]
    got = []
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    for i, case in enumerate(cases):
        prev = (None, 0, None, None, None) if i == 0 else \
            (p(works[(i - 1) % 2]), works[(i - 1) % 2].numel() * 4, slot(i - 1), p(got[-1][2]), p(got[-1][3]))
        got.append(_run_partial(L, "chain", case, c, k, code, works[i % 2], slot(i), prev, st))
    last = works[(n - 1) % 2]
    _lib.check(L.sihc_event_finalize(1, _lib.ptr_array([last.data_ptr()]), _lib.size_array([last.numel() * 4]),
                                     slot(n - 1),
                                     _lib.ptr_array([None if got[-1][2] is None else got[-1][2].data_ptr()]),
                                     _lib.ptr_array([None if got[-1][3] is None else got[-1][3].data_ptr()]),
                                     k, c, code, st))
    torch.cuda.synchronize()
    for i, (a, case) in enumerate(zip(got, cases)):
        for j in range(4):
            if case[3][j] is None:
                continue
            assert torch.equal(a[j], case[3][j]), f"event {i} output {j} differs"


def test_chained_finalize_rejects_overlapping_workspaces():
    import ctypes

    from sihc_hip import _lib

    announce("chained event finalize argument checks")
    L = _lib.lib()
    cases, c, k = _finalize_chain_case(torch.bfloat16, 4, 3, seed=3)  # cases[0]: a full event with tokens
    nws = L.sihc_event_backward_workspace_size(3, 16, k, c)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    info = (ctypes.c_int * 4)()
    slot = lambda i: ctypes.cast(ctypes.addressof(info) + 8 * i, ctypes.POINTER(ctypes.c_int))  # noqa: E731
    work = torch.empty(nws // 4 + 16, device="cuda")
    got = _run_partial(L, "partial", cases[0], c, k, _lib.DTYPE_BF16, work, slot(0), None, st)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    with pytest.raises(_lib.SihcError, match="overlaps this call's workspace"):
        _run_partial(L, "chain", cases[0], c, k, _lib.DTYPE_BF16, work, slot(1),
                     (p(work), work.numel() * 4, slot(0), p(got[2]), p(got[3])), st)
    other = torch.empty_like(work)
    with pytest.raises(_lib.SihcError, match="partial rows need"):
        _run_partial(L, "chain", cases[0], c, k, _lib.DTYPE_BF16, other, slot(1),
                     (p(work), 4096, slot(0), p(got[2]), p(got[3])), st)
    with pytest.raises(_lib.SihcError, match="overlap this call's"):
        _run_partial(L, "chain", cases[0], c, k, _lib.DTYPE_BF16, other, slot(1),
                     (p(work), work.numel() * 4, slot(0), p(got[2]), p(got[3])), st, reuse=got)
    torch.cuda.synchronize()
