"""GPU: the HIP-backed ops under fullgraph torch.compile and HIP-graph capture.

Mirrors the reference's compile and graph contracts (research/tests/
test_sublayer_kernels.py:187-213, :268-286; test_runtime_compatibility.py:102-151):
the custom ops trace through their fake implementations with no graph break, their
autograd rules run under AOTAutograd, and captured launches replay correctly. The
compile backend is aot_eager (tracing, functionalisation and AOT autograd without
generating any kernels), so the only device code that runs is this library's.
"""
from __future__ import annotations

import pytest
import torch

from helpers import announce, assert_parity
from sihc_hip.event_ops import event_write_read, literal_stage
from sihc_hip.sublayer_kernels import sublayer_read, sublayer_triangular, sublayer_write

pytestmark = pytest.mark.gpu


def stage(x, alpha, beta):
    """The reference's fused stage schedule (sublayer.py:52-72) with tanh bodies."""
    events = alpha.shape[0]
    base = sublayer_read(x, alpha)
    gamma = (alpha[:, None] * beta[None, :]).sum(-1)
    updates = []
    for i in range(events):
        z = base[i] if i == 0 else sublayer_triangular(base[i], updates, gamma[i, :i].contiguous())
        updates.append((0.05 * torch.tanh(z)).contiguous())
    return sublayer_write(x, updates, beta)


def _inputs(dtype, events=8, slots=4, c=64, seed=0):
    torch.manual_seed(seed)
    k = 2 if slots == 4 else 4
    x = torch.randn(2, 4 * k, 4 * k, c, device="cuda", dtype=dtype)
    alpha = (0.25 + 0.05 * torch.randn(events, c, slots, device="cuda")).to(dtype)
    beta = (1.0 + 0.05 * torch.randn(events, c, slots, device="cuda")).to(dtype)
    return x, alpha, beta


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fullgraph_compile_of_stage_forward_backward(dtype):
    announce(f"compile stage dtype={dtype}")
    torch._dynamo.reset()
    x, alpha, beta = _inputs(dtype)
    leaves = [t.clone().requires_grad_() for t in (x, alpha, beta)]
    eager = stage(*leaves)
    go = torch.randn_like(eager) * 0.1
    ge = torch.autograd.grad(eager, leaves, go)
    compiled = torch.compile(stage, backend="aot_eager", fullgraph=True)
    leaves2 = [t.clone().requires_grad_() for t in (x, alpha, beta)]
    out = compiled(*leaves2)
    gc = torch.autograd.grad(out, leaves2, go)
    assert torch.equal(out, eager)
    # the traced backward may add the autograd contributions in another order
    for a, b in zip(gc, ge):
        assert_parity(a, b, dtype, kind="chained")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fullgraph_compile_of_literal_stage(dtype):
    announce(f"compile literal dtype={dtype}")
    torch._dynamo.reset()
    x, alpha, beta = _inputs(dtype, events=5)
    fns = [lambda z, i=i: 0.1 * torch.tanh((1 + 0.1 * i) * z) for i in range(5)]

    def fn(x, a, b):
        return literal_stage(x, a, b, fns)

    leaves = [t.clone().requires_grad_() for t in (x, alpha, beta)]
    eager = fn(*leaves)
    go = torch.randn_like(eager) * 0.1
    ge = torch.autograd.grad(eager, leaves, go)
    leaves2 = [t.clone().requires_grad_() for t in (x, alpha, beta)]
    out = torch.compile(fn, backend="aot_eager", fullgraph=True)(*leaves2)
    gc = torch.autograd.grad(out, leaves2, go)
    assert torch.equal(out, eager)
    for a, b in zip(gc, ge):
        assert_parity(a, b, dtype, kind="chained")


def test_hip_graph_capture_and_replay_of_stage_forward():
    announce("hip graph stage forward")
    x, alpha, beta = _inputs(torch.bfloat16, events=12, seed=1)
    static_x = x.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm up allocations outside the capture
        for _ in range(2):
            stage(static_x, alpha, beta)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = stage(static_x, alpha, beta)
    for r in range(4):
        fresh = torch.randn_like(x) * (1 + r)
        static_x.copy_(fresh)
        graph.replay()
        # eager work and a synchronisation between replays
        expected = stage(fresh, alpha, beta)
        torch.cuda.synchronize()
        assert torch.equal(static_out, expected), f"replay {r} differs from eager"


def test_hip_graph_capture_of_event_backward_chain():
    announce("hip graph event fwd+bwd")
    x, alpha, beta = _inputs(torch.bfloat16, events=3, seed=2)
    dz = torch.randn(2, 16, 64, device="cuda", dtype=torch.bfloat16)
    static = [t.clone().requires_grad_() for t in (x, dz)]
    g_x = 1e-2 * torch.randn_like(x)
    g_z = 1e-2 * torch.randn_like(dz)

    def run(xx, dd):
        # upstream gradients are given, so no reduction kernel is captured
        xo, zo = event_write_read(xx, dd, beta[0], alpha[1])
        return torch.autograd.grad((xo, zo), (xx, dd), (g_x, g_z))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            run(*static)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gx, gd = run(*static)
    for r in range(3):
        nx, nd = torch.randn_like(x), torch.randn_like(dz)
        with torch.no_grad():
            static[0].copy_(nx)
            static[1].copy_(nd)
        graph.replay()
        ex, ed = run(nx.clone().requires_grad_(), nd.clone().requires_grad_())
        torch.cuda.synchronize()
        assert torch.equal(gx, ex) and torch.equal(gd, ed), f"replay {r} differs from eager"


def test_hip_graph_capture_of_a_cold_weight_gradient():
    # The pipelined weight-gradient kernel sizes its grid from an occupancy query (host
    # side, cached per kernel shape) on the first launch of a shape. Here that first
    # launch happens inside the capture: the replays must match eager calls bit for bit.
    announce("hip graph weight gradient, first launch of its shape inside the capture")
    torch.manual_seed(5)
    from sihc_hip import launch

    x = torch.randn(2, 32, 32, 72, device="cuda").to(torch.bfloat16)  # 4-slot cells, 13 events
    ups = [torch.randn(2, 256, 72, device="cuda").to(torch.bfloat16) for _ in range(13)]
    w = torch.randn(13, 72, 4, device="cuda").to(torch.bfloat16)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = launch.weight_grad(x, ups, w, out_dtype=torch.float32)
    for r in range(3):
        with torch.no_grad():
            x.copy_(torch.randn_like(x.float()).to(torch.bfloat16))
        graph.replay()
        expected = launch.weight_grad(x, ups, w, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert torch.equal(static_out, expected), f"replay {r} differs from eager"


def test_hip_graph_capture_of_a_chained_event_backward():
    # Three per-event backwards as the benchmark step launches them -- a deferred call,
    # two chained calls each finalizing its predecessor's partial rows in its trailing
    # blocks, then the last call's finalize -- captured into one HIP graph (no memset is
    # recorded: every partial row is written before it is read) and replayed with fresh
    # inputs and eager work in between: every replay bit-equal to the eager chain.
    import ctypes

    from sihc_hip import _lib

    announce("hip graph chained event backward")
    torch.manual_seed(7)
    L = _lib.lib()
    b, c, n = 2, 72, 3
    bf = torch.bfloat16
    x_out = torch.randn(b, 32, 32, c, device="cuda").to(bf)
    dz = [torch.randn(b, 256, c, device="cuda").to(bf) for _ in range(n)]
    h = (1e-2 * torch.randn(b, 32, 32, c, device="cuda")).to(bf)
    gz = (1e-2 * torch.randn(b, 256, c, device="cuda")).to(bf)
    beta = [(1.0 + 0.05 * torch.randn(c, 4, device="cuda")).to(bf) for _ in range(n)]
    alpha = [(0.25 + 0.05 * torch.randn(c, 4, device="cuda")).to(bf) for _ in range(n)]
    nws = L.sihc_event_backward_workspace_size(b, 16, 2, c)
    works = [torch.empty(nws // 4 + 16, device="cuda") for _ in range(2)]
    info = (ctypes.c_int * (2 * n))()
    slot = lambda i: ctypes.cast(ctypes.addressof(info) + 8 * i, ctypes.POINTER(ctypes.c_int))  # noqa: E731
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731

    def outputs():
        return ([torch.empty_like(x_out) for _ in range(n)], [torch.empty_like(dz[0]) for _ in range(n)],
                [torch.empty_like(beta[0]) for _ in range(n)], [torch.empty_like(alpha[0]) for _ in range(n)])

    def chain(out):
        gx, gdz, gb, ga = out
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for i in range(n):
            args = (p(h), p(gz), p(x_out), p(dz[i]), p(beta[i]), p(alpha[i]), p(gx[i]), p(gdz[i]), p(gb[i]),
                    p(ga[i]), b, 16, 2, c, None, _lib.DTYPE_BF16, _lib.DTYPE_BF16, p(works[i % 2]),
                    works[i % 2].numel() * 4, slot(i))
            if i == 0:
                _lib.check(L.sihc_event_backward_partial(*args, st))
            else:
                prev = works[(i - 1) % 2]
                _lib.check(L.sihc_event_backward_chain(*args, p(prev), prev.numel() * 4, slot(i - 1), p(gb[i - 1]),
                                                       p(ga[i - 1]), st))
        last = works[(n - 1) % 2]
        _lib.check(L.sihc_event_finalize(1, _lib.ptr_array([last.data_ptr()]), _lib.size_array([last.numel() * 4]),
                                         slot(n - 1), _lib.ptr_array([gb[-1].data_ptr()]),
                                         _lib.ptr_array([ga[-1].data_ptr()]), 2, c, _lib.DTYPE_BF16, st))

    static = outputs()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        chain(static)  # warm-up: occupancy queries and info slots
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        chain(static)
    for r in range(3):
        with torch.no_grad():
            h.copy_((1e-2 * torch.randn_like(h.float())).to(bf))
            gz.copy_((1e-2 * torch.randn_like(gz.float())).to(bf))
        graph.replay()
        eager = outputs()
        chain(eager)  # eager work between the replays
        torch.cuda.synchronize()
        for k, (a_list, e_list) in enumerate(zip(static, eager)):
            for i, (a, e) in enumerate(zip(a_list, e_list)):
                assert torch.equal(a, e), f"replay {r}: output {k} of event {i} differs from eager"
