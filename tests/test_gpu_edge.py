"""GPU edge cases: empty batches, NaN/Inf propagation, misaligned (but packed) views
that force the scalar path, and the 16-slot cell at a larger shape."""
from __future__ import annotations

import pytest
import torch

from helpers import announce, assert_parity
from oracle import sihc_oracle as O
from sihc_hip import launch
from sihc_hip.sublayer_kernels import sublayer_read, sublayer_triangular, sublayer_write

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_empty_batch(dtype):
    announce(f"empty batch dtype={dtype}")
    x = torch.empty(0, 32, 32, 64, device="cuda", dtype=dtype, requires_grad=True)
    a = torch.randn(3, 64, 4, device="cuda", dtype=dtype, requires_grad=True)
    b = torch.randn(3, 64, 4, device="cuda", dtype=dtype, requires_grad=True)
    zs = sublayer_read(x, a)
    assert all(z.shape == (0, 256, 64) for z in zs)
    out = sublayer_write(x, [z.detach().requires_grad_() for z in zs], b)
    assert out.shape == x.shape
    ga, = torch.autograd.grad(sum(z.sum() for z in zs), (a,))
    assert ga.shape == a.shape and torch.count_nonzero(ga) == 0
    assert torch.count_nonzero(launch.weight_grad(x.detach(), [zz.detach() for zz in zs], b)) == 0
    base = torch.empty(0, 256, 64, device="cuda", dtype=dtype)
    assert sublayer_triangular(base, [base], torch.ones(1, 64, device="cuda")).shape == base.shape
    gg = launch.triangular_gamma_grad(base, [base, base], torch.ones(2, 64, device="cuda", dtype=dtype))
    assert torch.count_nonzero(gg) == 0
    beta1 = torch.randn(64, 4, device="cuda", dtype=dtype)
    xo, zo = launch.event_forward(x.detach(), base, beta1, beta1)
    assert xo.shape == x.shape and zo.shape == base.shape
    gx, gdz, gb, gaa = launch.event_backward(None, base, xo, base, beta1, beta1)
    assert torch.count_nonzero(gb) == 0 and torch.count_nonzero(gaa) == 0


def test_nan_and_inf_propagate_like_the_oracle():
    announce("nan/inf propagation")
    torch.manual_seed(3)
    x = torch.randn(2, 8, 8, 64, device="cuda")
    x[0, 0, 0, 3] = float("nan")
    x[1, 5, 6, 10] = float("inf")
    a = torch.randn(2, 64, 4, device="cuda")
    ups = [torch.randn(2, 16, 64, device="cuda") for _ in range(2)]
    ups[1][0, 2, 7] = float("-inf")
    for got, exp in zip(sublayer_read(x, a), O.read(x.cpu(), a.cpu())):
        assert torch.equal(torch.isnan(got).cpu(), torch.isnan(exp))
        assert torch.equal(torch.isinf(got).cpu(), torch.isinf(exp))
    got, exp = sublayer_write(x, ups, a), O.write(x.cpu(), [u.cpu() for u in ups], a.cpu())
    assert torch.equal(torch.isnan(got).cpu(), torch.isnan(exp))
    assert torch.equal(torch.isinf(got).cpu(), torch.isinf(exp))
    fin = torch.isfinite(exp)
    assert torch.allclose(got.cpu()[fin], exp[fin], rtol=1e-5, atol=1e-5)
    # bf16 NaN outputs are quiet NaNs (the hardware conversion keeps the sign and top
    # payload bits of the NaN that produced them; torch canonicalises to 0x7fc0)
    xb = x.to(torch.bfloat16)
    zb = sublayer_read(xb, a.to(torch.bfloat16))[0]
    nan_bits = zb.view(torch.int16)[torch.isnan(zb)].int() & 0x7FC0
    assert nan_bits.numel() > 0 and torch.all(nan_bits == 0x7FC0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_misaligned_packed_views_take_the_scalar_path(dtype):
    # Contiguous tensors at an odd element offset: no vector width is legal, every
    # kernel must fall back to one element per lane and stay exact.
    announce(f"misaligned views dtype={dtype}")
    torch.manual_seed(4)
    c = 64
    buf = torch.randn(2 * 8 * 8 * c + 1, device="cuda", dtype=dtype)
    x = buf[1:].view(2, 8, 8, c)
    assert x.is_contiguous() and x.data_ptr() % 16 != 0
    a = (0.25 + 0.05 * torch.randn(3, c, 4, device="cuda")).to(dtype)
    zb = torch.randn(3 * 2 * 16 * c + 1, device="cuda", dtype=dtype)
    ups = [zb[1 + i * 2 * 16 * c: 1 + (i + 1) * 2 * 16 * c].view(2, 16, c) for i in range(3)]
    for got, exp in zip(sublayer_read(x, a), O.read(x.cpu(), a.cpu())):
        assert_parity(got, exp, dtype, what="read")
    assert_parity(sublayer_write(x, ups, a), O.write(x.cpu(), [u.cpu() for u in ups], a.cpu()), dtype, what="write")
    assert_parity(launch.weight_grad(x, ups, a), O.weight_grad(x.cpu(), [u.cpu() for u in ups], 4).to(dtype), dtype,
                  what="weight grad", kind="reduced")
    g = torch.randn(2, c, device="cuda")
    assert_parity(sublayer_triangular(ups[0], ups[1:], g),
                  O.triangular_torch(ups[0].cpu(), [u.cpu() for u in ups[1:]], g.cpu()), dtype, what="triangular")
    xo, zo = launch.event_forward(x, ups[0], a[0], a[1])
    rx, rz = O.event_forward(x.cpu(), ups[0].cpu(), a[0].cpu(), a[1].cpu())
    assert_parity(xo, rx, dtype, what="event x_out")
    assert_parity(zo, rz, dtype, what="event z_out")


def test_sixteen_slot_cells_at_batch_32():
    # p4 geometry (4x4 cells, 64x64 carrier) at a larger shape: read, write and the
    # per-event pair against the oracle on batch slices.
    announce("p4 batch 32")
    torch.manual_seed(5)
    bf = torch.bfloat16
    x = torch.randn(32, 64, 64, 256, device="cuda").to(bf)
    a = (1 / 16 + 0.01 * torch.randn(12, 256, 16, device="cuda")).to(bf)
    b = (1.0 + 0.02 * torch.randn(12, 256, 16, device="cuda")).to(bf)
    zs = sublayer_read(x, a)
    ref = O.read(x[:2].cpu(), a.cpu())
    for e in (0, 11):
        assert_parity(zs[e][:2], ref[e], bf, what=f"p4 read {e}")
    ups = [torch.randn(32, 256, 256, device="cuda").to(bf) for _ in range(12)]
    out = sublayer_write(x, ups, b)
    assert_parity(out[-2:], O.write(x[-2:].cpu(), [u[-2:].cpu() for u in ups], b.cpu()), bf, what="p4 write")
    xo, zo = launch.event_forward(x, ups[0], b[0], a[1])
    rx, rz = O.event_forward(x[:2].cpu(), ups[0][:2].cpu(), b[0].cpu(), a[1].cpu())
    assert_parity(xo[:2], rx, bf, what="p4 event x_out")
    assert_parity(zo[:2], rz, bf, what="p4 event z_out")
    wg = launch.weight_grad(x, ups, a)
    exp = O.weight_grad(x[:, :, :, :32].cpu(), [u[:, :, :32].cpu() for u in ups], 16)
    assert_parity(wg[:, :32], exp.to(bf), bf, what="p4 weight grad (channel slice)", kind="reduced")


STREAM_CASES = [(0, 1, 0), (1, 1, 0), (2, 1, 0), (2, 2, 0), (4, 2, 0), (2, 2, 1), (4, 2, 2)]


@pytest.mark.parametrize("nr,nw,shape", STREAM_CASES, ids=[f"{r}:{w}-shape{s}" for r, w, s in STREAM_CASES])
def test_stream_calibration_kernel(nr, nw, shape):
    # sihc_stream (the HBM ceiling the bench reports). Unit u (4 KB of a workspace-shaped
    # array, 16 KB of a carrier-shaped one), thread t: acc = {u, t, 0, 0} XOR every vector
    # the thread loads (vector u*256 + t of a workspace-shaped source, u*1024 + q*256 + t,
    # q < 4, of a carrier-shaped one); destination j gets acc ^ j, or acc ^ (4j + q) for
    # carrier-shaped ones. Shapes 1 and 2: the first source(s) and the first destination
    # are carrier-shaped (1 and 2 carrier sources).
    import ctypes

    from sihc_hip import _lib

    announce(f"stream calibration {nr}:{nw} shape {shape}")
    L = _lib.lib()
    units = 37
    n = 4096 * units
    r4 = {0: 0, 1: 1, 2: 2}[shape]
    w4 = 0 if shape == 0 else 1
    g = torch.Generator(device="cuda").manual_seed(nr * 10 + nw + 100 * shape)
    rint = lambda m: torch.randint(0, 2 ** 31 - 1, (m * n // 4,), device="cuda", generator=g, dtype=torch.int32)  # noqa
    srcs = [rint(4 if r < r4 else 1) for r in range(nr)]
    dsts = [torch.zeros((4 if w < w4 else 1) * n // 4, device="cuda", dtype=torch.int32) for w in range(nw)]
    sp = (ctypes.c_void_p * max(nr, 1))(*[t.data_ptr() for t in srcs])
    dp = (ctypes.c_void_p * nw)(*[t.data_ptr() for t in dsts])
    _lib.check(L.sihc_stream(sp, nr, dp, nw, n, shape, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    acc = torch.zeros(units, 256, 4, device="cuda", dtype=torch.int32)
    acc[:, :, 0] = torch.arange(units, device="cuda", dtype=torch.int32)[:, None]
    acc[:, :, 1] = torch.arange(256, device="cuda", dtype=torch.int32)[None, :]
    for r, t in enumerate(srcs):
        if r < r4:
            for q in range(4):
                acc ^= t.view(units, 4, 256, 4)[:, q]
        else:
            acc ^= t.view(units, 256, 4)
    for j, d in enumerate(dsts):
        if j < w4:
            for q in range(4):
                assert torch.equal(d.view(units, 4, 256, 4)[:, q], acc ^ (4 * j + q)), f"output {j} slot {q}"
        else:
            assert torch.equal(d.view(units, 256, 4), acc ^ j), f"output {j}"


# (sources, carrier-shaped sources, destinations, carrier-shaped destinations, slots): the
# mixes of a 16-slot read and write, a read-only weight gradient (sink), the triangular op
# and its fused backward, a write-only mix, and 9-17 vectors (two and three load batches)
MIX_CASES = [(1, 1, 5, 0, 16), (3, 1, 1, 1, 16), (9, 1, 0, 0, 4), (13, 0, 1, 0, 1), (12, 0, 11, 0, 1),
             (0, 0, 2, 1, 4), (2, 2, 3, 2, 4), (32, 0, 32, 0, 1)]


@pytest.mark.parametrize("ns,ncs,nd,ncd,slots", MIX_CASES,
                         ids=[f"{a}c{b}-{c}c{d}-s{e}" for a, b, c, d, e in MIX_CASES])
def test_stream_mix_kernel(ns, ncs, nd, ncd, slots):
    # sihc_stream_mix: unit u, thread t: acc = {u, t, 0, 0} XOR every source vector of the
    # thread (vector u*256 + t of a workspace-shaped source, (u*slots + q)*256 + t of a
    # carrier-shaped one); destination w gets acc ^ (w*slots + q) (carrier-shaped) or acc ^ w;
    # with no destination each wave's XOR over its 64 lanes lands in sink[u*4 + wave].
    import ctypes

    from sihc_hip import _lib

    announce(f"stream mix {ns}({ncs}):{nd}({ncd}) slots {slots}")
    L = _lib.lib()
    units = 37
    n = 4096 * units
    g = torch.Generator(device="cuda").manual_seed(ns * 100 + nd * 10 + slots)
    rint = lambda m: torch.randint(0, 2 ** 31 - 1, (m * n // 4,), device="cuda", generator=g, dtype=torch.int32)  # noqa
    srcs = [rint(slots if r < ncs else 1) for r in range(ns)]
    dsts = [torch.zeros((slots if w < ncd else 1) * n // 4, device="cuda", dtype=torch.int32) for w in range(nd)]
    sink = torch.zeros(units * 4 * 4, device="cuda", dtype=torch.int32)
    sp = (ctypes.c_void_p * max(ns, 1))(*[t.data_ptr() for t in srcs])
    dp = (ctypes.c_void_p * max(nd, 1))(*[t.data_ptr() for t in dsts])
    _lib.check(L.sihc_stream_mix(sp, ns, ncs, dp, nd, ncd, slots, n, ctypes.c_void_p(sink.data_ptr()),
                                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    acc = torch.zeros(units, 256, 4, device="cuda", dtype=torch.int32)
    acc[:, :, 0] = torch.arange(units, device="cuda", dtype=torch.int32)[:, None]
    acc[:, :, 1] = torch.arange(256, device="cuda", dtype=torch.int32)[None, :]
    for r, t in enumerate(srcs):
        if r < ncs:
            for q in range(slots):
                acc ^= t.view(units, slots, 256, 4)[:, q]
        else:
            acc ^= t.view(units, 256, 4)
    for w, d in enumerate(dsts):
        if w < ncd:
            for q in range(slots):
                assert torch.equal(d.view(units, slots, 256, 4)[:, q], acc ^ (w * slots + q)), f"output {w} slot {q}"
        else:
            assert torch.equal(d.view(units, 256, 4), acc ^ w), f"output {w}"
    if nd == 0:
        waves = acc.view(units, 4, 64, 4)
        red = waves[:, :, 0]
        for lane in range(1, 64):
            red = red ^ waves[:, :, lane]
        assert torch.equal(sink.view(units, 4, 4), red), "sink"
    else:
        assert not sink.any(), "the sink is written only by read-only mixes"


@pytest.mark.parametrize("form", [0, 1, 2, 3], ids=["fma-reg", "fma-literal", "dot2", "fmac"])
@pytest.mark.parametrize("chains", [4, 8, 16])
def test_fma_rate_kernel(chains, form):
    # sihc_fma_rate (the vector-ALU calibration bench.py --mode valu times): thread t of any
    # block starts chain k at t * 1e-3 + k, applies a = fma(a, 1.0000001, 1e-7) (forms 0, 1)
    # or a += (0.5, 0.25) . (0.5, 0.5) = 0.375 (form 2, a bf16 pair dot) or a = fma(1.0000001,
    # 1e-7, a) (form 3, the accumulating form) 4 x iters times, and
    # stores the sum of its chains. Checked against a float64 replay rounded to float32 after
    # every step (the kernel's single rounding may differ in the last bit).
    import ctypes

    import numpy as np

    from sihc_hip import _lib

    announce(f"fma rate kernel chains={chains} form={form}")
    blocks, iters = 3, 5
    out = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
    _lib.check(_lib.lib().sihc_fma_rate(ctypes.c_void_p(out.data_ptr()), chains, form, blocks, iters,
                                        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    t = np.arange(256, dtype=np.float64)
    a = np.stack([np.float32(t * 1e-3 + k) for k in range(chains)]).astype(np.float64)
    for _ in range(4 * iters):
        if form == 2:
            a = (a + 0.375).astype(np.float32).astype(np.float64)
        elif form == 3:
            a = (a + np.float64(np.float32(1.0000001)) * np.float64(np.float32(1e-7))).astype(np.float32).astype(np.float64)
        else:
            a = (a * np.float64(np.float32(1.0000001)) + np.float64(np.float32(1e-7))).astype(np.float32).astype(np.float64)
    exp = torch.from_numpy(a.sum(axis=0).astype(np.float32)).repeat(blocks)
    got = out.cpu()
    assert torch.allclose(got, exp, rtol=1e-6, atol=0), (got - exp).abs().max()
