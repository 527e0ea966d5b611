"""GPU parity of the drop-in `sihc::` ops (HIP kernels through the C ABI) against
the CPU oracle (the reference's unfused PyTorch path, restated in oracle/).

Mirrors the reference's kernel tests (research/tests/test_sublayer_kernels.py,
test_blockwise_tuple_kernels.py) with the tier's parity bar (tests/helpers.py).
"""
from __future__ import annotations

import pytest
import torch

from helpers import announce, assert_parity, rel_l2
from oracle import sihc_oracle as O
from sihc_hip import launch
from sihc_hip.blockwise_kernels import blockwise_read, blockwise_triangular, blockwise_write
from sihc_hip.sublayer_kernels import (_tri_gamma_backward, _weights_backward, _write_impl, sublayer_read,
                                       sublayer_triangular, sublayer_write)

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.bfloat16]


def _cpu_leaf(t):
    return t.detach().cpu().clone().requires_grad_()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("slots", [4, 16])
@pytest.mark.parametrize("events", [1, 8, 24, 32])
def test_read_and_adjoint_with_token_and_channel_tails(dtype, slots, events):
    # M=147 tokens and C=67 channels cross every tile boundary (reference :128-143).
    announce(f"read tails dtype={dtype} slots={slots} events={events}")
    torch.manual_seed(317)
    k = O.cell_edge(slots)
    x = torch.randn(3, 7 * k, 7 * k, 67, device="cuda", dtype=dtype).requires_grad_()
    alpha = (torch.randn(events, 67, slots, device="cuda", dtype=dtype) * 0.05).requires_grad_()
    out = sublayer_read(x, alpha)
    up = [torch.randn(3, 49, 67, device="cuda", dtype=dtype) * 0.1 for _ in range(events)]
    gx, ga = torch.autograd.grad(sum((z * u).sum() for z, u in zip(out, up)), (x, alpha))
    torch.cuda.synchronize()
    xc, ac = _cpu_leaf(x), _cpu_leaf(alpha)
    ref = O.read(xc, ac)
    rgx, rga = torch.autograd.grad(sum((z * u.cpu()).sum() for z, u in zip(ref, up)), (xc, ac))
    for e in range(events):
        assert_parity(out[e], ref[e], dtype, what=f"z[{e}]")
    # the oracle's autograd rounds each event's contribution to dX and adds them in bf16;
    # the kernel sums all events in fp32 and rounds once, so it is checked against the
    # exact (float64) adjoint sum_e alpha_e * up_e at the 1-ulp bar
    assert_parity(gx, rgx, dtype, what="dX vs oracle autograd", kind="elementwise" if events == 1 else "chained")
    exact = O.write(xc.detach().double(), [u.cpu().double() for u in up], ac.detach().double(), add_x=False)
    assert_parity(gx, exact, dtype, what="dX vs exact adjoint")
    assert_parity(ga, rga, dtype, what="dalpha", kind="reduced")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("slots", [4, 16])
@pytest.mark.parametrize("events", [1, 8, 12, 16, 24])
def test_write_forward_and_adjoint(dtype, slots, events):
    # M=363 tokens, C=67 channels (reference test_blockwise_tuple_kernels.py:182-213).
    announce(f"write dtype={dtype} slots={slots} events={events}")
    torch.manual_seed(291)
    k = O.cell_edge(slots)
    x = torch.randn(3, 11 * k, 11 * k, 67, device="cuda", dtype=dtype).requires_grad_()
    ups = [torch.randn(3, 121, 67, device="cuda", dtype=dtype).requires_grad_() for _ in range(events)]
    beta = (torch.randn(events, 67, slots, device="cuda", dtype=dtype) * 0.05).requires_grad_()
    out = sublayer_write(x, ups, beta)
    go = torch.randn_like(out) * 0.03
    grads = torch.autograd.grad(out, (x, *ups, beta), go)
    torch.cuda.synchronize()
    xc, bc = _cpu_leaf(x), _cpu_leaf(beta)
    uc = [_cpu_leaf(u) for u in ups]
    ref = O.write(xc, uc, bc)
    rgrads = torch.autograd.grad(ref, (xc, *uc, bc), go.cpu())
    assert_parity(out, ref, dtype, what="X'")
    assert grads[0].data_ptr() == go.data_ptr() or torch.equal(grads[0], go)  # identity carry
    for i, (a, b) in enumerate(zip(grads, rgrads)):
        assert_parity(a, b, dtype, what=f"grad[{i}]", kind="reduced" if i == events + 1 else "elementwise")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("active", [1, 3, 7, 11, 23])
@pytest.mark.parametrize("gamma_fp32", [True, False])
def test_triangular_forward_and_gradients(dtype, active, gamma_fp32):
    # reference :187-213 and test_blockwise_tuple_kernels.py:232-251
    announce(f"triangular dtype={dtype} active={active} gamma_fp32={gamma_fp32}")
    torch.manual_seed(583)
    base = torch.randn(3, 49, 67, device="cuda", dtype=dtype).requires_grad_()
    ups = [torch.randn_like(base).requires_grad_() for _ in range(active)]
    gdt = torch.float32 if gamma_fp32 else dtype
    gamma = (torch.randn(active, 67, device="cuda", dtype=gdt) * 0.05).requires_grad_()
    out = sublayer_triangular(base, ups, gamma)
    loss = out.float().square().mean() + sum(u.float().square().mean() for u in ups)
    grads = torch.autograd.grad(loss, (base, *ups, gamma))
    torch.cuda.synchronize()
    bc, gc = _cpu_leaf(base), _cpu_leaf(gamma)
    uc = [_cpu_leaf(u) for u in ups]
    ref = O.triangular_torch(bc, uc, gc)
    rloss = ref.float().square().mean() + sum(u.float().square().mean() for u in uc)
    rgrads = torch.autograd.grad(rloss, (bc, *uc, gc))
    assert_parity(out, ref, dtype, what="tri")
    for i, (a, b) in enumerate(zip(grads, rgrads)):
        # update gradients: the triangular term plus the square-mean term, added in bf16
        # by autograd on both sides; gamma: a reduction over tokens
        kind = "elementwise" if i == 0 else ("chained" if i < active + 1 else "reduced")
        assert_parity(a, b, dtype if i < active + 1 else gdt, what=f"grad[{i}]", kind=kind)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("slots", [4, 16])
@pytest.mark.parametrize("events", [16, 24])
def test_fused_stage_schedule_and_all_gradients(dtype, slots, events):
    # The reference's stage schedule (sublayer.py:52-72) on HIP ops vs the same schedule
    # on the oracle ops; fp32 also against the literal dense recurrence (:79-108).
    announce(f"stage dtype={dtype} slots={slots} events={events}")
    torch.manual_seed(92)
    k = O.cell_edge(slots)
    x = torch.randn(2, 4 * k, 4 * k, 37, device="cuda", dtype=dtype).requires_grad_()
    alpha = (torch.randn(events, 37, slots, device="cuda", dtype=dtype) * 0.07).requires_grad_()
    beta = (torch.randn_like(alpha) * 0.07).requires_grad_()

    def stage(x, alpha, beta, read, tri, write):
        base = read(x, alpha)
        gamma = (alpha[:, None] * beta[None, :]).sum(-1)
        updates = []
        for i in range(events):
            z = base[i] if i == 0 else tri(base[i], updates, gamma[i, :i].contiguous())
            updates.append((0.05 * z.tanh()).contiguous())
        return write(x, updates, beta)

    out = stage(x, alpha, beta, sublayer_read, sublayer_triangular, sublayer_write)
    go = torch.randn_like(out) * 0.1
    grads = torch.autograd.grad(out, (x, alpha, beta), go)
    torch.cuda.synchronize()
    xc, ac, bc = _cpu_leaf(x), _cpu_leaf(alpha), _cpu_leaf(beta)
    ref = stage(xc, ac, bc, O.read, O.triangular_torch, O.write)
    rgrads = torch.autograd.grad(ref, (xc, ac, bc), go.cpu())
    assert_parity(out, ref, dtype, what="stage out", kind="chained")
    for name, a, b in zip(("dX", "dalpha", "dbeta"), grads, rgrads):
        assert_parity(a, b, dtype, what=name, kind="chained" if name == "dX" else "reduced")
    if dtype == torch.float32:
        lit = O.literal_stage(xc.detach().double(), ac.detach().double(), bc.detach().double(),
                              [lambda z: 0.05 * z.tanh()] * events)
        assert rel_l2(out.detach().cpu(), lit) < 1e-5


def test_unused_reads_give_zero_weight_rows_and_update_count_check():
    announce("unused reads")
    x = torch.randn(1, 16, 16, 37, device="cuda", requires_grad=True)
    a = torch.randn(16, 37, 16, device="cuda", requires_grad=True)
    base = sublayer_read(x, a)
    base[0].sum().backward()
    assert torch.count_nonzero(a.grad[1:]) == 0
    assert torch.count_nonzero(a.grad[0]) > 0
    with pytest.raises(ValueError, match="one workspace update"):
        sublayer_write(x.detach(), [base[0].detach()], a.detach())
    with pytest.raises(ValueError, match="contiguous|packed"):
        sublayer_read(x.transpose(1, 2), a)
    for events in (8, 12):
        xb = torch.randn(2, 16, 16, 37, device="cuda", requires_grad=True)
        ab = torch.randn(events, 37, 16, device="cuda", requires_grad=True)
        blockwise_read(xb, ab)[0].sum().backward()
        assert torch.count_nonzero(ab.grad[1:]) == 0


@pytest.mark.parametrize("events", [8, 12])
@pytest.mark.parametrize("dtype", DTYPES)
def test_blockwise_adapters(events, dtype):
    announce(f"blockwise events={events} dtype={dtype}")
    torch.manual_seed(153)
    x = torch.randn(3, 22, 22, 67, device="cuda", dtype=dtype)
    a = torch.randn(events, 67, 4, device="cuda", dtype=dtype) * 0.05
    out = blockwise_read(x, a)
    for z, r in zip(out, O.read(x.cpu(), a.cpu())):
        assert_parity(z, r, dtype, what="blockwise read")
    z = [torch.randn(3, 121, 67, device="cuda", dtype=dtype) for _ in range(events)]
    assert_parity(blockwise_write(x, z, a), O.write(x.cpu(), [u.cpu() for u in z], a.cpu()), dtype)
    g = torch.randn(5, 67, device="cuda") * 0.05
    t = blockwise_triangular(z[0], z[1:6], g)
    assert_parity(t, O.triangular_torch(z[0].cpu(), [u.cpu() for u in z[1:6]], g.cpu()), dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_weight_reductions_are_deterministic_and_exact(dtype):
    # Atomics-free reductions: bitwise identical across runs; fp32 partial sums agree
    # with the fp64 oracle (reference :147-161 checks the fp32 accumulator pre-cast).
    announce(f"determinism dtype={dtype}")
    torch.manual_seed(671)
    x = torch.randn(3, 44, 44, 64, device="cuda", dtype=dtype)
    ups = [torch.randn(3, 484, 64, device="cuda", dtype=dtype) * 0.1 for _ in range(24)]
    w32 = torch.empty(24, 64, 4, device="cuda", dtype=torch.float32)
    r1 = launch.weight_grad(x, ups, w32)
    r2 = launch.weight_grad(x, ups, w32)
    assert torch.equal(r1, r2)
    exp = O.weight_grad(x.cpu(), [u.cpu() for u in ups], 4)
    assert_parity(r1, exp, torch.float32, what="fp32 weight-grad accumulator")
    gamma32 = torch.empty(23, 64, device="cuda")  # only its dtype (fp32 output) is used
    g1 = launch.triangular_gamma_grad(ups[0], ups[1:], gamma32)
    g2 = launch.triangular_gamma_grad(ups[0], ups[1:], gamma32)
    assert torch.equal(g1, g2)
    assert_parity(g1, O.triangular_gamma_grad(ups[0].cpu(), [u.cpu() for u in ups[1:]]), torch.float32)


def test_fp32_carrier_with_bf16_updates_chained_writes():
    # research/normalized_sensitivity/code/test_carrier_write.py:9-22: fp32 carrier,
    # bf16 updates and coefficients, 4 chained writes, atol 2e-6.
    announce("carrier write audit")
    torch.manual_seed(42)
    b, g, k, c = 2, 3, 4, 64
    carrier = torch.randn(b, g * k, g * k, c, device="cuda")
    reference = carrier.cpu().double()
    for _ in range(4):
        delta = torch.randn(b, g * g, c, device="cuda", dtype=torch.bfloat16)
        beta = torch.randn(1, c, k * k, device="cuda", dtype=torch.bfloat16)
        output = launch.write(carrier, [delta], beta)
        reference = O.write_torch(reference, [delta.cpu().double()], [beta[0].cpu().double()])
        torch.testing.assert_close(output.cpu().double(), reference, rtol=2e-6, atol=2e-6)
        carrier = output


def test_baseline_config0_single_event_fp32():
    # benchmark config 0: B8, 256 tokens, 4 slots, D=768, fp32; alpha ~ N(0.25,0.02),
    # beta ~ N(1,0.02) drawn [S,C] and passed [C,S]; loss <gX', X'> + <gz, z>.
    announce("config0 fp32 one event fwd+bwd")
    torch.manual_seed(0)
    x = torch.randn(8, 32, 32, 768)
    alpha = 0.25 + 0.02 * torch.randn(4, 768)
    beta = 1.0 + 0.02 * torch.randn(4, 768)
    y = torch.randn(8, 256, 768)
    gxp = 1e-2 * torch.randn(8, 32, 32, 768)
    gz = 1e-2 * torch.randn(8, 256, 768)
    a_cs, b_cs = alpha.T.contiguous(), beta.T.contiguous()
    dev = [t.cuda().requires_grad_() for t in (x, a_cs, b_cs, y)]
    z = sublayer_read(dev[0], dev[1][None])[0]
    xp = sublayer_write(dev[0], [dev[3]], dev[2][None])
    loss = (xp * gxp.cuda()).sum() + (z * gz.cuda()).sum()
    grads = torch.autograd.grad(loss, dev)
    cpu = [t.double().requires_grad_() for t in (x, a_cs, b_cs, y)]
    zr = O.read_torch(cpu[0], cpu[1])
    xr = O.write_torch(cpu[0], [cpu[3]], [cpu[2]])
    rl = (xr * gxp.double()).sum() + (zr * gz.double()).sum()
    rgrads = torch.autograd.grad(rl, cpu)
    assert_parity(z, zr, torch.float32, what="z")
    assert_parity(xp, xr, torch.float32, what="X'")
    for name, a, b in zip(("dX", "dalpha", "dbeta", "dy"), grads, rgrads):
        assert_parity(a, b, torch.float32, what=name)


def test_write_impl_without_carrier_add_and_gamma_cast():
    announce("write_impl add_x=False")
    torch.manual_seed(7)
    x = torch.randn(2, 8, 8, 16, device="cuda", dtype=torch.bfloat16)
    a = torch.randn(3, 16, 4, device="cuda", dtype=torch.bfloat16)
    g = [torch.randn(2, 16, 16, device="cuda", dtype=torch.bfloat16) for _ in range(3)]
    out = _write_impl(x, g, a, False)
    assert_parity(out, O.write(x.cpu(), [t.cpu() for t in g], a.cpu(), add_x=False), torch.bfloat16)
    wg = _weights_backward(x, g, a)
    assert wg.dtype == torch.bfloat16 and wg.shape == a.shape
    dg = _tri_gamma_backward(g[0], g[1:], torch.ones(2, 16, device="cuda", dtype=torch.bfloat16))
    assert dg.dtype == torch.bfloat16 and dg.shape == (2, 16)
