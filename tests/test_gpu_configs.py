"""GPU checks at the full sizes of the benchmark configurations (0-4).

The kernels treat tokens independently, so per-token outputs are checked on batch
slices against the CPU oracle; token reductions (weight gradients) are checked
against float64 CPU sums on channel slices; everything is checked for bitwise
run-to-run determinism. Two cases use a carrier with more than 2**31 elements to
exercise 64-bit addressing (the per-event forward, and the stage read / write / weight
gradient).
"""
from __future__ import annotations

import pytest
import torch

from helpers import announce, assert_parity
from oracle import sihc_oracle as O
from sihc_hip import launch
from sihc_hip.indexed import gather_cells, group_index, scatter_cells

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def _draw(batch, channels, seed, dtype=BF16):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(batch, 32, 32, channels, device="cuda", generator=g).to(dtype)
    alpha = (0.25 + 0.02 * torch.randn(4, channels, device="cuda", generator=g)).T.contiguous().to(dtype)
    beta = (1.0 + 0.02 * torch.randn(4, channels, device="cuda", generator=g)).T.contiguous().to(dtype)
    dz = torch.randn(batch, 256, channels, device="cuda", generator=g).to(dtype)
    return x, alpha, beta, dz


def test_config2_event_forward_and_backward_full_batch():
    announce("config2 shape B256 D1152 bf16 event fwd+bwd")
    x, alpha, beta, dz = _draw(256, 1152, seed=2)
    x_out, z_out = launch.event_forward(x, dz, beta, alpha)
    for sl in (slice(0, 2), slice(254, 256)):
        rx, rz = O.event_forward(x[sl].cpu(), dz[sl].cpu(), beta.cpu(), alpha.cpu())
        assert_parity(x_out[sl], rx, BF16, what="x_out slice")
        assert_parity(z_out[sl], rz, BF16, what="z_out slice")
    g = torch.Generator(device="cuda").manual_seed(22)
    h = (1e-2 * torch.randn(x.shape, device="cuda", generator=g)).to(BF16)
    gz = (1e-2 * torch.randn(dz.shape, device="cuda", generator=g)).to(BF16)
    gx, gdz, gb, ga = launch.event_backward(h, gz, x_out, dz, beta, alpha)
    again = launch.event_backward(h, gz, x_out, dz, beta, alpha)
    for a, b in zip((gx, gdz, gb, ga), again):
        assert torch.equal(a, b)
    for sl in (slice(0, 2), slice(254, 256)):
        ref = O.event_backward(h[sl].cpu(), gz[sl].cpu(), x_out[sl].cpu(), dz[sl].cpu(), beta.cpu(), alpha.cpu())
        assert_parity(gx[sl], ref[0], BF16, what="grad_x slice")
        assert_parity(gdz[sl], ref[1], BF16, what="grad_dz slice")
    # weight gradients over all 65,536 tokens (fp32 accumulate, one bf16 cast)
    # dbeta[c,s] = sum_m dz[m,c] t[m,s,c] with t = h + alpha*gz in fp64 from the bf16 inputs
    hc, gzc, xoc, dzc = h.cpu(), gz.cpu(), x_out.cpu(), dz.cpu()
    db = torch.zeros(1152, 4, dtype=torch.float64)
    da = torch.zeros(1152, 4, dtype=torch.float64)
    a64 = alpha.cpu().double()
    for b0 in range(0, 256, 16):
        t = O.high_to_cells(hc[b0:b0 + 16], 4).double() + gzc[b0:b0 + 16].double().unsqueeze(2) * a64.T[None, None]
        db += torch.einsum("bnsc,bnc->cs", t, dzc[b0:b0 + 16].double())
        da += torch.einsum("bnsc,bnc->cs", O.high_to_cells(xoc[b0:b0 + 16], 4).double(), gzc[b0:b0 + 16].double())
    assert_parity(gb, db, BF16, what="grad_beta (65,536 tokens)", kind="reduced")
    assert_parity(ga, da, BF16, what="grad_alpha (65,536 tokens)", kind="reduced")


def test_config1_stage_read_write_24_events():
    announce("config1 shape B256 D768 bf16 read/write E=24")
    x, _, _, _ = _draw(256, 768, seed=1)
    g = torch.Generator(device="cuda").manual_seed(11)
    alpha = (0.25 + 0.02 * torch.randn(24, 768, 4, device="cuda", generator=g)).to(BF16)
    beta = (1.0 + 0.02 * torch.randn(24, 768, 4, device="cuda", generator=g)).to(BF16)
    base = launch.read(x, alpha)
    again = launch.read(x, alpha)
    assert all(torch.equal(a, b) for a, b in zip(base, again))
    ref = O.read(x[:2].cpu(), alpha.cpu())
    for e in (0, 11, 23):
        assert_parity(base[e][:2], ref[e], BF16, what=f"base[{e}] slice")
    ups = [(0.1 * torch.randn(256, 256, 768, device="cuda", generator=g)).to(BF16) for _ in range(24)]
    out = launch.write(x, ups, beta)
    refw = O.write(x[-2:].cpu(), [u[-2:].cpu() for u in ups], beta.cpu())
    assert_parity(out[-2:], refw, BF16, what="stage write slice")
    # weight gradient over 65,536 tokens on two channel slices
    wg = launch.weight_grad(x, ups, beta)
    for cs in (slice(0, 32), slice(736, 768)):
        exp = torch.zeros(24, 32, 4, dtype=torch.float64)
        for b0 in range(0, 256, 32):
            cells = O.high_to_cells(x[b0:b0 + 32, :, :, cs].cpu(), 4).double()
            z = torch.stack([u[b0:b0 + 32, :, cs].cpu().double() for u in ups])
            exp += torch.einsum("bnsc,ebnc->ecs", cells, z)
        assert_parity(wg[:, cs], exp, BF16, what=f"weight grad channels {cs}", kind="reduced")


def test_config3_indexed_gather_scatter_full_size():
    announce("config3 shape B128 D1152 bf16 gather/scatter")
    x, _, _, _ = _draw(128, 1152, seed=3)
    idx = group_index(128, 16, 5, seed=3).cuda()
    cells = gather_cells(x, idx, validate=True)
    assert torch.equal(cells.cpu(), O.gather_cells(x.cpu(), idx.cpu(), 4))
    assert torch.equal(scatter_cells(cells, idx), x)


def test_config3_indexed_event_forward_and_backward_full_size():
    # The timed config-3 workload: batch 128, D = 1152, the seeded group-of-5 state index.
    # Per-token outputs on batch slices against gather -> oracle -> scatter; the weight
    # gradients over all 32,768 tokens against float64 sums of the gathered states.
    announce("config3 shape B128 D1152 bf16 indexed event fwd+bwd")
    x, alpha, beta, dz = _draw(128, 1152, seed=3)
    idx = group_index(128, 16, 5, seed=3).cuda()
    x_out, z_out = launch.event_forward(x, dz, beta, alpha, index=idx)
    for sl in (slice(0, 2), slice(126, 128)):
        ic = idx[sl].cpu()
        states = O.cells_to_high(O.gather_cells(x[sl].cpu(), ic, 4))  # token-ordered carrier
        rx, rz = O.event_forward(states, dz[sl].cpu(), beta.cpu(), alpha.cpu())
        assert_parity(x_out[sl], O.scatter_cells(O.high_to_cells(rx, 4), ic), BF16, what="indexed x_out slice")
        assert_parity(z_out[sl], rz, BF16, what="indexed z_out slice")
    g = torch.Generator(device="cuda").manual_seed(33)
    h = (1e-2 * torch.randn(x.shape, device="cuda", generator=g)).to(BF16)
    gz = (1e-2 * torch.randn(dz.shape, device="cuda", generator=g)).to(BF16)
    gx, gdz, gb, ga = launch.event_backward(h, gz, x_out, dz, beta, alpha, index=idx)
    again = launch.event_backward(h, gz, x_out, dz, beta, alpha, index=idx)
    for a, b in zip((gx, gdz, gb, ga), again):
        assert torch.equal(a, b)
    for sl in (slice(0, 2), slice(126, 128)):
        ic = idx[sl].cpu()
        gather = lambda t: O.cells_to_high(O.gather_cells(t[sl].cpu(), ic, 4))  # noqa: E731
        ref = O.event_backward(gather(h), gz[sl].cpu(), gather(x_out), dz[sl].cpu(), beta.cpu(), alpha.cpu())
        assert_parity(gx[sl], O.scatter_cells(O.high_to_cells(ref[0], 4), ic), BF16, what="indexed grad_x slice")
        assert_parity(gdz[sl], ref[1], BF16, what="indexed grad_dz slice")
    ic = idx.cpu()
    hc, gzc, xoc, dzc = h.cpu(), gz.cpu(), x_out.cpu(), dz.cpu()
    db = torch.zeros(1152, 4, dtype=torch.float64)
    da = torch.zeros(1152, 4, dtype=torch.float64)
    a64 = alpha.cpu().double()
    for b0 in range(0, 128, 16):
        bs = slice(b0, b0 + 16)
        t = O.gather_cells(hc[bs], ic[bs], 4).double() + gzc[bs].double().unsqueeze(2) * a64.T[None, None]
        db += torch.einsum("bnsc,bnc->cs", t, dzc[bs].double())
        da += torch.einsum("bnsc,bnc->cs", O.gather_cells(xoc[bs], ic[bs], 4).double(), gzc[bs].double())
    assert_parity(gb, db, BF16, what="indexed grad_beta (32,768 tokens)", kind="reduced")
    assert_parity(ga, da, BF16, what="indexed grad_alpha (32,768 tokens)", kind="reduced")


def test_carrier_over_2_pow_31_elements():
    # 2048 x 32 x 32 x 1152 = 2.42e9 elements (4.8 GB bf16): 64-bit offsets.
    announce("max size carrier B2048 D1152 bf16 event fwd")
    x, alpha, beta, dz = _draw(2048, 1152, seed=4)
    assert x.numel() > 2 ** 31
    x_out, z_out = launch.event_forward(x, dz, beta, alpha)
    sl = slice(2046, 2048)
    rx, rz = O.event_forward(x[sl].cpu(), dz[sl].cpu(), beta.cpu(), alpha.cpu())
    assert_parity(x_out[sl], rx, BF16, what="x_out tail")
    assert_parity(z_out[sl], rz, BF16, what="z_out tail")
    del x, x_out, z_out, dz
    torch.cuda.empty_cache()


def test_stage_ops_over_2_pow_31_carrier_elements():
    # The stage kernels at the same 2.42e9-element carrier (64-bit offsets in every
    # kernel shape: non-temporal reads with 2 events, 8-event reads and writes, the
    # pipelined weight gradient). Per-token outputs are checked on the last two batch
    # items; the weight gradient gets updates that are zero outside those items, so its
    # full-size reduction equals the oracle's sum over that slice.
    announce("max size carrier B2048 D1152 bf16 stage ops")
    B, C, E = 2048, 1152, 8
    g = torch.Generator(device="cuda").manual_seed(6)
    x = torch.randn(B, 32, 32, C, device="cuda", generator=g).to(BF16)
    assert x.numel() > 2 ** 31
    w = (0.2 + 0.05 * torch.randn(E, C, 4, device="cuda", generator=g)).to(BF16)
    sl = slice(B - 2, B)
    xs = x[sl].cpu()
    for e in (2, E):
        got = launch.read(x, w[:e].contiguous())
        exp = O.read(xs, w[:e].cpu())
        for i in range(e):
            assert_parity(got[i][sl], exp[i], BF16, what=f"read E={e} output {i} tail")
        del got
    ups = [torch.zeros(B, 256, C, device="cuda", dtype=BF16) for _ in range(E)]
    for u in ups:
        u[sl] = torch.randn(2, 256, C, device="cuda", generator=g).to(BF16)
    out = launch.write(x, ups, w)
    assert_parity(out[sl], O.write(xs, [u[sl].cpu() for u in ups], w.cpu()), BF16, what="write tail")
    del out
    torch.cuda.empty_cache()
    wg = launch.weight_grad(x, ups, w, out_dtype=torch.float32)
    assert_parity(wg, O.weight_grad(xs, [u[sl].cpu() for u in ups], 4), torch.float32, what="weight grad")
    del x, ups, wg
    torch.cuda.empty_cache()
