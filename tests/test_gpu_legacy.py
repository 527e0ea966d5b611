"""GPU: the fixed-arity block-wise ops (the reference's kernels.py) on the HIP kernels.

Mirrors the reference's own tests of these ops (research/tests/
test_blockwise_kernels.py:20-87: every prefix family, forward and all gradients
including "no gradient" for inactive updates; research/tests/test_p8_kernels.py:
42-140: split reads and final accumulation, forward and backward) with this tier's
parity bar instead of their looser bf16 tolerances, and adds the b4 geometries, the
stand-alone gradient ops, cell_mean and a compiled stage. Expected values come from
the oracle (its PyTorch restatement, differentiated by autograd in float64).
"""
from __future__ import annotations

import pytest
import torch

from helpers import announce, assert_parity
from oracle import sihc_oracle as O
from sihc_hip import kernels as K
from sihc_hip.sublayer_kernels import sublayer_read, sublayer_triangular, sublayer_write

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16]
SPLIT = {"b4_12": K.all_base_b4_12_split_traceable, "b4_8": K.all_base_b4_8_split_traceable,
         "p8_12": K.all_base_p8_12_split_traceable}
FINAL = {"b4_12": K.final_accumulate_b4_12_traceable, "b4_8": K.final_accumulate_b4_8_traceable,
         "p8_12": K.final_accumulate_p8_12_traceable}


def _leaf(t):
    return t.detach().clone().requires_grad_(True)


def _f64(ts):
    return [t.detach().cpu().double().requires_grad_(True) for t in ts]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("stage,active", [(8, 1), (8, 4), (8, 7), (12, 1), (12, 6), (12, 11)])
def test_triangular_active_ops_forward_and_fused_backward(stage, active, dtype):
    announce(f"legacy triangular stage={stage} active={active} dtype={dtype}")
    torch.manual_seed(1000 + stage * 10 + active)
    shape = (1, 256, 97)
    base = torch.randn(shape, device="cuda", dtype=dtype, requires_grad=True)
    dzs = [torch.randn(shape, device="cuda", dtype=dtype, requires_grad=True) for _ in range(stage)]
    gamma = torch.randn(stage, shape[-1], device="cuda", dtype=dtype, requires_grad=True)
    upstream = torch.randn(shape, device="cuda", dtype=dtype)
    ops = K.triangular_accumulate_b4_8_ptr_active_traceable_ops if stage == 8 else \
        K.triangular_accumulate_b4_12_ptr_active_traceable_ops
    out = ops[active - 1](base, *dzs, gamma.contiguous())
    grads = torch.autograd.grad(out, (base, *dzs, gamma), upstream, allow_unused=True)

    expected = O.triangular_torch(base.detach().cpu(), [d.detach().cpu() for d in dzs[:active]],
                                  gamma.detach().cpu())
    assert_parity(out, expected, dtype, what="forward")
    rb, *rdz, rg = _f64([base, *dzs, gamma])
    ref = O.triangular_torch(rb, rdz[:active], rg)
    rgrads = torch.autograd.grad(ref, (rb, *rdz, rg), upstream.cpu().double(), allow_unused=True)
    assert torch.equal(grads[0], upstream)  # identity to base
    for i, (a, r) in enumerate(zip(grads[1:1 + stage], rgrads[1:1 + stage])):
        if i >= active:
            assert a is None and r is None, f"dz{i} of an inactive slot must get no gradient"
        else:
            assert_parity(a, r, dtype, what=f"grad dz{i}")
    assert grads[-1].dtype == dtype
    assert_parity(grads[-1], rgrads[-1], dtype, what="grad gamma", kind="reduced")
    assert torch.count_nonzero(grads[-1][active:]) == 0


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("tag", ["b4_12", "b4_8", "p8_12"])
def test_all_base_split_forward_and_backward(tag, dtype):
    announce(f"legacy all_base {tag} dtype={dtype}")
    edge, cell, blocks = K.GEOMETRY[tag]
    torch.manual_seed(810)
    c = 37
    x = torch.randn(2, edge, edge, c, device="cuda", dtype=dtype, requires_grad=True)
    alpha = torch.randn(blocks, c, cell * cell, device="cuda", dtype=dtype, requires_grad=True)
    outs = SPLIT[tag](x, alpha)
    assert len(outs) == blocks
    for e, (a, r) in enumerate(zip(outs, O.read(x.detach().cpu(), alpha.detach().cpu()))):
        assert_parity(a, r, dtype, what=f"read {e}")
    upstream = [torch.randn_like(o) for o in outs]
    gx, ga = torch.autograd.grad(outs, (x, alpha), upstream)
    rx, ra = _f64([x, alpha])
    ref = O.read(rx, ra)
    ex, ea = torch.autograd.grad(ref, (rx, ra), [u.cpu().double() for u in upstream])
    assert gx.dtype == dtype and ga.dtype == dtype
    assert_parity(gx, ex, dtype, what="grad x0")
    assert_parity(ga, ea, dtype, what="grad alpha", kind="reduced")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("tag", ["b4_12", "b4_8", "p8_12"])
def test_final_accumulate_forward_and_backward(tag, dtype):
    announce(f"legacy final_accumulate {tag} dtype={dtype}")
    edge, cell, blocks = K.GEOMETRY[tag]
    torch.manual_seed(812)
    c = 37
    x = torch.randn(2, edge, edge, c, device="cuda", dtype=dtype, requires_grad=True)
    dzs = [torch.randn(2, 256, c, device="cuda", dtype=dtype, requires_grad=True) for _ in range(blocks)]
    betas = [torch.randn(c, cell * cell, device="cuda", dtype=dtype, requires_grad=True) for _ in range(blocks)]
    out = FINAL[tag](x, *dzs, *betas)
    expected = O.write_torch(x.detach().cpu(), [d.detach().cpu() for d in dzs], [b.detach().cpu() for b in betas])
    assert_parity(out, expected, dtype, what="forward")
    upstream = torch.randn_like(out)
    grads = torch.autograd.grad(out, (x, *dzs, *betas), upstream)
    leaves = _f64([x, *dzs, *betas])
    ref = O.write_torch(leaves[0], leaves[1:1 + blocks], leaves[1 + blocks:])
    rgrads = torch.autograd.grad(ref, leaves, upstream.cpu().double())
    for i, (a, r) in enumerate(zip(grads, rgrads)):
        assert a.dtype == dtype
        assert_parity(a, r, dtype, what=f"grad input {i}", kind="reduced" if i > blocks else "elementwise")


def test_final_accumulate_fp32_carrier_with_bf16_updates():
    announce("legacy final_accumulate mixed dtypes")
    torch.manual_seed(813)
    c = 64
    x = torch.randn(2, 64, 64, c, device="cuda", requires_grad=True)
    dzs = [torch.randn(2, 256, c, device="cuda", dtype=torch.bfloat16, requires_grad=True) for _ in range(8)]
    betas = [torch.randn(c, 16, device="cuda", dtype=torch.bfloat16, requires_grad=True) for _ in range(8)]
    out = K.final_accumulate_b4_8_traceable(x, *dzs, *betas)
    assert out.dtype == torch.float32
    expected = O.write_torch(x.detach().cpu(), [d.detach().cpu() for d in dzs], [b.detach().cpu() for b in betas])
    assert_parity(out, expected, torch.float32, what="forward")
    upstream = torch.randn_like(out)
    grads = torch.autograd.grad(out, (x, *dzs, *betas), upstream)
    leaves = _f64([x, *dzs, *betas])
    rgrads = torch.autograd.grad(O.write_torch(leaves[0], leaves[1:9], leaves[9:]), leaves, upstream.cpu().double())
    for i, (a, r) in enumerate(zip(grads, rgrads)):
        assert_parity(a, r, torch.float32 if i == 0 else torch.bfloat16, what=f"grad input {i}",
                      kind="reduced" if i > 8 else "elementwise")


@pytest.mark.parametrize("dtype", DTYPES)
def test_stand_alone_gradient_ops(dtype):
    announce(f"legacy gradient ops dtype={dtype}")
    torch.manual_seed(7)
    c = 48
    x = torch.randn(2, 64, 64, c, device="cuda", dtype=dtype)
    grad_base = torch.randn(12, 2, 256, c, device="cuda", dtype=dtype)
    alpha = torch.randn(12, c, 16, device="cuda", dtype=dtype)
    gx = K.all_base_b4_12_grad_x_traceable(grad_base, alpha)
    assert_parity(gx, O.write(x.cpu(), list(grad_base.cpu().unbind(0)), alpha.cpu(), add_x=False), dtype,
                  what="grad_x")
    ga = K.all_base_b4_12_split_grad_alpha_traceable(x, grad_base)
    assert ga.dtype == torch.float32
    assert_parity(ga, O.weight_grad(x.cpu(), list(grad_base.cpu().unbind(0)), 16), torch.float32, what="grad_alpha")
    betas = list(alpha.unbind(0))
    gdz = K.final_accumulate_b4_12_grad_dz_ptr_traceable(x, *betas)
    assert gdz.shape == (12, 2, 256, c)
    for e, r in enumerate(O.read(x.cpu(), alpha.cpu())):
        assert_parity(gdz[e], r, dtype, what=f"grad_dz {e}")
    gb = K.final_accumulate_b4_12_grad_beta_ptr_traceable(x, *grad_base.unbind(0))
    assert gb.dtype == torch.float32
    assert_parity(gb, O.weight_grad(x.cpu(), list(grad_base.cpu().unbind(0)), 16), torch.float32, what="grad_beta")
    # triangular prefix 5 of 12: grad_dz, grad_gamma and the fused pair
    op = torch.ops.sihc.triangular_accumulate_b4_12_ptr_active5_grad_fused
    g = grad_base[0]
    dzs = list(grad_base[1:].unbind(0)) + [torch.zeros_like(g)]
    gamma = alpha[:, :, 0].contiguous()
    ddz, dg = op(g, *dzs, gamma)
    rdz, rdg = O.triangular_backward(g.cpu(), [d.cpu() for d in dzs[:5]], gamma.cpu())
    assert ddz.shape == (5, 2, 256, c) and dg.shape == (12, c) and dg.dtype == torch.float32
    for j in range(5):
        assert torch.equal(ddz[j].cpu(), rdz[j]), f"grad_fused dz{j} not bit-exact"
    assert_parity(dg[:5], rdg, torch.float32, what="grad_fused gamma")
    assert torch.count_nonzero(dg[5:]) == 0
    assert torch.equal(torch.ops.sihc.triangular_accumulate_b4_12_ptr_active5_grad_dz(g, gamma), ddz)
    # the stand-alone gamma op reduces in another (fixed) order than the fused pass
    dg_alone = torch.ops.sihc.triangular_accumulate_b4_12_ptr_active5_grad_gamma(g, *dzs, gamma)
    assert_parity(dg_alone[:5], rdg, torch.float32, what="grad_gamma")
    assert torch.count_nonzero(dg_alone[5:]) == 0


@pytest.mark.parametrize("dtype", DTYPES)
def test_cell_mean_b4_is_exact(dtype):
    announce(f"legacy cell_mean dtype={dtype}")
    torch.manual_seed(9)
    x = torch.randn(3, 64, 64, 40, device="cuda", dtype=dtype, requires_grad=True)
    z = K.cell_mean_b4_traceable(x)
    assert torch.equal(z.cpu(), O.cell_mean(x.detach().cpu())), "cell mean must match the fp32 slot-order sum"
    g = torch.randn_like(z)
    (gx,) = torch.autograd.grad(z, (x,), g)
    expected = O.cells_to_high((g.float() / 16).to(dtype)[:, :, None, :].expand(3, 256, 16, 40).cpu())
    assert torch.equal(gx.cpu(), expected)


def _legacy_stage(x0, alpha, beta):
    """The reference model's fused schedule stage (model.py:434-470) with tanh bodies."""
    n = alpha.shape[0]
    split = K.all_base_b4_12_split_traceable if n == 12 else K.all_base_b4_8_split_traceable
    ops = K.triangular_accumulate_b4_12_ptr_active_traceable_ops if n == 12 else \
        K.triangular_accumulate_b4_8_ptr_active_traceable_ops
    final = K.final_accumulate_b4_12_traceable if n == 12 else K.final_accumulate_b4_8_traceable
    base = split(x0, alpha)
    gamma = (alpha[:, None] * beta[None]).sum(-1)
    zero = torch.zeros_like(base[0])
    dz_list = []
    for i in range(n):
        z = base[i]
        if dz_list:
            args = tuple(dz_list[j] if j < i else zero for j in range(n))
            z = ops[i - 1](z, *args, gamma[i].contiguous())
        dz_list.append((0.05 * torch.tanh(z)).contiguous())
    return final(x0, *dz_list, *[b.contiguous() for b in beta.unbind(0)])


def _sublayer_stage(x0, alpha, beta):
    base = sublayer_read(x0, alpha)
    gamma = (alpha[:, None] * beta[None]).sum(-1)
    updates = []
    for i in range(alpha.shape[0]):
        z = base[i] if i == 0 else sublayer_triangular(base[i], updates, gamma[i, :i].contiguous())
        updates.append((0.05 * torch.tanh(z)).contiguous())
    return sublayer_write(x0, updates, beta)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("blocks", [8, 12])
def test_legacy_stage_equals_sublayer_stage_and_compiles(blocks, dtype):
    announce(f"legacy stage blocks={blocks} dtype={dtype}")
    torch._dynamo.reset()
    torch.manual_seed(11)
    c = 64
    x = torch.randn(2, 64, 64, c, device="cuda", dtype=dtype)
    alpha = (1 / 16 + 0.01 * torch.randn(blocks, c, 16, device="cuda")).to(dtype)
    beta = (1 + 0.05 * torch.randn(blocks, c, 16, device="cuda")).to(dtype)
    leaves = [_leaf(t) for t in (x, alpha, beta)]
    out = _legacy_stage(*leaves)
    go = 0.1 * torch.randn_like(out)
    grads = torch.autograd.grad(out, leaves, go)
    ref_leaves = [_leaf(t) for t in (x, alpha, beta)]
    ref = _sublayer_stage(*ref_leaves)
    ref_grads = torch.autograd.grad(ref, ref_leaves, go)
    # same kernels in the same order: bit-identical
    assert torch.equal(out, ref)
    for a, b in zip(grads, ref_grads):
        assert torch.equal(a, b)
    comp_leaves = [_leaf(t) for t in (x, alpha, beta)]
    comp = torch.compile(_legacy_stage, backend="aot_eager", fullgraph=True)(*comp_leaves)
    comp_grads = torch.autograd.grad(comp, comp_leaves, go)
    assert torch.equal(comp, out)
    # the traced backward may add the autograd contributions in another order
    for a, b in zip(comp_grads, grads):
        assert_parity(a, b, dtype, kind="chained")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("events", [1, 2, 3])
@pytest.mark.parametrize("c", [37, 64])
def test_few_event_reductions_direct_and_staged(events, c, dtype):
    # One or two event lanes take the direct-load reduction, three the LDS-staged one;
    # odd token counts exercise the chunk tails, C=37 the one-element vectors.
    announce(f"few-event reductions events={events} c={c} dtype={dtype}")
    from sihc_hip import launch
    torch.manual_seed(20 + events)
    x = torch.randn(3, 14, 14, c, device="cuda", dtype=dtype)            # 147 tokens, 2x2 cells
    ups = [torch.randn(3, 49, c, device="cuda", dtype=dtype) for _ in range(events)]
    w = torch.randn(events, c, 4, device="cuda", dtype=dtype)
    assert_parity(launch.weight_grad(x, ups, w), O.weight_grad(x.cpu(), [u.cpu() for u in ups], 4).to(dtype),
                  dtype, what="carrier weight grad", kind="reduced")
    grad = torch.randn(3, 49, c, device="cuda", dtype=dtype)
    gamma = torch.randn(events, c, device="cuda")
    ddz, dg = launch.triangular_backward(grad, ups, gamma)
    rdz, rdg = O.triangular_backward(grad.cpu(), [u.cpu() for u in ups], gamma.cpu())
    for j in range(events):
        assert torch.equal(ddz[j].cpu(), rdz[j]), f"update gradient {j} not bit-exact"
    assert_parity(dg, rdg, torch.float32, what="gamma grad")
