"""GPU: the SiHC denoiser compiled by Inductor (torch.compile mode="default",
fullgraph=True), forward and backward, against the same model run eagerly.

Mirrors the reference's compile contract (research/tests/test_sublayer_kernels.py:
266-286): fp32 parameters, bf16 autocast or fp32, output and every parameter gradient
compared with the reference's tolerances. Inductor generates the kernels of the bodies
and of the elementwise work around the routing; the routing itself stays on this
library's custom ops, which the compiler sees only through their fake implementations.
The triangular op's traced backward leaves the update gradients grad * gamma_j to
Inductor by default (as the reference does, sublayer_kernels.py:369-379); the
one-pass HIP alternative (COMPILED_TRIANGULAR_BACKWARD = "fused") is checked too.
"""
from __future__ import annotations

import copy
import time

import pytest
import torch

from helpers import announce, assert_close_reference, assert_parity
from sihc_hip import sublayer_kernels
from sihc_hip.sublayer_kernels import sublayer_triangular
from sihc_hip.e2e import SiHCDenoiser

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _serial_compile(monkeypatch):
    # compile in this process only: no pool of compile workers on the GPU box
    import torch._inductor.config as cfg

    monkeypatch.setattr(cfg, "compile_threads", 1)
    torch._dynamo.reset()
    yield
    torch._dynamo.reset()


def _model(schedule, depth, patch, seed=42):
    torch.manual_seed(seed)
    stages = (depth,)
    return SiHCDenoiser(hidden=64, depth=depth, heads=4, patch=patch, stages=stages,
                        schedule=schedule).random_init(seed=seed).cuda()


def _inputs(seed=3):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(1, 3, 256, 256, device="cuda", generator=g)
    t = torch.rand(1, device="cuda", generator=g)
    y = torch.zeros(1, device="cuda", dtype=torch.long)
    return x, t, y


def _run(fn, module, x, t, y, bf16):
    """Forward through `fn` (the module or its compiled wrapper), backward, and the
    gradients of `module`'s parameters by name."""
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=bf16):
        out = fn(x, t, y)
    out.float().square().mean().backward()
    return out.detach(), {n: p.grad.detach().clone() for n, p in module.named_parameters()}


CASES = [  # (schedule, depth, patch, bf16 autocast, traced triangular backward)
    ("stage", 8, 4, True, "visible"),
    ("literal", 8, 4, True, "visible"),
    ("stage", 12, 8, False, "visible"),
    ("stage", 8, 4, True, "fused"),
]


@pytest.mark.parametrize("schedule,depth,patch,bf16,tri", CASES,
                         ids=[f"{c[0]}-d{c[1]}-p{c[2]}-{'bf16' if c[3] else 'fp32'}-{c[4]}" for c in CASES])
def test_inductor_fullgraph_forward_backward(schedule, depth, patch, bf16, tri, monkeypatch):
    announce(f"inductor fullgraph {schedule} depth={depth} patch={patch} bf16={bf16} tri={tri}")
    monkeypatch.setattr(sublayer_kernels, "COMPILED_TRIANGULAR_BACKWARD", tri)
    model = _model(schedule, depth, patch)
    twin = copy.deepcopy(model)
    x, t, y = _inputs()
    eager_out, eager_grads = _run(model, model, x, t, y, bf16)
    compiled = torch.compile(twin, mode="default", fullgraph=True)
    t0 = time.perf_counter()
    out, grads = _run(compiled, twin, x, t, y, bf16)
    torch.cuda.synchronize()
    announce(f"  compiled forward+backward (with compilation) {time.perf_counter() - t0:.1f} s")
    dtype = torch.bfloat16
    # reference tolerances (test_sublayer_kernels.py:282-286)
    torch.testing.assert_close(out, eager_out, atol=0.025 if bf16 else 3e-5, rtol=0.03 if bf16 else 3e-4)
    if bf16:  # logs the achieved margin; fp32 keeps the reference's absolute/relative bar above
        assert_parity(out, eager_out, dtype, kind="chained", what="compiled output")
    for name, g in grads.items():
        assert torch.isfinite(g).all(), name
        torch.testing.assert_close(g, eager_grads[name], atol=5e-4 if bf16 else 3e-5,
                                   rtol=0.15 if bf16 else 0.003, msg=name)


TRI_CASES = [(d, a, tri) for d in (torch.float32, torch.bfloat16) for a in (3, 23) for tri in ("visible", "fused")]


@pytest.mark.parametrize("dtype,active,tri", TRI_CASES,
                         ids=[f"{str(d)[6:]}-a{a}-{t}" for d, a, t in TRI_CASES])
def test_triangular_compiled_gradient_accumulation_and_tails(dtype, active, tri, monkeypatch):
    # The triangular op alone under torch.compile(mode="default", fullgraph=True), with the
    # reference's case (research/tests/test_sublayer_kernels.py:185-213): 3 x 49 rows x 67
    # channels (token and channel tails), an fp32 gamma with a bf16 (or fp32) workspace, and a
    # second loss term on every update, so the compiled backward must add the triangular
    # op's update gradient to the update's own gradient. Eager, compiled and a plain
    # PyTorch restatement agree within the reference's tolerances; both traced forms of
    # the op's backward are compiled.
    announce(f"inductor triangular op dtype={dtype} active={active} traced backward={tri}")
    monkeypatch.setattr(sublayer_kernels, "COMPILED_TRIANGULAR_BACKWARD", tri)
    torch.manual_seed(583)
    base = torch.randn(3, 49, 67, device="cuda", dtype=dtype).requires_grad_()
    updates = [torch.randn_like(base).requires_grad_() for _ in range(active)]
    gamma = (torch.randn(active, 67, device="cuda") * 0.05).requires_grad_()  # fp32 gamma
    inputs = (base, *updates, gamma)

    def fn(base, updates, gamma):
        out = sublayer_triangular(base, updates, gamma)
        return out.float().square().mean() + sum(u.float().square().mean() for u in updates)

    loss = fn(base, updates, gamma)
    eager = torch.autograd.grad(loss, inputs)
    ref = (base.float() + sum(u.float() * g for u, g in zip(updates, gamma))).to(dtype)
    ref_loss = ref.float().square().mean() + sum(u.float().square().mean() for u in updates)
    expected = torch.autograd.grad(ref_loss, inputs)
    compiled = torch.compile(fn, mode="default", fullgraph=True)
    actual = compiled(base, updates, gamma)
    compiled_grads = torch.autograd.grad(actual, inputs)
    tol = dict(atol=2e-4, rtol=2e-4) if dtype == torch.float32 else dict(atol=0.025, rtol=0.03)
    assert_close_reference(actual, loss, what="compiled loss", **tol)
    names = ["base"] + [f"update {j}" for j in range(active)] + ["gamma"]
    gtol = dict(atol=1e-7, rtol=3e-4) if dtype == torch.float32 else dict(atol=2e-5, rtol=0.035)
    for name, a, b, c in zip(names, eager, expected, compiled_grads):
        assert a.dtype == b.dtype == c.dtype, name
        assert_close_reference(a, b, what=f"eager grad {name} vs plain PyTorch", **gtol)
        assert_close_reference(c, a, what=f"compiled grad {name} vs eager", **gtol)
