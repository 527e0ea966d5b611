"""GPU: a complete SiHC sublayer denoiser routed by the HIP ops.

Pattern of the reference's integration test (research/tests/test_sublayer_kernels.py:
216-263, full model vs a literal dense carrier): the same model, same weights and
same inputs, once with the HIP ops and once with the oracle's PyTorch read/write
(run on the same device), compared on the output and on every parameter gradient.
"""
from __future__ import annotations

import copy

import pytest
import torch

from helpers import announce, assert_parity, rel_l2
from oracle import sihc_oracle as O
from sihc_hip.e2e import SiHCDenoiser

pytestmark = pytest.mark.gpu


def _oracle_routing(model):
    model.read = lambda x, alpha: O.read(x, alpha)
    model.triangular = lambda base, ups, gamma: O.triangular_torch(base, ups, gamma)
    model.write = lambda x, ups, beta: O.write(x, ups, beta)
    return model


def _small(schedule, depth=8, patch=8, seed=0):
    stages = (8,) if depth == 8 else (8, 12)
    torch.manual_seed(seed)
    return SiHCDenoiser(hidden=64, depth=depth, heads=4, patch=patch, stages=stages,
                        schedule=schedule).random_init(seed=seed).cuda()


def _inputs(batch=2, seed=1):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(batch, 3, 256, 256, device="cuda", generator=g)
    t = torch.rand(batch, device="cuda", generator=g)
    y = torch.randint(0, 1000, (batch,), device="cuda", generator=g)
    return x, t, y


@pytest.mark.parametrize("depth,patch", [(8, 8), (20, 8), (8, 4)])
def test_stage_schedule_model_matches_oracle_routing_fp32(depth, patch):
    announce(f"e2e stage fp32 depth={depth} patch={patch}")
    model = _small("stage", depth, patch)
    ref = _oracle_routing(copy.deepcopy(model))
    x, t, y = _inputs()
    out, expected = model(x, t, y), ref(x, t, y)
    out.float().square().mean().backward()
    expected.float().square().mean().backward()
    assert_parity(out, expected, torch.float32, what="output")
    for (name, a), (_, b) in zip(model.named_parameters(), ref.named_parameters()):
        assert a.grad is not None and torch.isfinite(a.grad).all(), name
        # gradients pass through attention/MLP bodies: compare in relative L2
        assert rel_l2(a.grad, b.grad) < 1e-4, (name, rel_l2(a.grad, b.grad))


def test_literal_schedule_model_matches_stage_schedule_fp32():
    announce("e2e literal vs stage fp32")
    lit = _small("literal")
    stage = _oracle_routing(copy.deepcopy(lit))
    stage.schedule = "stage"
    x, t, y = _inputs()
    a, b = lit(x, t, y), stage(x, t, y)
    a.float().square().mean().backward()
    b.float().square().mean().backward()
    assert rel_l2(a, b) < 1e-5
    for (name, p), (_, q) in zip(lit.named_parameters(), stage.named_parameters()):
        assert rel_l2(p.grad, q.grad) < 1e-4, (name, rel_l2(p.grad, q.grad))


def test_bf16_model_matches_oracle_routing():
    announce("e2e stage bf16")
    model = _small("stage").to(torch.bfloat16)
    ref = _oracle_routing(copy.deepcopy(model))
    x, t, y = _inputs()
    with torch.no_grad():
        out, expected = model(x.bfloat16(), t, y), ref(x.bfloat16(), t, y)
    assert_parity(out, expected, torch.bfloat16, what="bf16 output")


@pytest.mark.parametrize("schedule", ["stage", "literal"])
def test_xl_shape_forward_runs(schedule):
    announce(f"e2e XL forward schedule={schedule}")
    model = SiHCDenoiser(schedule=schedule).random_init().cuda().to(torch.bfloat16).eval()
    x, t, y = _inputs(batch=2)
    with torch.no_grad():
        out = model(x.bfloat16(), t, y)
    assert out.shape == (2, 3, 256, 256) and torch.isfinite(out.float()).all()
