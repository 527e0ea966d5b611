"""GPU: the benchmark's two-stream schedule (two half-batch chains of per-event launches on
two HIP streams, one deferred finalize of both halves' partial rows) computes what the
one-stream chain computes. Per-token outputs are bit-identical (the same kernels on the same
tokens); the weight gradients sum the same products in another fixed order (each half has
its own reduction chunks), so they agree to fp32 reduction accuracy, and repeat bit for bit.
A smaller event count than the benchmark's keeps the test short."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

from helpers import announce, assert_parity

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
import bench  # noqa: E402

pytestmark = pytest.mark.gpu


def _snapshot(step):
    torch.cuda.synchronize()
    E = step.E
    return {"x_last": step.x[E].clone(), "z1": step.z[1].clone(), "gdz0": step.gdz[0].clone(),
            "gdz_last": step.gdz[E - 1].clone(), "gx": [g.clone() for g in step.gx],
            "gbeta": step.gbeta.clone(), "galpha": step.galpha.clone()}


@pytest.mark.parametrize("batch,events", [(16, 6), (6, 3)])
def test_two_stream_step_matches_one_stream(batch, events):
    announce(f"two-stream literal step batch={batch} events={events} D=1152")
    step = bench.LiteralStep(batch, 1152, events, seed=5)
    assert step.halves is not None
    step.step()
    one = _snapshot(step)
    step.step2()
    two = _snapshot(step)
    step.step2()
    again = _snapshot(step)
    for k in ("x_last", "z1", "gdz0", "gdz_last"):
        assert torch.equal(one[k], two[k]), k
    for a, b in zip(one["gx"], two["gx"]):
        assert torch.equal(a, b), "carrier gradient"
    for k in ("gbeta", "galpha"):
        assert_parity(two[k], one[k].float(), torch.bfloat16, kind="reduced", what=f"{k} two-stream vs one")
        assert torch.equal(two[k], again[k]), f"{k} not repeatable"


def test_overlapped_finalize_is_bit_identical():
    """The one-stream step whose first finalize batch runs on a second stream: the same
    partial rows summed by the same kernel, so every output has the same bits."""
    announce("one-stream step with overlapped finalize batch=8 events=7 D=1152")
    step = bench.LiteralStep(8, 1152, 7, seed=9)
    step.step()
    one = _snapshot(step)
    step.step_overlap()
    two = _snapshot(step)
    for k in ("x_last", "z1", "gdz0", "gdz_last", "gbeta", "galpha"):
        assert torch.equal(one[k], two[k]), k
