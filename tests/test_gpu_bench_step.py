"""GPU: the benchmark's config-2 step under its two finalize schedules computes the same
bits. The step strings the per-event backward launches of a 56-event literal chain (here
fewer events and a smaller batch) through the C ABI; the schedules differ only in where
each event's weight-gradient partial rows are summed:

* deferred: sihc_event_backward_partial for every event, then sihc_event_finalize;
* chain: sihc_event_backward_chain, each launch finalizing the previous event's rows in
  its trailing blocks, and one finalize launch for the last call.

The partial rows and the fixed-order sums are the same in both, so every output
(carrier and workspace gradients, dbeta, dalpha) must be bit-identical, step after step.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

from helpers import announce

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
import bench  # noqa: E402

pytestmark = pytest.mark.gpu


def _snapshot(step):
    torch.cuda.synchronize()
    E = step.E
    return {"x_last": step.x[E].clone(), "z1": step.z[1].clone(), "gdz0": step.gdz[0].clone(),
            "gdz_last": step.gdz[E - 1].clone(), "gx": [g.clone() for g in step.gx],
            "gbeta": step.gbeta.clone(), "galpha": step.galpha.clone()}


def _poison(step):
    # every weight gradient NaN before the step: an output a schedule leaves unwritten shows
    with torch.no_grad():
        step.gbeta.fill_(float("nan"))
        step.galpha.fill_(float("nan"))


def _same(a, b, what):
    for k in ("x_last", "z1", "gdz0", "gdz_last", "gbeta", "galpha"):
        assert torch.equal(a[k], b[k]), f"{what}: {k}"
    for x, y in zip(a["gx"], b["gx"]):
        assert torch.equal(x, y), f"{what}: carrier gradient"


@pytest.mark.parametrize("batch,events", [(8, 7), (3, 34)])
def test_finalize_schedules_are_bit_identical(batch, events):
    announce(f"config-2 step finalize schedules batch={batch} events={events} D=1152")
    step = bench.LiteralStep(batch, 1152, events, seed=9)
    step.use_chain(False)
    _poison(step)
    step.step()
    deferred = _snapshot(step)
    assert torch.isfinite(deferred["gbeta"].float()).all() and torch.isfinite(deferred["galpha"].float()).all()
    step.use_chain(True)
    for r in range(2):
        _poison(step)
        step.step()
        _same(_snapshot(step), deferred, f"chain step {r}")
