"""GPU: the benchmark's config-2 step under its two finalize schedules computes the same
bits. The step strings the per-event backward launches of a 56-event literal chain (here
fewer events and a smaller batch) through the C ABI; the schedules differ only in where
each event's weight-gradient partial rows are summed:

* deferred: sihc_event_backward_partial for every event, then sihc_event_finalize;
* chain: sihc_event_backward_chain, each launch finalizing the previous event's rows in
  its trailing blocks, and one finalize launch for the last call.

The partial rows and the fixed-order sums are the same in both, so every output
(carrier and workspace gradients, dbeta, dalpha) must be bit-identical, step after step.

The config-3 step (the same launches through a state index) is checked the same way: with
the identity index against the step without one, and with a group-of-5 permutation index
against the step without one over the carrier whose cells are in token order.
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


def _run(step):
    _poison(step)
    step.step()
    return _snapshot(step)


def test_identity_index_step_matches_unindexed():
    # the config-3 step (every launch through a state index) with the identity index: the
    # same launches, so the same bits as the step without an index
    announce("config-3 step, identity index vs no index, batch=3 events=7 D=1152")
    batch, events = 3, 7
    ident = torch.arange(256, device="cuda", dtype=torch.int32).repeat(batch, 1)
    plain = _run(bench.LiteralStep(batch, 1152, events, seed=13))
    indexed = _run(bench.LiteralStep(batch, 1152, events, seed=13, index=ident))
    _same(indexed, plain, "identity index")


def test_permutation_index_step_matches_unindexed_on_gathered_carrier():
    # Through a per-image permutation index (the seeded groups of 5), token n of image b
    # reads and writes cell index[b, n]. The step without an index over the carrier whose
    # cell n is that cell computes the same per-token values in the same token order, so
    # every output matches bit for bit: the carriers after gathering their cells, the
    # workspace outputs and gradients as they are, and the weight gradients (their
    # partial sums run over the same values in the same order).
    from sihc_hip import launch
    from sihc_hip.indexed import group_index

    announce("config-3 step, group-of-5 index vs no index on gathered cells, batch=3 events=7")
    batch, events = 3, 7
    idx = group_index(batch, 16, 5, seed=3).cuda()
    ident = torch.arange(256, device="cuda", dtype=torch.int32).repeat(batch, 1)
    si = bench.LiteralStep(batch, 1152, events, seed=17, index=idx)
    su = bench.LiteralStep(batch, 1152, events, seed=17)
    # the unindexed step's carrier inputs: the indexed step's cells in token order
    in_token_order = lambda t: launch.scatter_cells(launch.gather_cells(t, idx, 4), ident)  # noqa: E731
    with torch.no_grad():
        su.x[0].copy_(in_token_order(si.x[0]))
        su.h_out.copy_(in_token_order(si.h_out))
    a, b = _run(si), _run(su)
    cells = lambda t, ix: launch.gather_cells(t, ix, 4)  # noqa: E731
    assert torch.equal(cells(a["x_last"], idx), cells(b["x_last"], ident)), "carrier after the last event"
    for x, y in zip(a["gx"], b["gx"]):
        assert torch.equal(cells(x, idx), cells(y, ident)), "carrier gradient"
    for k in ("z1", "gdz0", "gdz_last", "gbeta", "galpha"):
        assert torch.equal(a[k], b[k]), k
