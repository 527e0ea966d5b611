"""Shared pytest setup: import paths, the `gpu` marker and parity helpers."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "residual-stream-burden_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True, scope="session")
def _no_tf32():
    # Tight fp32 oracles: no reduced-precision matmul anywhere in the checks.
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    yield


def pytest_terminal_summary(terminalreporter):
    """Worst achieved parity margins per bar (the achieved errors of every check)."""
    from helpers import RECORDS

    if not RECORDS:
        return
    tr = terminalreporter
    tr.section("parity margins")
    for kind in ("elementwise", "reduced", "chained", "fp32", "reference"):
        rows = [r for r in RECORDS if r[3] == kind]
        if not rows:
            continue
        if kind == "reference":  # r[5] holds the worst fraction of the reference's own bar
            worst = max(rows, key=lambda r: r[5])
            tr.write_line(f"{kind:11s} {len(rows):4d} checks; worst {worst[5]:.3f} of the reference's bar "
                          f"({worst[1]}, {worst[0]})")
            continue
        worst_rel = max(rows, key=lambda r: r[7])
        line = f"{kind:11s} {len(rows):4d} checks; worst rel-L2 {worst_rel[7]:.2e} ({worst_rel[1]}, {worst_rel[0]})"
        if kind == "elementwise":
            worst = max(rows, key=lambda r: r[6])
            line += f"; worst {worst[6]:.2f} ulp ({worst[1]}, {worst[0]})"
        else:
            worst = max(rows, key=lambda r: r[4] / max(r[5], 1e-30))
            line += f"; worst max-abs/scale {worst[4] / max(worst[5], 1e-30):.2e} ({worst[1]}, {worst[0]})"
        tr.write_line(line)
