"""GPU: the C ABI driven from plain C, with no Python in the process.

`sihc_abi_selftest` (residual-stream-burden_amd/csrc/abi_selftest.c, built next to
libsihc_hip.so by build.py) allocates device memory through the HIP runtime, calls
read / write / weight gradient / triangular / fused triangular backward, the per-event
fused forward and backward (without and with a permutation state index; also as a
deferred call followed by a chained call that finalizes it in its trailing blocks) and the cell
gather / scatter through include/sihc_hip.h on fp32 inputs, compares every result with
direct loops over the cell index map (the cell copies bit for bit, including
scatter(gather(x)) == x), and checks that an argument error is reported before any
launch.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

from helpers import announce

pytestmark = pytest.mark.gpu

BIN = Path(__file__).resolve().parents[1] / "residual-stream-burden_amd" / "sihc_hip" / "sihc_abi_selftest"


def test_c_caller_of_the_abi():
    announce("C ABI self-test")
    assert BIN.exists(), f"{BIN} is missing: build with python residual-stream-burden_amd/build.py"
    proc = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=120)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "all checks passed" in proc.stdout
    assert proc.stdout.count("chain: ") == 8, "the chained backward checks did not run"
