"""CPU: bench.py's command-line contract that needs no GPU.

This build measures one GPU: `--gpus N` with N > 1 (or a WORLD_SIZE above 1, as under
torch.distributed.run) must exit with status 2 and say why, before touching a device.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

BENCH = Path(__file__).resolve().parents[1] / "bench.py"


def _run(args, env_extra=None):
    env = dict(os.environ)
    env.update(env_extra or {})
    return subprocess.run([sys.executable, str(BENCH), *args], capture_output=True, text=True, timeout=120, env=env)


def test_more_than_one_gpu_is_refused_with_a_message():
    proc = _run(["--gpus", "2"])
    assert proc.returncode == 2, proc.stderr
    assert "one GPU only" in proc.stderr


def test_a_multi_rank_launch_is_refused():
    proc = _run(["--gpus", "1"], {"WORLD_SIZE": "4"})
    assert proc.returncode == 2, proc.stderr
    assert "one GPU only" in proc.stderr
