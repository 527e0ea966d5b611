"""Parity helpers shared by the GPU tests."""
from __future__ import annotations

import os
import sys

import torch


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def assert_parity(actual: torch.Tensor, expected: torch.Tensor, dtype: torch.dtype, *, what: str = "") -> None:
    """The tier's parity bar, relative to the output's own scale.

    fp32: max-abs error <= 1e-5 * max|expected| and relative L2 <= 1e-5.
    bf16: max-abs error <= 2e-2 * max(1, max|expected|) and relative L2 <= 1e-2
          (bf16 outputs with fp32 accumulation; the max(1, .) scaling only matters for
          large-magnitude reductions such as weight gradients over many tokens).
    """
    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    assert torch.isfinite(a).all() == torch.isfinite(e).all(), f"{what}: finiteness differs"
    scale = float(e.abs().max()) if e.numel() else 0.0
    err = float((a - e).abs().max()) if e.numel() else 0.0
    r = rel_l2(a, e) if e.numel() and float(e.norm()) > 0 else err
    if dtype == torch.float32:
        assert err <= 1e-5 * max(scale, 1e-30), f"{what}: fp32 max-abs {err:.3e} > 1e-5 * {scale:.3e}"
        assert r <= 1e-5, f"{what}: fp32 rel-L2 {r:.3e} > 1e-5"
    else:
        assert err <= 2e-2 * max(1.0, scale), f"{what}: bf16 max-abs {err:.3e} > 2e-2 * max(1, {scale:.3e})"
        assert r <= 1e-2, f"{what}: bf16 rel-L2 {r:.3e} > 1e-2"


def announce(msg: str) -> None:
    """Name the case on stdout before a GPU step (survives a box that dies mid-step)."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()
    os.fsync(sys.stdout.fileno()) if hasattr(sys.stdout, "fileno") and _is_file(sys.stdout) else None


def _is_file(stream) -> bool:
    try:
        return os.path.isfile(f"/proc/self/fd/{stream.fileno()}")
    except Exception:
        return False
