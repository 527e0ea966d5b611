"""Block-wise adapters over the HIP `sihc::` ops.

Mirror of the reference's sihc/models/sihc/blockwise_kernels.py:15-38: the same
three functions and checks (8/12-block stages, 1..11 active triangular updates),
routed to the HIP-backed ops of `sublayer_kernels`.
"""
from __future__ import annotations

from torch import Tensor

from .sublayer_kernels import sublayer_read, sublayer_triangular, sublayer_write


def _require_block_events(weights: Tensor) -> None:
    if weights.ndim != 3 or weights.shape[0] not in (8, 12):
        raise ValueError("block-wise weights must have shape [8 or 12, channels, slots]")


def blockwise_read(x: Tensor, alpha: Tensor) -> list[Tensor]:
    """Base reads of an 8- or 12-block stage, one workspace tensor per block."""
    _require_block_events(alpha)
    return sublayer_read(x, alpha)


def blockwise_write(x: Tensor, updates: list[Tensor], beta: Tensor) -> Tensor:
    """Stage-end carrier: x plus the 8 or 12 block updates through beta."""
    _require_block_events(beta)
    return sublayer_write(x, updates, beta)


def blockwise_triangular(base: Tensor, updates: list[Tensor], gamma: Tensor) -> Tensor:
    """Block read of the stage: base plus gamma-weighted earlier block updates (1..11)."""
    if not 1 <= len(updates) <= 11:
        raise ValueError("block-wise triangular accumulation requires 1..11 active updates")
    return sublayer_triangular(base, updates, gamma)


__all__ = ["blockwise_read", "blockwise_write", "blockwise_triangular"]
