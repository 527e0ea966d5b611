"""Spatially indexed read/write: each token carries an int32 index of its state.

Specification (the reference has no such op; this module defines it):

* ``index`` is an int32 tensor [B, G*G]. Token (b, n) of the workspace is assigned
  the prediction state (carrier cell) ``index[b, n]`` of batch b: the K*K carrier
  pixels (b, wy*K+uy, wx*K+ux) with wy, wx = divmod(index[b, n], G).
* gather:  cells[b, n, s, :] = x[pixel (index[b, n], s), :]   -- bit-exact copies; any
  index with values in [0, G*G) (repeats allowed). Its adjoint is a scatter-add: each
  state receives the fp32 sum, in ascending token order, of the gradient rows of the
  tokens that selected it (zero where none did), rounded once -- atomics-free and
  deterministic, and bit-identical to the scatter for a permutation index.
* scatter: x[pixel (index[b, n], s), :] = cells[b, n, s, :]   -- index must be a
  permutation of 0..G*G-1 in every batch row (each state written exactly once)
* indexed read/write: the read/write maps applied to the gathered states, and the
  written states scattered back, fused into single passes (no gathered tile is
  materialised). With ``index[b] = arange(G*G)`` every op here is bit-identical to
  its non-indexed counterpart.

``group_index`` builds the seeded assignment used by the benchmark workload: the
G*G grid positions are shuffled per batch row, cut into consecutive groups of
``group`` positions (the last group may be smaller), each group is sorted
ascending, and the groups are concatenated in order.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor
from torch.library import custom_op, register_autograd

from . import launch
from .sublayer_kernels import _geometry, _require_packed, _validate_updates


def group_index(batch: int, grid: int = 16, group: int = 5, seed: int = 3,
                device: torch.device | str = "cpu") -> Tensor:
    """Seeded per-batch assignment of the grid into groups of `group` positions."""
    gen = torch.Generator().manual_seed(seed)
    n = grid * grid
    rows = []
    for _ in range(batch):
        perm = torch.randperm(n, generator=gen)
        parts = [perm[i:i + group].sort().values for i in range(0, n, group)]
        rows.append(torch.cat(parts))
    return torch.stack(rows).to(torch.int32).to(device)


def check_index(index: Tensor, batch: int, grid: int, *, permutation: bool, validate: bool = True) -> None:
    """Layout checks always; value checks (a host sync) when `validate`."""
    _require_packed("spatial index", index=index)
    if index.dtype != torch.int32 or index.shape != (batch, grid * grid):
        raise ValueError(f"index must be int32 [{batch}, {grid * grid}], got {index.dtype} {tuple(index.shape)}")
    if not validate or index.numel() == 0:
        return
    lo, hi = int(index.min()), int(index.max())
    if lo < 0 or hi >= grid * grid:
        raise ValueError(f"index values must lie in [0, {grid * grid}), got [{lo}, {hi}]")
    if permutation:
        ref = torch.arange(grid * grid, device=index.device, dtype=index.dtype)
        if not torch.equal(index.sort(dim=1).values, ref.expand_as(index)):
            raise ValueError("index rows must be permutations of the grid positions")


def _same_device(index: Tensor, x: Tensor) -> None:
    if index.device != x.device:
        raise ValueError("index must live on the carrier's device")


@custom_op("sihc::indexed_read", mutates_args=())
def _indexed_read(x: Tensor, alpha: Tensor, index: Tensor) -> list[Tensor]:
    _geometry(x, alpha)
    _same_device(index, x)
    return launch.read(x, alpha, index=index)


@_indexed_read.register_fake
def _indexed_read_fake(x, alpha, index):
    b, h, _, c = x.shape
    k = 2 if alpha.shape[2] == 4 else 4
    g = h // k
    return [x.new_empty((b, g * g, c)) for _ in range(alpha.shape[0])]


@custom_op("sihc::indexed_write_impl", mutates_args=())
def _indexed_write_impl(x: Tensor, updates: list[Tensor], beta: Tensor, index: Tensor, add_x: bool) -> Tensor:
    _validate_updates(x, beta, updates)
    _same_device(index, x)
    return launch.write(x, updates, beta, add_x=add_x, index=index)


@_indexed_write_impl.register_fake
def _indexed_write_impl_fake(x, updates, beta, index, add_x):
    return torch.empty_like(x)


@custom_op("sihc::indexed_weight_grad", mutates_args=())
def _indexed_weight_grad(x: Tensor, updates: list[Tensor], weights: Tensor, index: Tensor) -> Tensor:
    _validate_updates(x, weights, updates)
    return launch.weight_grad(x, updates, weights, index=index)


@_indexed_weight_grad.register_fake
def _indexed_weight_grad_fake(x, updates, weights, index):
    return weights.new_empty((len(updates), weights.shape[1], weights.shape[2]))


def _iread_setup(ctx, inputs, output):
    ctx.save_for_backward(*inputs)


def _iread_backward(ctx, grads):
    x, alpha, index = ctx.saved_tensors
    shape = (x.shape[0], x.shape[1] * x.shape[2] // alpha.shape[2], x.shape[3])
    gs = [g.contiguous() if g is not None else x.new_zeros(shape) for g in grads]
    return (_indexed_write_impl(x, gs, alpha, index, False), _indexed_weight_grad(x, gs, alpha, index), None)


register_autograd(_indexed_read, _iread_backward, setup_context=_iread_setup)


@custom_op("sihc::indexed_write", mutates_args=())
def _indexed_write(x: Tensor, updates: list[Tensor], beta: Tensor, index: Tensor) -> Tensor:
    return _indexed_write_impl(x, updates, beta, index, True)


@_indexed_write.register_fake
def _indexed_write_fake(x, updates, beta, index):
    return torch.empty_like(x)


def _iwrite_setup(ctx, inputs, output):
    _, updates, beta, index = inputs
    ctx.save_for_backward(beta, index, *updates)


def _iwrite_backward(ctx, grad):
    beta, index, *updates = ctx.saved_tensors
    grad = grad.contiguous()
    return grad, _indexed_read(grad, beta, index), _indexed_weight_grad(grad, updates, beta, index), None


register_autograd(_indexed_write, _iwrite_backward, setup_context=_iwrite_setup)


@custom_op("sihc::gather_cells", mutates_args=())
def _gather_cells(x: Tensor, index: Tensor, slots: int) -> Tensor:
    return launch.gather_cells(x, index, slots)


@_gather_cells.register_fake
def _gather_cells_fake(x, index, slots):
    b, h, _, c = x.shape
    k = 2 if slots == 4 else 4
    g = h // k
    return x.new_empty((b, g * g, slots, c))


@custom_op("sihc::scatter_cells", mutates_args=())
def _scatter_cells(cells: Tensor, index: Tensor) -> Tensor:
    return launch.scatter_cells(cells, index)


@_scatter_cells.register_fake
def _scatter_cells_fake(cells, index):
    b, n, s, c = cells.shape
    k = 2 if s == 4 else 4
    g = int(round(n ** 0.5))
    return cells.new_empty((b, g * k, g * k, c))


@custom_op("sihc::scatter_add_cells", mutates_args=())
def _scatter_add_cells(cells: Tensor, index: Tensor) -> Tensor:
    return launch.scatter_add_cells(cells, index)


@_scatter_add_cells.register_fake
def _scatter_add_cells_fake(cells, index):
    return _scatter_cells_fake(cells, index)


def _gather_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[1])


def _gather_backward(ctx, grad):
    # the gather accepts repeated indices: its adjoint sums the rows of every token
    # that selected a state (and leaves unselected states at zero)
    (index,) = ctx.saved_tensors
    return _scatter_add_cells(grad.contiguous(), index), None, None


def _scatter_setup(ctx, inputs, output):
    ctx.slots = inputs[0].shape[2]
    ctx.save_for_backward(inputs[1])


def _scatter_backward(ctx, grad):
    (index,) = ctx.saved_tensors
    return _gather_cells(grad.contiguous(), index, ctx.slots), None


register_autograd(_gather_cells, _gather_backward, setup_context=_gather_setup)
register_autograd(_scatter_cells, _scatter_backward, setup_context=_scatter_setup)


def _carrier_grid(x: Tensor, slots: int) -> tuple[int, int]:
    k = 2 if slots == 4 else 4
    return x.shape[0], x.shape[1] // k


def gather_cells(x: Tensor, index: Tensor, slots: int = 4, *, validate: bool = True) -> Tensor:
    """[B, G*G, S, C] copy of each token's state (any in-range index)."""
    if x.ndim != 4 or slots not in (4, 16):
        raise ValueError("expected NHWC carrier and 4 or 16 slots")
    _require_packed("gather_cells", x=x)
    b, g = _carrier_grid(x, slots)
    check_index(index, b, g, permutation=False, validate=validate)
    _same_device(index, x)
    return _gather_cells(x, index, slots)


def scatter_cells(cells: Tensor, index: Tensor, *, validate: bool = True) -> Tensor:
    """New NHWC carrier with every state written back (permutation index)."""
    if cells.ndim != 4 or cells.shape[2] not in (4, 16):
        raise ValueError("expected [B, G*G, S, C] cells with 4 or 16 slots")
    _require_packed("scatter_cells", cells=cells)
    g = int(round(cells.shape[1] ** 0.5))
    if g * g != cells.shape[1]:
        raise ValueError("cells must cover a square workspace grid")
    check_index(index, cells.shape[0], g, permutation=True, validate=validate)
    _same_device(index, cells)
    return _scatter_cells(cells, index)


def indexed_read(x: Tensor, alpha: Tensor, index: Tensor, *, validate: bool = True) -> list[Tensor]:
    """E reads of the indexed states: z_e[b,n] = sum_s alpha_e[:, s] * state(index[b,n])[s]."""
    b, c, g, k = _geometry(x, alpha)
    check_index(index, b, g, permutation=True, validate=validate)
    return _indexed_read(x, alpha, index)


def indexed_write(x: Tensor, updates: list[Tensor], beta: Tensor, index: Tensor, *,
                  validate: bool = True) -> Tensor:
    """Carrier with state(index[b,n]) += sum_e beta_e * updates_e[b,n]."""
    b, c, g, k = _validate_updates(x, beta, updates)
    check_index(index, b, g, permutation=True, validate=validate)
    return _indexed_write(x, updates, beta, index)


__all__ = ["group_index", "check_index", "gather_cells", "scatter_cells", "indexed_read", "indexed_write"]
