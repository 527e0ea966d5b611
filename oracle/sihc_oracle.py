"""CPU oracle of the SiHC read/write path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module, and only as the checker / the timed CPU baseline. The product (sihc_hip)
never calls it and has no CPU fallback.

Two independent restatements of the reference's algorithm live here:

1. `read_torch` / `write_torch` / `triangular_torch` and the stage schedules: plain
   PyTorch on CPU with the reference's rounding sites (fp32 products, one cast at the
   output), following tongtongliang/residual-stream-burden
   sihc/bench/fusion_controls.py:14-85, sihc/models/sihc/reference.py:22-84 and the
   adjoint formulas of sihc/docs/kernel_fusion/README.md:36-84.
2. `brute_*`: explicit loops in float64 over tokens, slots and channels, written from
   the index map of sihc/models/sihc/sublayer_kernels.py:21-25 (`_high_offsets`).
   They share no code with (1) and generate the committed golden fixtures.

Pins (tests/test_oracle.py): the reference's known-answer slot order
(research/tests/test_reference_variants.py:85-94), bit-exact cell round trips, (1)
against (2) on the golden fixtures, adjoint identities, the identity-initialised
stage (test_reference_variants.py:97-123), literal recurrence == fused stage
schedule, weight gradients == autograd, and the gather/scatter index semantics
against torch advanced indexing.
"""
from __future__ import annotations

from typing import Callable, Optional, Sequence

import numpy as np
import torch
from torch import Tensor

GRID = 16


# --------------------------------------------------------------------------------
# geometry (reference.py:22-51; sublayer_kernels.py:21-25)
# --------------------------------------------------------------------------------
def cell_edge(slots: int) -> int:
    k = int(round(slots ** 0.5))
    if k * k != slots:
        raise ValueError(f"slots must be a square, got {slots}")
    return k


def high_to_cells(x: Tensor, slots: int) -> Tensor:
    """[B,H,W,C] carrier -> [B, G*G, S, C] cells (reference.py:22-35)."""
    b, h, w, c = x.shape
    k = cell_edge(slots)
    g = h // k
    return x.reshape(b, g, k, g, k, c).permute(0, 1, 3, 2, 4, 5).reshape(b, g * g, k * k, c)


def cells_to_high(cells: Tensor) -> Tensor:
    """Inverse of high_to_cells (reference.py:37-51)."""
    b, n, s, c = cells.shape
    g, k = int(round(n ** 0.5)), cell_edge(s)
    return cells.reshape(b, g, g, k, k, c).permute(0, 1, 3, 2, 4, 5).reshape(b, g * k, g * k, c)


def carrier_offset(m: int, s: int, c: int, channels: int, grid: int, k: int) -> int:
    """Flat NHWC offset of (token m, slot s, channel c): `_high_offsets`, :21-25."""
    n = m % (grid * grid)
    b = m // (grid * grid)
    row = b * grid * k + (n // grid) * k + s // k
    col = (n % grid) * k + s % k
    return (row * grid * k + col) * channels + c


# --------------------------------------------------------------------------------
# (1) PyTorch restatement with the reference's rounding sites
# --------------------------------------------------------------------------------
def _acc(t: Tensor) -> Tensor:
    """Accumulation type: fp32 for fp32/bf16 tensors (the reference's `.float()`),
    fp64 for fp64 tensors (used only to pin the algebra tightly)."""
    return t.double() if t.dtype == torch.float64 else t.float()


def read_torch(x: Tensor, alpha_cs: Tensor) -> Tensor:
    """One event's read, alpha [C,S]: fusion_controls.py:14-20 (grid from x and S)."""
    b, h, _, c = x.shape
    k = cell_edge(alpha_cs.shape[1])
    g = h // k
    cells = x.reshape(b, g, k, g, k, c)
    weights = alpha_cs.T.reshape(1, 1, k, 1, k, c)
    return (_acc(cells) * _acc(weights)).sum((2, 4)).reshape(b, g * g, c).to(x.dtype)


def write_torch(x: Tensor, updates: Sequence[Tensor], betas: Sequence[Tensor], add_x: bool = True) -> Tensor:
    """x + sum_e beta_e dz_e with [C,S] betas: fusion_controls.py:23-31."""
    b, h, _, c = x.shape
    k = cell_edge(betas[0].shape[1])
    g = h // k
    value = _acc(x.reshape(b, g, k, g, k, c))
    if not add_x:
        value = torch.zeros_like(value)
    for dz, beta in zip(updates, betas):
        delta = _acc(dz.reshape(b, g, 1, g, 1, c))
        weight = _acc(beta.T.reshape(1, 1, k, 1, k, c))
        value = value + delta * weight
    return value.reshape_as(x).to(x.dtype)


def triangular_torch(base: Tensor, updates: Sequence[Tensor], gamma: Tensor) -> Tensor:
    """base + sum_j gamma_j dz_j: fusion_controls.py:34-38."""
    value = _acc(base)
    for j, dz in enumerate(updates):
        value = value + _acc(dz) * _acc(gamma[j])
    return value.to(base.dtype)


def read(x: Tensor, alpha: Tensor) -> list[Tensor]:
    """Stacked read, alpha [E,C,S] -> E workspace tensors (the sublayer_read op)."""
    return [read_torch(x, a) for a in alpha.unbind(0)]


def write(x: Tensor, updates: Sequence[Tensor], beta: Tensor, add_x: bool = True) -> Tensor:
    """Stacked write, beta [E,C,S] (the sublayer_write / _write_impl op)."""
    return write_torch(x, updates, list(beta.unbind(0)), add_x=add_x)


def weight_grad(x: Tensor, updates: Sequence[Tensor], slots: int) -> Tensor:
    """[E,C,S] fp32: sum_m cells(x)[m,s,c] * z_e[m,c] (README.md:73-84 adjoints)."""
    cells = high_to_cells(x, slots).double()
    z = torch.stack([u.double() for u in updates])          # [E,B,N,C]
    return torch.einsum("bnsc,ebnc->ecs", cells, z).float()


def triangular_gamma_grad(grad: Tensor, updates: Sequence[Tensor]) -> Tensor:
    """[A,C] fp32: sum over rows of grad * dz_j (sublayer_kernels.py:324-334 semantics)."""
    g = grad.double().reshape(-1, grad.shape[-1])
    return torch.stack([(g * u.double().reshape(-1, g.shape[1])).sum(0) for u in updates]).float()


def triangular_backward(grad: Tensor, updates: Sequence[Tensor], gamma: Tensor) -> tuple[list[Tensor], Tensor]:
    """(update gradients, fp32 [A,C] gamma gradient) of triangular_torch.

    Update gradient j = fp32 grad * gamma_j cast to grad's dtype
    (sublayer_kernels.py:369-379; the fused kernel of kernels.py:1095-1186 stores the
    same products).
    """
    ddz = [(_acc(grad) * _acc(gamma[j])).to(grad.dtype) for j in range(len(updates))]
    return ddz, triangular_gamma_grad(grad, updates)


def cell_mean(x: Tensor, slots: int = 16) -> Tensor:
    """[B,G*G,C]: fp32 sum of each cell's pixels in slot order, times 1/S, cast to x's
    dtype (kernels.py:36-67, `_cell_mean_b4_fwd_kernel`)."""
    cells = high_to_cells(x, slots)
    acc = torch.zeros(cells[:, :, 0].shape, dtype=_acc(x).dtype)
    for s in range(slots):
        acc = acc + _acc(cells[:, :, s])
    return (acc * (1.0 / slots)).to(x.dtype)


def gamma_matrix(alpha: Tensor, beta: Tensor) -> Tensor:
    """gamma[i,j,c] = sum_s alpha_i[c,s] beta_j[c,s] (sublayer.py:60, README.md:45)."""
    return (alpha[:, None] * beta[None, :]).sum(dim=-1)


def fused_stage(x0: Tensor, alpha: Tensor, beta: Tensor,
                branches: Sequence[Callable[[Tensor], Tensor]]) -> Tensor:
    """The reference's late-materialised stage (sublayer.py:52-72) on the oracle ops."""
    base = read(x0, alpha)
    gamma = gamma_matrix(alpha, beta)
    updates: list[Tensor] = []
    for i, branch in enumerate(branches):
        z = base[i]
        if updates:
            z = triangular_torch(z, updates, gamma[i, :i])
        updates.append(branch(z))
    return write(x0, updates, beta)


def literal_stage(x0: Tensor, alpha: Tensor, beta: Tensor,
                  branches: Sequence[Callable[[Tensor], Tensor]]) -> Tensor:
    """Per-event recurrence (fusion_controls.py:64,80, implementation "literal")."""
    x = x0
    for i, branch in enumerate(branches):
        z = read_torch(x, alpha[i])
        dz = branch(z)
        x = write_torch(x, [dz], [beta[i]])
    return x


def event_forward(x: Tensor, dz: Tensor, beta_cs: Tensor, alpha_next_cs: Optional[Tensor]):
    """(write_torch(x, [dz], [beta]), read_torch of that carrier with alpha_next)."""
    x_out = write_torch(x, [dz], [beta_cs])
    z_out = None if alpha_next_cs is None else read_torch(x_out, alpha_next_cs)
    return x_out, z_out


def event_backward(grad_x_out: Optional[Tensor], grad_z_out: Optional[Tensor], x_out: Tensor, dz: Tensor,
                   beta_cs: Tensor, alpha_next_cs: Optional[Tensor]):
    """fp64 adjoint of event_forward: (grad_x, grad_dz, grad_beta, grad_alpha_next).

    t = h + alpha_next (x) g ; grad_dz = sum_s beta t ; grad_beta = sum_m dz t ;
    grad_alpha_next = sum_m x_out g  (README.md:73-84 with one event).
    """
    s = beta_cs.shape[1]
    cells_shape = high_to_cells(x_out, s).shape
    h = torch.zeros(cells_shape, dtype=torch.float64) if grad_x_out is None \
        else high_to_cells(grad_x_out, s).double()
    g = None if grad_z_out is None else grad_z_out.double()
    t = h.clone()
    grad_alpha = None
    if g is not None:
        t = t + g.unsqueeze(2) * alpha_next_cs.double().T[None, None]
        grad_alpha = torch.einsum("bnsc,bnc->cs", high_to_cells(x_out, s).double(), g)
    grad_dz = (t * beta_cs.double().T[None, None]).sum(2)
    grad_beta = torch.einsum("bnsc,bnc->cs", t, dz.double())
    return cells_to_high(t), grad_dz, grad_beta, grad_alpha


def gather_cells(x: Tensor, index: Optional[Tensor], slots: int) -> Tensor:
    """cells[b,n] = high_to_cells(x)[b, index[b,n]] by torch advanced indexing."""
    cells = high_to_cells(x, slots)
    if index is None:
        return cells.clone()
    b = torch.arange(cells.shape[0])[:, None]
    return cells[b, index.long()]


def scatter_cells(cells: Tensor, index: Optional[Tensor]) -> Tensor:
    """Inverse of gather_cells for a permutation index (index_copy semantics)."""
    if index is None:
        return cells_to_high(cells)
    out = torch.empty_like(cells)
    b = torch.arange(cells.shape[0])[:, None]
    out[b, index.long()] = cells
    return cells_to_high(out)


def scatter_add_cells(cells: Tensor, index: Tensor) -> Tensor:
    """Adjoint of gather_cells for any in-range index (repeats allowed): state n of batch
    b receives the fp32 sum, over the tokens t with index[b,t] == n in ascending t, of
    cells[b,t], rounded once to the cells' dtype; states no token selects are zero. The
    sum starts from -0.0 (the identity of fp32 addition: one contributor is copied bit
    for bit). Builder-defined semantics (the reference has no indexed variant); pinned
    by torch's index_add_ on exactly representable sums and by the permutation case,
    where it must equal scatter_cells."""
    b_n, n_tok, s_n, c = cells.shape
    acc = torch.full((b_n, n_tok, s_n, c), -0.0, dtype=torch.float32)
    hits = torch.zeros(b_n, n_tok, dtype=torch.int64)
    rows = torch.arange(b_n)
    idx = index.long()
    for t in range(n_tok):  # one index per batch row per step: no conflicts within a step
        acc[rows, idx[:, t]] += cells[:, t].float()
        hits[rows, idx[:, t]] += 1
    acc[hits == 0] = 0.0
    return cells_to_high(acc.to(cells.dtype))


# --------------------------------------------------------------------------------
# (2) float64 brute force (explicit loops; small shapes only)
# --------------------------------------------------------------------------------
def brute_read(x: np.ndarray, alpha: np.ndarray) -> np.ndarray:
    """x [B,H,W,C] flat-indexed via carrier_offset; alpha [E,C,S] -> [E,B,G*G,C]."""
    b, h, _, c = x.shape
    e_n, _, s_n = alpha.shape
    k = cell_edge(s_n)
    g = h // k
    flat = x.reshape(-1).astype(np.float64)
    out = np.zeros((e_n, b * g * g, c))
    for m in range(b * g * g):
        for ch in range(c):
            vals = [flat[carrier_offset(m, s, ch, c, g, k)] for s in range(s_n)]
            for e in range(e_n):
                out[e, m, ch] = sum(float(alpha[e, ch, s]) * vals[s] for s in range(s_n))
    return out.reshape(e_n, b, g * g, c)


def brute_write(x: np.ndarray, updates: np.ndarray, beta: np.ndarray, add_x: bool = True) -> np.ndarray:
    """updates [E,B,G*G,C], beta [E,C,S] -> carrier like x (float64)."""
    b, h, _, c = x.shape
    e_n, _, s_n = beta.shape
    k = cell_edge(s_n)
    g = h // k
    src = x.reshape(-1).astype(np.float64)
    out = src.copy() if add_x else np.zeros_like(src)
    upd = updates.reshape(e_n, b * g * g, c).astype(np.float64)
    for m in range(b * g * g):
        for ch in range(c):
            for s in range(s_n):
                off = carrier_offset(m, s, ch, c, g, k)
                out[off] += sum(float(beta[e, ch, s]) * upd[e, m, ch] for e in range(e_n))
    return out.reshape(x.shape)


def brute_weight_grad(x: np.ndarray, updates: np.ndarray, slots: int) -> np.ndarray:
    """[E,C,S] = sum_m x[m,s,c] * z_e[m,c] (float64)."""
    b, h, _, c = x.shape
    k = cell_edge(slots)
    g = h // k
    e_n = updates.shape[0]
    flat = x.reshape(-1).astype(np.float64)
    upd = updates.reshape(e_n, b * g * g, c).astype(np.float64)
    out = np.zeros((e_n, c, slots))
    for m in range(b * g * g):
        for ch in range(c):
            for s in range(slots):
                xv = flat[carrier_offset(m, s, ch, c, g, k)]
                for e in range(e_n):
                    out[e, ch, s] += xv * upd[e, m, ch]
    return out


def brute_triangular(base: np.ndarray, updates: np.ndarray, gamma: np.ndarray) -> np.ndarray:
    out = base.astype(np.float64).copy()
    for j in range(updates.shape[0]):
        for idx in np.ndindex(base.shape):
            out[idx] += float(gamma[j, idx[-1]]) * float(updates[j][idx])
    return out


def brute_gather(x: np.ndarray, index: np.ndarray, slots: int) -> np.ndarray:
    """cells[b,n,s,:] = x[pixel(index[b,n], s), :] from carrier_offset (exact copies)."""
    b, h, _, c = x.shape
    k = cell_edge(slots)
    g = h // k
    flat = x.reshape(-1)
    out = np.empty((b, g * g, slots, c), dtype=x.dtype)
    for bi in range(b):
        for n in range(g * g):
            m_src = bi * g * g + int(index[bi, n])
            for s in range(slots):
                off = carrier_offset(m_src, s, 0, c, g, k)
                out[bi, n, s] = flat[off:off + c]
    return out


__all__ = [name for name in dir() if not name.startswith("_")]
