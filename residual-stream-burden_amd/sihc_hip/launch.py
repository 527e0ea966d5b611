"""Tensor-level launchers over the C ABI (include/sihc_hip.h).

Each function allocates its outputs from the PyTorch caching allocator, passes raw
device pointers to libsihc_hip.so and enqueues on the current HIP stream of the
inputs' device. No host synchronisation happens here, so the launchers are safe
under HIP-graph capture. Shape/layout validation that the reference performs in
Python lives in the op modules (sublayer_kernels, event_ops, indexed); these
launchers only assert what the C ABI itself needs.
"""
from __future__ import annotations

import ctypes
import functools
from typing import Optional, Sequence

import torch
from torch import Tensor

from ._lib import DTYPE_BF16, DTYPE_F32, MAX_EVENTS, check, lib, ptr_array

_DTYPES = {torch.float32: DTYPE_F32, torch.bfloat16: DTYPE_BF16}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}: expected float32 or bfloat16") from None


def _on_tensor_device(fn):
    """Run a launcher with its first tensor argument's GPU as the current HIP device:
    the library launches on that device's current stream and sizes grids from the
    current device's properties, which must be the same device."""

    @functools.wraps(fn)
    def wrapper(*args, **kwargs):
        dev = next((a.device for a in (*args, *kwargs.values()) if isinstance(a, Tensor) and a.is_cuda), None)
        if dev is None or dev.index is None or dev.index == torch.cuda.current_device():
            return fn(*args, **kwargs)
        with torch.cuda.device(dev):
            return fn(*args, **kwargs)

    return wrapper


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t: Optional[Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _workspace(nbytes: int, device: torch.device) -> Tensor:
    # Rounded up to 16 floats; torch allocations are at least 256-byte aligned.
    return torch.empty((max(nbytes, 4) + 63) // 64 * 16, dtype=torch.float32, device=device)


def carrier_geometry(x: Tensor, slots: int) -> tuple[int, int, int, int]:
    """(batch, grid, cell, channels) of a packed NHWC carrier with `slots` per cell."""
    b, h, w, c = x.shape
    k = 2 if slots == 4 else 4
    return b, h // k, k, c


@_on_tensor_device
def read(x: Tensor, alpha: Tensor, index: Optional[Tensor] = None,
         out: Optional[Sequence[Tensor]] = None) -> list[Tensor]:
    """E base reads of carrier x [B,H,W,C] with stacked alpha [E,C,S] (into `out` if given)."""
    b, g, k, c = carrier_geometry(x, alpha.shape[2])
    events = alpha.shape[0]
    if out is None:
        out = [torch.empty((b, g * g, c), device=x.device, dtype=x.dtype) for _ in range(events)]
    out = list(out)
    check(lib().sihc_read(x.data_ptr(), alpha.data_ptr(), ptr_array(o.data_ptr() for o in out), events,
                          b, g, k, c, _ptr(index), dtype_code(x.dtype), _stream(x.device)))
    return out


@_on_tensor_device
def write(x: Tensor, updates: Sequence[Tensor], beta: Tensor, add_x: bool = True,
          index: Optional[Tensor] = None, out: Optional[Tensor] = None) -> Tensor:
    """(add_x ? x : 0) + sum_e beta_e * updates_e written into a new carrier."""
    b, g, k, c = carrier_geometry(x, beta.shape[2])
    if out is None:
        out = torch.empty_like(x)
    check(lib().sihc_write(x.data_ptr() if add_x else None, ptr_array(u.data_ptr() for u in updates),
                           beta.data_ptr(), out.data_ptr(), len(updates), b, g, k, c, int(add_x),
                           _ptr(index), dtype_code(x.dtype), dtype_code(beta.dtype), _stream(x.device)))
    return out


@_on_tensor_device
def weight_grad(x: Tensor, updates: Sequence[Tensor], weights: Optional[Tensor],
                index: Optional[Tensor] = None, out_dtype: Optional[torch.dtype] = None,
                slots: Optional[int] = None) -> Tensor:
    """[E,C,S] = sum over tokens of x[m,s,c] * updates_e[m,c], reduced in fp32.

    Stored in out_dtype (default: the weights' dtype); `slots` and `out_dtype` stand in
    for `weights` when there is no weight tensor at hand.
    """
    b, g, k, c = carrier_geometry(x, slots if weights is None else weights.shape[-1])
    events = len(updates)
    out = torch.empty((events, c, k * k), device=x.device, dtype=out_dtype or weights.dtype)
    L = lib()
    nbytes = L.sihc_weight_grad_workspace_size(events, b, g, k, c)
    ws = _workspace(nbytes, x.device)
    check(L.sihc_weight_grad(x.data_ptr(), ptr_array(u.data_ptr() for u in updates), out.data_ptr(), events,
                             b, g, k, c, _ptr(index), dtype_code(x.dtype), dtype_code(out.dtype),
                             ws.data_ptr(), ws.numel() * 4, _stream(x.device)))
    return out


@_on_tensor_device
def triangular(base: Tensor, updates: Sequence[Tensor], gamma: Tensor) -> Tensor:
    """base + sum_j gamma[j] * updates_j over a [B,N,C] workspace."""
    c = base.shape[-1]
    rows = base.numel() // c if c else 0
    out = torch.empty_like(base)
    check(lib().sihc_triangular(base.data_ptr(), ptr_array(u.data_ptr() for u in updates), gamma.data_ptr(),
                                out.data_ptr(), len(updates), rows, c, dtype_code(base.dtype),
                                dtype_code(gamma.dtype), _stream(base.device)))
    return out


@_on_tensor_device
def triangular_gamma_grad(grad: Tensor, updates: Sequence[Tensor], gamma: Optional[Tensor],
                          out_dtype: Optional[torch.dtype] = None) -> Tensor:
    """[A,C] (out_dtype, default gamma's dtype) = sum over rows of grad * updates_j."""
    c = grad.shape[-1]
    rows = grad.numel() // c if c else 0
    active = len(updates)
    out = torch.empty((active, c), device=grad.device, dtype=out_dtype or gamma.dtype)
    L = lib()
    ws = _workspace(L.sihc_triangular_gamma_grad_workspace_size(active, rows, c), grad.device)
    check(L.sihc_triangular_gamma_grad(grad.data_ptr(), ptr_array(u.data_ptr() for u in updates),
                                       out.data_ptr(), active, rows, c, dtype_code(grad.dtype),
                                       dtype_code(out.dtype), ws.data_ptr(), ws.numel() * 4,
                                       _stream(grad.device)))
    return out


@_on_tensor_device
def triangular_backward(grad: Tensor, updates: Sequence[Tensor], gamma: Tensor,
                        out_dtype: Optional[torch.dtype] = None) -> tuple[Tensor, Tensor]:
    """One pass: ([A,B,N,C] stack of grad * gamma[j], [A,C] sum over rows of grad * updates_j).

    The update gradients share grad's dtype; the gamma gradient is out_dtype (default
    gamma's dtype), reduced in fp32.
    """
    c = grad.shape[-1]
    rows = grad.numel() // c if c else 0
    active = len(updates)
    ddz = torch.empty((active, *grad.shape), device=grad.device, dtype=grad.dtype)
    dg = torch.empty((active, c), device=grad.device, dtype=out_dtype or gamma.dtype)
    L = lib()
    ws = _workspace(L.sihc_triangular_gamma_grad_workspace_size(active, rows, c), grad.device)
    check(L.sihc_triangular_backward(grad.data_ptr(), ptr_array(u.data_ptr() for u in updates), gamma.data_ptr(),
                                     ptr_array(d.data_ptr() for d in ddz.unbind(0)), dg.data_ptr(), active, rows,
                                     c, dtype_code(grad.dtype), dtype_code(gamma.dtype), dtype_code(dg.dtype),
                                     ws.data_ptr(), ws.numel() * 4, _stream(grad.device)))
    return ddz, dg


@_on_tensor_device
def event_forward(x: Tensor, dz: Tensor, beta: Tensor, alpha_next: Optional[Tensor],
                  index: Optional[Tensor] = None) -> tuple[Tensor, Optional[Tensor]]:
    """x_out = x + beta*dz and z_out = read(x_out, alpha_next) in one pass."""
    b, g, k, c = carrier_geometry(x, beta.shape[1])
    x_out = torch.empty_like(x)
    z_out = None if alpha_next is None else torch.empty((b, g * g, c), device=x.device, dtype=x.dtype)
    check(lib().sihc_event_forward(x.data_ptr(), dz.data_ptr(), beta.data_ptr(), _ptr(alpha_next),
                                   x_out.data_ptr(), _ptr(z_out), b, g, k, c, _ptr(index),
                                   dtype_code(x.dtype), _stream(x.device)))
    return x_out, z_out


@_on_tensor_device
def event_backward(grad_x_out: Optional[Tensor], grad_z_out: Optional[Tensor], x_out: Optional[Tensor],
                   dz: Optional[Tensor], beta: Optional[Tensor], alpha_next: Optional[Tensor],
                   index: Optional[Tensor] = None, grad_x: Optional[Tensor] = None,
                   alias_grad_x: bool = False, carrier_like: Optional[Tensor] = None):
    """Adjoint of event_forward: (grad_x, grad_dz, grad_beta, grad_alpha_next).

    `beta`/`dz` None drops the write part (adjoint of a plain read). With
    `alias_grad_x` and no read part, grad_x is grad_x_out itself (not copied).
    `carrier_like` supplies the carrier shape when x_out is None.
    """
    ref = x_out if x_out is not None else (carrier_like if carrier_like is not None else grad_x_out)
    w = beta if beta is not None else alpha_next
    for t in (beta, alpha_next):
        if t is not None and t.dtype != ref.dtype:
            raise ValueError(f"event weights must share the carrier dtype {ref.dtype}, got {t.dtype}")
    b, g, k, c = carrier_geometry(ref, w.shape[1])
    alias = alias_grad_x and grad_z_out is None
    if alias:
        grad_x = grad_x_out
    elif grad_x is None:
        grad_x = torch.empty(ref.shape, device=ref.device, dtype=ref.dtype)
    grad_dz = None if beta is None else torch.empty((b, g * g, c), device=ref.device, dtype=ref.dtype)
    grad_beta = None if beta is None else torch.empty_like(beta)
    grad_alpha = None if alpha_next is None else torch.empty_like(alpha_next)
    L = lib()
    ws = _workspace(L.sihc_event_backward_workspace_size(b, g, k, c), ref.device)
    check(L.sihc_event_backward(_ptr(grad_x_out), _ptr(grad_z_out), _ptr(x_out), _ptr(dz), _ptr(beta),
                                _ptr(alpha_next), None if alias else grad_x.data_ptr(), _ptr(grad_dz),
                                _ptr(grad_beta), _ptr(grad_alpha), b, g, k, c, _ptr(index),
                                dtype_code(ref.dtype), dtype_code(w.dtype), ws.data_ptr(),
                                ws.numel() * 4, _stream(ref.device)))
    return grad_x, grad_dz, grad_beta, grad_alpha


@_on_tensor_device
def gather_cells(x: Tensor, index: Optional[Tensor], slots: int) -> Tensor:
    """[B,G*G,S,C] bit-exact copy of each token's cell (cell index[b,n] when given)."""
    b, g, k, c = carrier_geometry(x, slots)
    cells = torch.empty((b, g * g, k * k, c), device=x.device, dtype=x.dtype)
    check(lib().sihc_gather_cells(x.data_ptr(), _ptr(index), cells.data_ptr(), b, g, k, c,
                                  dtype_code(x.dtype), _stream(x.device)))
    return cells


@_on_tensor_device
def scatter_cells(cells: Tensor, index: Optional[Tensor], out: Optional[Tensor] = None) -> Tensor:
    """Inverse of gather_cells for a permutation index: new (or `out`) NHWC carrier."""
    b, n, s, c = cells.shape
    k = 2 if s == 4 else 4
    g = int(round(n ** 0.5))
    if out is None:
        out = torch.empty((b, g * k, g * k, c), device=cells.device, dtype=cells.dtype)
    check(lib().sihc_scatter_cells(cells.data_ptr(), _ptr(index), out.data_ptr(), b, g, k, c,
                                   dtype_code(cells.dtype), _stream(cells.device)))
    return out


@_on_tensor_device
def scatter_add_cells(cells: Tensor, index: Optional[Tensor], out: Optional[Tensor] = None) -> Tensor:
    """Adjoint of gather_cells for any in-range index (repeats allowed): each carrier cell
    gets the fp32 sum, in ascending token order, of the cells rows that select it, and
    zeros where none does. Equals scatter_cells bit for bit for a permutation index."""
    b, n, s, c = cells.shape
    k = 2 if s == 4 else 4
    g = int(round(n ** 0.5))
    if out is None:
        out = torch.empty((b, g * k, g * k, c), device=cells.device, dtype=cells.dtype)
    check(lib().sihc_scatter_add_cells(cells.data_ptr(), _ptr(index), out.data_ptr(), b, g, k, c,
                                       dtype_code(cells.dtype), _stream(cells.device)))
    return out


@_on_tensor_device
def copy_(dst: Tensor, src: Tensor) -> Tensor:
    """Byte copy src -> dst (same number of bytes) with the library's copy kernel."""
    nbytes = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() != nbytes:
        raise ValueError("copy_ needs equally sized tensors")
    check(lib().sihc_copy(src.data_ptr(), dst.data_ptr(), nbytes, _stream(src.device)))
    return dst


__all__ = [
    "MAX_EVENTS", "dtype_code", "carrier_geometry", "read", "write", "weight_grad", "triangular",
    "triangular_gamma_grad", "triangular_backward", "event_forward", "event_backward", "gather_cells",
    "scatter_cells", "scatter_add_cells", "copy_",
]
