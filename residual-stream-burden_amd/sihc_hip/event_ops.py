"""Per-event fused read/write (the literal schedule) with autograd.

The reference's literal control (sihc/bench/fusion_controls.py:41-85, implementation
"literal") routes the carrier after every connection event:

    z_i     = read(X_i, alpha_i)                       read_torch,  :14-20
    dz_i    = F_i(z_i)                                 attention / MLP update
    X_{i+1} = X_i + beta_i * dz_i                      write_torch, :23-31

`sihc::event_write_read` fuses the write of event i with the read of event i+1 into
one pass over the carrier: each carrier element is read once and written once per
connection event, and the next workspace is produced from the freshly rounded
carrier (the literal schedule's rounding sites). Its backward is one pass too: the
carrier gradient, the update gradient and per-block partials of both weight
gradients, followed by a fixed-order reduction (no atomics).

`literal_stage` strings the events of one stage (or a whole network) together with
arbitrary PyTorch branch functions in between.
"""
from __future__ import annotations

from typing import Callable, Optional, Sequence

import torch
from torch import Tensor
from torch.library import custom_op, register_autograd

from . import launch
from .sublayer_kernels import _require_packed, sublayer_read, sublayer_write


def _validate_event(x: Tensor, dz: Tensor, beta: Tensor, alpha_next: Optional[Tensor]) -> None:
    _require_packed("event write/read", x=x, dz=dz, beta=beta)
    if alpha_next is not None:
        _require_packed("event write/read", alpha_next=alpha_next)
    if x.ndim != 4 or beta.ndim != 2:
        raise ValueError("expected NHWC carrier and [channels, slots] event weights")
    b, h, w, c = x.shape
    if beta.shape[0] != c or beta.shape[1] not in (4, 16):
        raise ValueError("event weights must be [channels, 4 or 16 slots]")
    if alpha_next is not None and alpha_next.shape != beta.shape:
        raise ValueError("alpha_next must have the shape of beta")
    k = 2 if beta.shape[1] == 4 else 4
    if h != w or h % k:
        raise ValueError("carrier grid must be square and divisible by the slot grid")
    g = h // k
    if dz.shape != (b, g * g, c):
        raise ValueError("update geometry does not match carrier")
    tensors = [x, dz, beta] + ([alpha_next] if alpha_next is not None else [])
    if any(t.dtype != x.dtype or t.device != x.device for t in tensors) or not x.is_cuda:
        raise ValueError("carrier, update and weights must share CUDA device and dtype")
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("carrier dtype must be float32 or bfloat16")


@custom_op("sihc::event_write_read", mutates_args=())
def event_write_read(x: Tensor, dz: Tensor, beta: Tensor, alpha_next: Tensor) -> tuple[Tensor, Tensor]:
    """(X + beta*dz, read(X + beta*dz, alpha_next)) for one event's [C,S] weights."""
    _validate_event(x, dz, beta, alpha_next)
    x_out, z_out = launch.event_forward(x, dz, beta, alpha_next)
    return x_out, z_out


@event_write_read.register_fake
def _event_write_read_fake(x, dz, beta, alpha_next):
    return torch.empty_like(x), torch.empty_like(dz)


def _event_setup(ctx, inputs, output):
    _, dz, beta, alpha_next = inputs
    ctx.save_for_backward(output[0], dz, beta, alpha_next)


@custom_op("sihc::event_write_read_backward", mutates_args=())
def _event_backward(grad_x_out: Optional[Tensor], grad_z_out: Optional[Tensor], x_out: Tensor,
                    dz: Tensor, beta: Tensor, alpha_next: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    gx, gdz, gb, ga = launch.event_backward(grad_x_out, grad_z_out, x_out, dz, beta, alpha_next)
    return gx, gdz, gb, ga


@_event_backward.register_fake
def _event_backward_fake(grad_x_out, grad_z_out, x_out, dz, beta, alpha_next):
    return (torch.empty_like(x_out), torch.empty_like(dz), torch.empty_like(beta),
            torch.empty_like(alpha_next))


def _event_autograd(ctx, grad_x_out, grad_z_out):
    x_out, dz, beta, alpha_next = ctx.saved_tensors
    if grad_x_out is not None:
        grad_x_out = grad_x_out.contiguous()
    if grad_z_out is not None:
        grad_z_out = grad_z_out.contiguous()
    return _event_backward(grad_x_out, grad_z_out, x_out, dz, beta, alpha_next)


register_autograd(event_write_read, _event_autograd, setup_context=_event_setup)


def literal_stage(x0: Tensor, alpha: Tensor, beta: Tensor,
                  branches: Sequence[Callable[[Tensor], Tensor]]) -> Tensor:
    """Literal per-event recurrence over stacked [E,C,S] weights.

    Equivalent (up to rounding sites) to the reference's fused stage schedule
    (sublayer.py:52-72), with the carrier routed after every event as in
    fusion_controls.py:64,80. Returns the carrier after the last event.
    """
    events = alpha.shape[0]
    if len(branches) != events or beta.shape[0] != events:
        raise ValueError("one branch function per connection event is required")
    z = sublayer_read(x0, alpha[:1])[0]
    x = x0
    for i, branch in enumerate(branches):
        dz = branch(z).contiguous()
        if i + 1 < events:
            x, z = event_write_read(x, dz, beta[i], alpha[i + 1])
        else:
            x = sublayer_write(x, [dz], beta[i:i + 1])
    return x


__all__ = ["event_write_read", "literal_stage"]
