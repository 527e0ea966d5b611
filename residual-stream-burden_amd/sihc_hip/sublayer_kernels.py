"""Drop-in `sublayer_kernels` for MI355X: the `sihc::` custom ops on HIP kernels.

Same op names, Python signatures, autograd rules, fake (meta) implementations and
ValueError contract as the reference module
sihc/models/sihc/sublayer_kernels.py (tongtongliang/residual-stream-burden), so
`from .sublayer_kernels import sublayer_read, sublayer_triangular, sublayer_write`
in the reference's sublayer.py:11 and blockwise_kernels.py:12 resolves to this
module unchanged. Every op body calls libsihc_hip.so through `launch`; there is no
Triton, no bf16-MMA dispatch (reference :196-216) and no CPU fallback.

Generalisation over the reference: any event count in 1..32 (reference: 8/12/16/24,
:186) and any channel count, including tails.
"""
from __future__ import annotations

import torch
from torch import Tensor
from torch.library import custom_op, register_autograd

from . import launch

MAX_EVENTS = launch.MAX_EVENTS


def _require_packed(op_name: str, **tensors: Tensor) -> None:
    """Reject views incompatible with linear indexing (reference kernels.py:26-32)."""
    for tensor_name, tensor in tensors.items():
        if not tensor.is_contiguous():
            raise ValueError(
                f"{op_name} requires contiguous {tensor_name}, got stride {tensor.stride()}")


def _geometry(x: Tensor, weights: Tensor) -> tuple[int, int, int, int]:
    """(batch, channels, grid, cell) of a carrier and its stacked weights.

    Follows reference sublayer_kernels.py:180-193, with events widened to 1..32.
    """
    _require_packed("sublayer read/write", x=x, weights=weights)
    if x.ndim != 4 or weights.ndim != 3:
        raise ValueError("expected NHWC carrier and [events, channels, slots] weights")
    b, h, w, c = x.shape
    events, wc, slots = weights.shape
    if not 1 <= events <= MAX_EVENTS or wc != c or slots not in (4, 16):
        raise ValueError(f"fused stages require 1..{MAX_EVENTS} events and 4/16 spatial slots")
    k = 2 if slots == 4 else 4
    if h != w or h % k:
        raise ValueError("carrier grid must be square and divisible by the slot grid")
    if x.dtype != weights.dtype or x.device != weights.device or not x.is_cuda:
        raise ValueError("carrier and weights must share CUDA device and dtype")
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("carrier dtype must be float32 or bfloat16")
    return b, c, h // k, k


def _validate_updates(x: Tensor, weights: Tensor, updates: list[Tensor]):
    """Reference sublayer_kernels.py:235-243."""
    b, c, g, k = _geometry(x, weights)
    if len(updates) != weights.shape[0]:
        raise ValueError("one workspace update is required per connection event")
    for dz in updates:
        _require_packed("sublayer write", update=dz)
        if dz.shape != (b, g * g, c) or dz.dtype != x.dtype or dz.device != x.device:
            raise ValueError("update geometry, dtype, or device does not match carrier")
    return b, c, g, k


@custom_op("sihc::sublayer_read", mutates_args=())
def sublayer_read(x: Tensor, alpha: Tensor) -> list[Tensor]:
    """E base reads z_e = sum_s alpha_e[:, s] * x[cell slot s] (reference :219-232)."""
    _geometry(x, alpha)
    return launch.read(x, alpha)


@custom_op("sihc::sublayer_write_impl", mutates_args=())
def _write_impl(x: Tensor, updates: list[Tensor], beta: Tensor, add_x: bool) -> Tensor:
    """(add_x ? x : 0) + sum_e beta_e * dz_e on the carrier (reference :246-258)."""
    _validate_updates(x, beta, updates)
    return launch.write(x, updates, beta, add_x=add_x)


@custom_op("sihc::sublayer_weight_grad", mutates_args=())
def _weights_backward(x: Tensor, updates: list[Tensor], weights: Tensor) -> Tensor:
    """[E,C,S] sum over tokens of x * z_e, fp32 then cast (reference :261-273).

    Atomics-free and deterministic (the reference uses fp32 atomic_add).
    """
    _validate_updates(x, weights, updates)
    return launch.weight_grad(x, updates, weights)


def _read_setup(ctx, inputs, output):
    ctx.save_for_backward(*inputs)


def _read_backward(ctx, grads):
    """Reference :280-284. Events whose output received no gradient are skipped
    instead of materialising zero tensors; their dalpha rows are exactly zero."""
    x, alpha = ctx.saved_tensors
    used = [i for i, g in enumerate(grads) if g is not None]
    if not used:
        return torch.zeros_like(x), torch.zeros_like(alpha)
    gs = [grads[i].contiguous() for i in used]
    if len(used) == alpha.shape[0]:
        a = alpha
    else:
        a = alpha[used].contiguous()
    dx = _write_impl(x, gs, a, False)
    da_used = _weights_backward(x, gs, a)
    if len(used) == alpha.shape[0]:
        return dx, da_used
    da = alpha.new_zeros(alpha.shape)
    da[used] = da_used
    return dx, da


register_autograd(sublayer_read, _read_backward, setup_context=_read_setup)


@custom_op("sihc::sublayer_write", mutates_args=())
def sublayer_write(x: Tensor, updates: list[Tensor], beta: Tensor) -> Tensor:
    """Stage write with identity carry (reference :290-292)."""
    return _write_impl(x, updates, beta, True)


def _write_setup(ctx, inputs, output):
    _, updates, beta = inputs
    ctx.save_for_backward(beta, *updates)


def _write_backward(ctx, grad):
    """Reference :300-303: identity to x, a read of the carrier gradient for the
    updates, and the weight reduction for beta."""
    beta, *updates = ctx.saved_tensors
    grad = grad.contiguous()
    return grad, sublayer_read(grad, beta), _weights_backward(grad, updates, beta)


register_autograd(sublayer_write, _write_backward, setup_context=_write_setup)


def _validate_triangular(base: Tensor, updates: list[Tensor], gamma: Tensor) -> None:
    """Reference :339-347 (active prefix widened to 1..32)."""
    _require_packed("sublayer triangular", base=base, gamma=gamma)
    if not 1 <= len(updates) <= MAX_EVENTS or gamma.shape != (len(updates), base.shape[-1]):
        raise ValueError(f"gamma must match the active prefix (1..{MAX_EVENTS}) and channel count")
    for dz in updates:
        _require_packed("sublayer triangular", update=dz)
        if dz.shape != base.shape or dz.dtype != base.dtype or dz.device != base.device:
            raise ValueError("active updates must match the workspace tensor")
    if gamma.device != base.device or gamma.dtype not in (base.dtype, torch.float32):
        raise ValueError("gamma must share workspace device and use workspace dtype or fp32")
    if base.dtype not in (torch.float32, torch.bfloat16) or not base.is_cuda:
        raise ValueError("workspace must be a float32 or bfloat16 CUDA tensor")


@custom_op("sihc::sublayer_triangular", mutates_args=())
def sublayer_triangular(base: Tensor, updates: list[Tensor], gamma: Tensor) -> Tensor:
    """base + sum_j gamma_j * dz_j over the active prefix (reference :337-352)."""
    _validate_triangular(base, updates, gamma)
    return launch.triangular(base, updates, gamma)


@custom_op("sihc::sublayer_triangular_gamma_backward", mutates_args=())
def _tri_gamma_backward(grad: Tensor, updates: list[Tensor], gamma: Tensor) -> Tensor:
    """dgamma_j = sum over rows of grad * dz_j, fp32 then cast (reference :355-361)."""
    return launch.triangular_gamma_grad(grad, updates, gamma)


@custom_op("sihc::sublayer_triangular_backward", mutates_args=())
def _tri_backward(grad: Tensor, updates: list[Tensor], gamma: Tensor) -> tuple[Tensor, Tensor]:
    """([A,B,N,C] update gradients grad * gamma_j, dgamma) from one pass over grad.

    Same values as the reference's backward (:369-379: fp32 products cast to the
    workspace dtype, and `_tri_gamma_backward`), with grad read once instead of A + 1
    times.
    """
    return launch.triangular_backward(grad, updates, gamma)


def _tri_setup(ctx, inputs, output):
    _, updates, gamma = inputs
    ctx.save_for_backward(gamma, *updates)


# How the triangular op's backward hands out the update gradients grad * gamma_j when
# torch.compile traces it (eager calls always take the one-pass HIP op):
#   "visible": the reference's fp32 products cast to the workspace dtype as plain torch
#              ops (:373-378), which Inductor fuses with the gradient accumulation of each
#              update, plus the gamma reduction op (:355-361);
#   "fused":   the one-pass HIP op, whose [A, B, N, C] stack of update gradients is
#              materialised before the accumulation.
COMPILED_TRIANGULAR_BACKWARD = "visible"


def _traced() -> bool:
    """True while torch.compile (AOTAutograd) traces an autograd rule. The public
    torch.compiler.is_compiling() is False there; an active tracing context is not."""
    return torch._guards.TracingContext.try_get() is not None


def _tri_autograd(ctx, grad):
    """Reference :369-379: identity to base, grad * gamma_j to each active update and
    the gamma reduction. Eager: all from one pass over grad (`_tri_backward`); under
    torch.compile the products stay visible to the compiler unless
    COMPILED_TRIANGULAR_BACKWARD is "fused"."""
    gamma, *updates = ctx.saved_tensors
    grad = grad.contiguous()
    if COMPILED_TRIANGULAR_BACKWARD == "visible" and _traced():
        g32 = grad.float()
        ddz = [(g32 * gamma[j].float()).to(grad.dtype) for j in range(len(updates))]
        return grad, ddz, _tri_gamma_backward(grad, updates, gamma)
    ddz, dg = _tri_backward(grad, updates, gamma)
    return grad, list(ddz.unbind(0)), dg


register_autograd(sublayer_triangular, _tri_autograd, setup_context=_tri_setup)


# Fake implementations (reference :387-416): device-free shape functions for fullgraph
# torch.compile and HIP-graph capture through the compiler. They run the same layout,
# geometry and update checks as the real ops (the reference's read and write fakes call
# `_geometry` / `_validate_updates`, :387-398; here the weight-gradient and triangular
# fakes check their operands too), so a bad shape fails at trace time, not at launch.
@sublayer_read.register_fake
def _read_fake(x, alpha):
    b, c, g, _ = _geometry(x, alpha)
    return [x.new_empty((b, g * g, c)) for _ in range(alpha.shape[0])]


@_write_impl.register_fake
def _write_impl_fake(x, updates, beta, add_x):
    _validate_updates(x, beta, updates)
    return torch.empty_like(x)


@sublayer_write.register_fake
def _write_fake(x, updates, beta):
    return _write_impl_fake(x, updates, beta, True)


@_weights_backward.register_fake
def _weight_fake(x, updates, weights):
    _validate_updates(x, weights, updates)
    return torch.empty_like(weights)


@sublayer_triangular.register_fake
def _tri_fake(base, updates, gamma):
    _validate_triangular(base, updates, gamma)
    return torch.empty_like(base)


@_tri_gamma_backward.register_fake
def _tri_gamma_backward_fake(grad, updates, gamma):
    _validate_triangular(grad, updates, gamma)
    return torch.empty_like(gamma)


@_tri_backward.register_fake
def _tri_backward_fake(grad, updates, gamma):
    _validate_triangular(grad, updates, gamma)
    return grad.new_empty((len(updates), *grad.shape)), torch.empty_like(gamma)


__all__ = ["sublayer_read", "sublayer_write", "sublayer_triangular", "_write_impl", "COMPILED_TRIANGULAR_BACKWARD",
           "_weights_backward", "_tri_gamma_backward", "_tri_backward", "_require_packed", "_geometry"]
