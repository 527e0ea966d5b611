"""Fixed-arity block-wise `sihc::` ops (the legacy stage API) on the HIP kernels.

Drop-in for sihc/models/sihc/kernels.py of tongtongliang/residual-stream-burden, the
module model.py:30-39 imports for its fused schedule: the same Python names, op names
(`sihc::all_base_b4_12_split_traceable`, ...), argument lists with one tensor per block
update / block weight, autograd rules and shape errors. Geometry tags:

    b4_12, b4_8   carrier [B, 64, 64, C], 4x4 cells (16 slots), 12 or 8 blocks
    p8_12         carrier [B, 32, 32, C], 2x2 cells (4 slots), 12 blocks

and the workspace is always [B, 256, C] (16x16 cells). Every op body runs on
libsihc_hip.so (`launch`); none has a CPU or PyTorch compute fallback. Weight lists
are stacked into one [E, C, S] tensor per call (E*C*S elements, negligible next to
the carrier) because the C ABI takes one weight pointer.

Dtypes: outputs use the carrier / workspace dtype as in the reference. The split
reads take alpha in the carrier dtype (as model.py builds it); updates, betas and
gamma may be bf16 under an fp32 carrier / workspace, and where a kernel needs one
dtype they are widened to fp32, which is exact. Any other mix raises ValueError.
"""
from __future__ import annotations

from typing import Callable

import torch
from torch import Tensor
from torch.library import custom_op, register_autograd

from . import launch
from .sublayer_kernels import _read_backward, _read_setup, _require_packed

# tag -> (carrier edge, cell edge, blocks)
GEOMETRY = {"b4_12": (64, 4, 12), "b4_8": (64, 4, 8), "p8_12": (32, 2, 12)}
WORKSPACE_TOKENS = 256


def _upcast(t: Tensor, dtype: torch.dtype, what: str) -> Tensor:
    """t in `dtype`, allowing only the exact bf16 -> fp32 widening."""
    if t.dtype == dtype:
        return t
    if t.dtype == torch.bfloat16 and dtype == torch.float32:
        return t.float()
    raise ValueError(f"{what}: {t.dtype} cannot be used with a {dtype} carrier/workspace")


def _check_cuda(what: str, *tensors: Tensor) -> None:
    dev = tensors[0].device
    for t in tensors:
        if not t.is_cuda or t.device != dev:
            raise ValueError(f"{what}: tensors must share one CUDA device")
        if t.dtype not in (torch.float32, torch.bfloat16):
            raise ValueError(f"{what}: dtype must be float32 or bfloat16, got {t.dtype}")


def _schema(args: list[str], ret: str) -> str:
    return "(" + ", ".join(f"Tensor {a}" for a in args) + ") -> " + ret


# ----------------------------------------------------------------------------------
# all_base_*_split: the stage's E base reads (reference kernels.py:2219-2300, :2334-2432,
# :2434-2530)
# ----------------------------------------------------------------------------------
def _make_all_base(tag: str):
    edge, cell, blocks = GEOMETRY[tag]
    slots = cell * cell
    name = f"all_base_{tag}_split"

    def check(x0: Tensor, alpha: Tensor) -> None:
        if (x0.ndim != 4 or x0.shape[1] != edge or x0.shape[2] != edge
                or tuple(alpha.shape) != (blocks, x0.shape[3], slots)):
            raise ValueError(f"{name} expects x0 [B,{edge},{edge},C] and alpha [{blocks},C,{slots}], "
                             f"got {tuple(x0.shape)} and {tuple(alpha.shape)}")
        _require_packed(name, x0=x0, alpha_stack=alpha)
        _check_cuda(name, x0, alpha)
        if alpha.dtype != x0.dtype:
            raise ValueError(f"{name}: alpha must share the carrier dtype {x0.dtype}, got {alpha.dtype}")

    @custom_op(f"sihc::{name}_traceable", mutates_args=())
    def split(x0: Tensor, alpha_stack: Tensor) -> list[Tensor]:
        """Base reads z_e = sum_s alpha[e,:,s] * x0[cell slot s], one [B,256,C] per block."""
        check(x0, alpha_stack)
        return launch.read(x0, alpha_stack)

    @split.register_fake
    def _(x0, alpha_stack):
        return [x0.new_empty((x0.shape[0], WORKSPACE_TOKENS, x0.shape[3])) for _ in range(blocks)]

    @custom_op(f"sihc::all_base_{tag}_grad_x", mutates_args=())
    def grad_x(grad_base: Tensor, alpha_stack: Tensor) -> Tensor:
        """dx0[m,s,c] = sum_e alpha[e,c,s] * grad_base[e,m,c] for stacked [E,B,256,C] grads."""
        _require_packed(f"all_base_{tag}_grad_x", grad_base=grad_base, alpha_stack=alpha_stack)
        out = grad_base.new_empty((grad_base.shape[1], edge, edge, grad_base.shape[3]))
        return launch.write(out, list(grad_base.unbind(0)), _upcast(alpha_stack, grad_base.dtype, name),
                            add_x=False, out=out)

    @grad_x.register_fake
    def _(grad_base, alpha_stack):
        return grad_base.new_empty((grad_base.shape[1], edge, edge, grad_base.shape[3]))

    @custom_op(f"sihc::{name}_grad_alpha", mutates_args=())
    def grad_alpha(x0: Tensor, grad_base: Tensor) -> Tensor:
        """fp32 [E,C,S] = sum over tokens of x0[cell slot s] * grad_base[e] (atomics-free)."""
        _require_packed(f"{name}_grad_alpha", x0=x0, grad_base=grad_base)
        return launch.weight_grad(x0, list(_upcast(grad_base, x0.dtype, name).unbind(0)), None,
                                  out_dtype=torch.float32, slots=slots)

    @grad_alpha.register_fake
    def _(x0, grad_base):
        return x0.new_empty((grad_base.shape[0], x0.shape[3], slots), dtype=torch.float32)

    # Backward of the split read: identical math to sublayer_read's (a zero-carry write
    # of the output gradients and the weight reduction), on the per-output gradients
    # without stacking them first (reference :2285-2292 stacks, then runs the two
    # kernels above).
    register_autograd(split, _read_backward, setup_context=_read_setup)
    return split, grad_x, grad_alpha


all_base_b4_12_split_traceable, all_base_b4_12_grad_x_traceable, all_base_b4_12_split_grad_alpha_traceable = \
    _make_all_base("b4_12")
all_base_b4_8_split_traceable, all_base_b4_8_grad_x_traceable, all_base_b4_8_split_grad_alpha_traceable = \
    _make_all_base("b4_8")
all_base_p8_12_split_traceable, all_base_p8_12_grad_x_traceable, all_base_p8_12_split_grad_alpha_traceable = \
    _make_all_base("p8_12")


# ----------------------------------------------------------------------------------
# final_accumulate_*: x0 + sum_e beta_e * dz_e on the carrier (reference kernels.py:
# 1189-1389, :1390-1606, :1608-1766)
# ----------------------------------------------------------------------------------
def _make_final_accumulate(tag: str):
    edge, cell, blocks = GEOMETRY[tag]
    slots = cell * cell
    name = f"final_accumulate_{tag}"
    dz_names = [f"dz{i}" for i in range(blocks)]
    beta_names = [f"beta{i}" for i in range(blocks)]

    def check(x0: Tensor, dzs, betas) -> None:
        if x0.ndim != 4 or x0.shape[1] != edge or x0.shape[2] != edge:
            raise ValueError(f"{name} expects x0 [B,{edge},{edge},C], got {tuple(x0.shape)}")
        b, c = x0.shape[0], x0.shape[3]
        _require_packed(name, x0=x0, **dict(zip(dz_names, dzs)), **dict(zip(beta_names, betas)))
        for i, dz in enumerate(dzs):
            if tuple(dz.shape) != (b, WORKSPACE_TOKENS, c):
                raise ValueError(f"{name} dz{i} must be [{b},{WORKSPACE_TOKENS},{c}], got {tuple(dz.shape)}")
        for i, beta in enumerate(betas):
            if tuple(beta.shape) != (c, slots):
                raise ValueError(f"{name} beta{i} must be [{c},{slots}], got {tuple(beta.shape)}")
        w = {t.dtype for t in (*dzs, *betas)}
        if len(w) != 1 or not (w == {x0.dtype} or w == {torch.bfloat16}):
            raise ValueError(f"{name}: updates and betas must share one dtype, the carrier's or bfloat16")
        _check_cuda(name, x0, *dzs, *betas)

    def forward(x0: Tensor, *rest: Tensor) -> Tensor:
        dzs, betas = rest[:blocks], rest[blocks:]
        check(x0, dzs, betas)
        return launch.write(x0, list(dzs), torch.stack(betas), add_x=True)

    fa = custom_op(f"sihc::{name}_traceable", forward, mutates_args=(),
                   schema=_schema(["x0", *dz_names, *beta_names], "Tensor"))
    fa.register_fake(lambda x0, *rest: torch.empty_like(x0))

    def grad_dz_impl(grad_out: Tensor, *betas: Tensor) -> Tensor:
        """[E,B,256,C] in grad_out's dtype: dz_e gradient = read of grad_out with beta_e."""
        _require_packed(f"{name}_grad_dz_ptr", grad_out=grad_out)
        b, c = grad_out.shape[0], grad_out.shape[3]
        out = grad_out.new_empty((blocks, b, WORKSPACE_TOKENS, c))
        w = _upcast(torch.stack(betas), grad_out.dtype, name)
        launch.read(grad_out, w, out=out.unbind(0))
        return out

    grad_dz = custom_op(f"sihc::{name}_grad_dz_ptr", grad_dz_impl, mutates_args=(),
                        schema=_schema(["grad_out", *beta_names], "Tensor"))
    grad_dz.register_fake(
        lambda g, *betas: g.new_empty((blocks, g.shape[0], WORKSPACE_TOKENS, g.shape[3])))

    def grad_beta_impl(grad_out: Tensor, *dzs: Tensor) -> Tensor:
        """fp32 [E,C,S] = sum over tokens of grad_out[cell slot s] * dz_e (atomics-free)."""
        _require_packed(f"{name}_grad_beta_ptr", grad_out=grad_out)
        ups = [_upcast(d, grad_out.dtype, name) for d in dzs]
        return launch.weight_grad(grad_out, ups, None, out_dtype=torch.float32, slots=slots)

    grad_beta = custom_op(f"sihc::{name}_grad_beta_ptr", grad_beta_impl, mutates_args=(),
                          schema=_schema(["grad_out", *dz_names], "Tensor"))
    grad_beta.register_fake(
        lambda g, *dzs: g.new_empty((blocks, g.shape[3], slots), dtype=torch.float32))

    def setup(ctx, inputs, output):
        ctx.save_for_backward(*inputs[1:])

    def backward(ctx, grad_out):
        """Reference :1369-1381: identity to x0, a read of grad_out per update, the
        fp32 weight reduction cast to each beta's dtype."""
        saved = ctx.saved_tensors
        dzs, betas = saved[:blocks], saved[blocks:]
        grad_out = grad_out.contiguous()
        gdz = grad_dz(grad_out, *betas)
        gbeta = grad_beta(grad_out, *dzs)
        return (grad_out, *gdz.unbind(0), *(g.to(b.dtype) for g, b in zip(gbeta.unbind(0), betas)))

    register_autograd(fa, backward, setup_context=setup)
    return fa, grad_dz, grad_beta


final_accumulate_b4_12_traceable, final_accumulate_b4_12_grad_dz_ptr_traceable, \
    final_accumulate_b4_12_grad_beta_ptr_traceable = _make_final_accumulate("b4_12")
final_accumulate_b4_8_traceable, final_accumulate_b4_8_grad_dz_ptr_traceable, \
    final_accumulate_b4_8_grad_beta_ptr_traceable = _make_final_accumulate("b4_8")
final_accumulate_p8_12_traceable, final_accumulate_p8_12_grad_dz_ptr_traceable, \
    final_accumulate_p8_12_grad_beta_ptr_traceable = _make_final_accumulate("p8_12")


# ----------------------------------------------------------------------------------
# triangular accumulation with a constant active prefix, one op per prefix length
# (reference kernels.py:1768-1988 for 12-block stages, :1990-2192 for 8-block stages)
# ----------------------------------------------------------------------------------
def _make_triangular(stage: int, active: int) -> Callable:
    if not 1 <= active <= stage - 1:
        raise ValueError(f"active must be in [1, {stage - 1}], got {active}")
    name = f"triangular_accumulate_b4_{stage}_ptr_active{active}"
    label = f"triangular_accumulate_b4_{stage}_active"
    dz_names = [f"dz{i}" for i in range(stage)]

    def check(base: Tensor, dzs, gamma: Tensor) -> None:
        c = base.shape[-1]
        if base.ndim != 3 or base.shape[1] != WORKSPACE_TOKENS or tuple(gamma.shape) != (stage, c):
            raise ValueError(f"{label} expects base [B,256,C] and gamma [{stage},C], "
                             f"got {tuple(base.shape)} and {tuple(gamma.shape)}")
        for i, dz in enumerate(dzs):
            if dz.shape != base.shape:
                raise ValueError(f"{label} dz{i} shape {tuple(dz.shape)} does not match base {tuple(base.shape)}")
        _require_packed(label, base=base, gamma=gamma, **dict(zip(dz_names[:active], dzs[:active])))
        _check_cuda(label, base, gamma, *dzs[:active])

    def active_inputs(base: Tensor, dzs, gamma: Tensor):
        ups = [_upcast(d, base.dtype, label) for d in dzs[:active]]
        g = gamma[:active]
        if g.dtype not in (base.dtype, torch.float32):
            g = _upcast(g, torch.float32, label)
        return ups, g

    def forward(base: Tensor, *rest: Tensor) -> Tensor:
        """base + sum_{j < active} gamma[j] * dz_j (dz_j for j >= active are not read)."""
        dzs, gamma = rest[:stage], rest[stage]
        check(base, dzs, gamma)
        ups, g = active_inputs(base, dzs, gamma)
        return launch.triangular(base, ups, g)

    op = custom_op(f"sihc::{name}", forward, mutates_args=(),
                   schema=_schema(["base", *dz_names, "gamma"], "Tensor"))
    op.register_fake(lambda base, *rest: torch.empty_like(base))

    def fused_impl(grad_out: Tensor, *rest: Tensor):
        """(grad_dz [active,B,256,C] in grad_out's dtype, fp32 grad_gamma [stage,C] whose
        rows past the prefix are zero), from one pass over grad_out."""
        dzs, gamma = rest[:stage], rest[stage]
        _require_packed(f"{name}_grad_fused", grad_out=grad_out)
        ups, g = active_inputs(grad_out, dzs, gamma)
        ddz, dg = launch.triangular_backward(grad_out, ups, g, out_dtype=torch.float32)
        if active < stage:
            dg = torch.cat([dg, dg.new_zeros((stage - active, dg.shape[1]))])
        return ddz, dg

    fused = custom_op(f"sihc::{name}_grad_fused", fused_impl, mutates_args=(),
                      schema=_schema(["grad_out", *dz_names, "gamma"], "(Tensor, Tensor)"))
    fused.register_fake(lambda g, *rest: (g.new_empty((active, *g.shape)),
                                          g.new_empty((stage, g.shape[-1]), dtype=torch.float32)))

    def grad_dz_impl(grad_out: Tensor, gamma: Tensor) -> Tensor:
        """[active,B,256,C]: grad_out * gamma[j] (fp32 product stored in grad_out's dtype)."""
        _require_packed(f"{name}_grad_dz", grad_out=grad_out, gamma=gamma)
        g = gamma[:active]
        if g.dtype not in (grad_out.dtype, torch.float32):
            g = _upcast(g, torch.float32, label)
        ddz, _ = launch.triangular_backward(grad_out, [grad_out] * active, g, out_dtype=torch.float32)
        return ddz

    grad_dz = custom_op(f"sihc::{name}_grad_dz", grad_dz_impl, mutates_args=(),
                        schema=_schema(["grad_out", "gamma"], "Tensor"))
    grad_dz.register_fake(lambda g, gamma: g.new_empty((active, *g.shape)))

    def grad_gamma_impl(grad_out: Tensor, *rest: Tensor) -> Tensor:
        """fp32 [stage,C]: rows j < active = sum over rows of grad_out * dz_j, others zero."""
        dzs = rest[:stage]
        _require_packed(f"{name}_grad_gamma", grad_out=grad_out)
        ups = [_upcast(d, grad_out.dtype, label) for d in dzs[:active]]
        dg = launch.triangular_gamma_grad(grad_out, ups, None, out_dtype=torch.float32)
        if active < stage:
            dg = torch.cat([dg, dg.new_zeros((stage - active, dg.shape[1]))])
        return dg

    grad_gamma = custom_op(f"sihc::{name}_grad_gamma", grad_gamma_impl, mutates_args=(),
                           schema=_schema(["grad_out", *dz_names, "gamma"], "Tensor"))
    grad_gamma.register_fake(lambda g, *rest: g.new_empty((stage, g.shape[-1]), dtype=torch.float32))

    def setup(ctx, inputs, output):
        ctx.save_for_backward(*inputs[1:])

    def backward(ctx, grad_out):
        """Reference :1956-1968: identity to base, the fused kernel for the active
        updates and gamma, no gradient for the inactive updates."""
        saved = ctx.saved_tensors
        gamma = saved[stage]
        ddz, dg = fused(grad_out.contiguous(), *saved)
        return (grad_out, *ddz.unbind(0), *([None] * (stage - active)), dg.to(gamma.dtype))

    register_autograd(op, backward, setup_context=setup)
    return op


# One op per prefix length: compiled graphs see the prefix as a constant (reference
# kernels.py:1979-1985).
triangular_accumulate_b4_12_ptr_active_traceable_ops = tuple(_make_triangular(12, a) for a in range(1, 12))
triangular_accumulate_b4_8_ptr_active_traceable_ops = tuple(_make_triangular(8, a) for a in range(1, 8))


# ----------------------------------------------------------------------------------
# cell_mean_b4: parameter-free stage seed of write-only SiHC (reference kernels.py:
# 2532-2587): the mean of each 4x4 cell of a [B,64,64,C] carrier.
# ----------------------------------------------------------------------------------
def _sixteenth(c: int, like: Tensor) -> Tensor:
    # 1/16 is a power of two: the weighted read sums x_s / 16 exactly as the mean does.
    return torch.full((1, c, 16), 1.0 / 16.0, device=like.device, dtype=like.dtype)


@custom_op("sihc::cell_mean_b4_traceable", mutates_args=())
def cell_mean_b4_traceable(x: Tensor) -> Tensor:
    """[B,256,C] fp32-accumulated mean of each token's 16 carrier pixels."""
    if x.ndim != 4 or x.shape[1] != 64 or x.shape[2] != 64:
        raise ValueError(f"cell_mean_b4 expects x [B,64,64,C], got {tuple(x.shape)}")
    _require_packed("cell_mean_b4", x=x)
    _check_cuda("cell_mean_b4", x)
    return launch.read(x, _sixteenth(x.shape[3], x))[0]


@cell_mean_b4_traceable.register_fake
def _(x):
    return x.new_empty((x.shape[0], WORKSPACE_TOKENS, x.shape[3]))


@custom_op("sihc::cell_mean_b4_backward_traceable", mutates_args=())
def cell_mean_b4_backward_traceable(grad_out: Tensor) -> Tensor:
    """[B,64,64,C]: every pixel of a cell receives its token's gradient / 16."""
    _require_packed("cell_mean_b4_backward", grad_out=grad_out)
    out = grad_out.new_empty((grad_out.shape[0], 64, 64, grad_out.shape[2]))
    return launch.write(out, [grad_out], _sixteenth(grad_out.shape[2], grad_out), add_x=False, out=out)


@cell_mean_b4_backward_traceable.register_fake
def _(grad_out):
    return grad_out.new_empty((grad_out.shape[0], 64, 64, grad_out.shape[2]))


register_autograd(cell_mean_b4_traceable, lambda ctx, g: cell_mean_b4_backward_traceable(g.contiguous()))


__all__ = [
    "_require_packed",
    "all_base_b4_12_split_traceable", "all_base_b4_12_grad_x_traceable", "all_base_b4_12_split_grad_alpha_traceable",
    "all_base_b4_8_split_traceable", "all_base_b4_8_grad_x_traceable", "all_base_b4_8_split_grad_alpha_traceable",
    "all_base_p8_12_split_traceable", "all_base_p8_12_grad_x_traceable", "all_base_p8_12_split_grad_alpha_traceable",
    "final_accumulate_b4_12_traceable", "final_accumulate_b4_12_grad_dz_ptr_traceable",
    "final_accumulate_b4_12_grad_beta_ptr_traceable",
    "final_accumulate_b4_8_traceable", "final_accumulate_b4_8_grad_dz_ptr_traceable",
    "final_accumulate_b4_8_grad_beta_ptr_traceable",
    "final_accumulate_p8_12_traceable", "final_accumulate_p8_12_grad_dz_ptr_traceable",
    "final_accumulate_p8_12_grad_beta_ptr_traceable",
    "triangular_accumulate_b4_12_ptr_active_traceable_ops", "triangular_accumulate_b4_8_ptr_active_traceable_ops",
    "cell_mean_b4_traceable", "cell_mean_b4_backward_traceable",
]
