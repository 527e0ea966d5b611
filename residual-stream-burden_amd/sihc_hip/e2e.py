"""Compact SiHC sublayer denoiser whose routing runs on the HIP ops (benchmark config 4).

Architecture (behaviour of tongtongliang/residual-stream-burden
sihc/models/sihc/sublayer.py:30-128, model.py:186-682 and components.py:14-324):
a patch stem maps a 256x256x3 image to the NHWC carrier [B, 256/p, 256/p, D]; each of
`depth` blocks has an AdaLN-modulated attention update and a SwiGLU MLP update
computed on the 16x16 workspace, each with its own static connection (read/write
weights [D, S]); stages of 8 or 12 blocks are routed either with the reference's
late-materialised schedule (read -> triangular -> write, `schedule="stage"`) or with
the per-event fused schedule (`schedule="literal"`); a modulated final layer maps the
carrier back to image space. With `in_context_len > 0` (the in-context variant,
model.py:565-682, sublayer.py:75-128) class-embedding prefix tokens join the workspace
sequence from block `in_context_start` on: attention and MLP run on
[prefix, workspace], the prefix takes ordinary residual updates and never enters the
routing, and its RoPE positions are unrotated (components.py:44-70).

The bodies are plain PyTorch (they are not part of the read/write path). Routing
calls go through replaceable hooks (`read`, `triangular`, `write`, and `event` for the
per-event write+read), so tests and benchmarks can swap in other implementations of
the same functions, and an optional list of HIP event pairs records the time spent in
routing.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from .event_ops import event_write_read
from .sublayer_kernels import sublayer_read, sublayer_triangular, sublayer_write


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x):
        xf = x.float()
        return (xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + self.eps) * self.weight.float()).to(x.dtype)


def rope_tables(head_dim: int, grid: int, theta: float = 10000.0):
    """2-D rotary tables over the workspace grid: half of each head rotates with the
    row index, half with the column index (pairs of adjacent channels)."""
    quarter = head_dim // 4
    inv = 1.0 / theta ** (torch.arange(quarter, dtype=torch.float64) * 2 / (head_dim // 2))
    pos = torch.arange(grid, dtype=torch.float64)
    ang = torch.outer(pos, inv).repeat_interleave(2, dim=-1)              # [grid, head_dim/2]
    rows = ang[:, None, :].expand(grid, grid, -1)
    cols = ang[None, :, :].expand(grid, grid, -1)
    full = torch.cat([rows, cols], dim=-1).reshape(grid * grid, head_dim)
    return full.cos().float(), full.sin().float()


def apply_rope(x, cos, sin):
    pairs = x.reshape(*x.shape[:-1], -1, 2)
    rotated = torch.stack((-pairs[..., 1], pairs[..., 0]), dim=-1).reshape_as(x)
    return x * cos + rotated * sin


class Attention(nn.Module):
    def __init__(self, dim: int, heads: int):
        super().__init__()
        self.heads, self.head_dim = heads, dim // heads
        self.qkv = nn.Linear(dim, 3 * dim)
        self.q_norm, self.k_norm = RMSNorm(self.head_dim), RMSNorm(self.head_dim)
        self.proj = nn.Linear(dim, dim)

    def forward(self, x, cos, sin):
        b, n, c = x.shape
        q, k, v = self.qkv(x).reshape(b, n, 3, self.heads, self.head_dim).permute(2, 0, 3, 1, 4).unbind(0)
        q = apply_rope(self.q_norm(q), cos, sin)
        k = apply_rope(self.k_norm(k), cos, sin)
        if q.dtype == torch.bfloat16:
            # fused attention kernels only: the math fallback would run batched bf16
            # products on transposed views
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                out = F.scaled_dot_product_attention(q, k, v)
        else:
            out = F.scaled_dot_product_attention(q, k, v)
        return self.proj(out.transpose(1, 2).reshape(b, n, c))


class SwiGLU(nn.Module):
    def __init__(self, dim: int, hidden: int):
        super().__init__()
        hidden = int(hidden * 2 / 3)
        self.w12 = nn.Linear(dim, 2 * hidden)
        self.w3 = nn.Linear(hidden, dim)

    def forward(self, x):
        a, b = self.w12(x).chunk(2, dim=-1)
        return self.w3(F.silu(a) * b)


def _modulate(x, shift, scale):
    return x * (1 + scale.unsqueeze(1)) + shift.unsqueeze(1)


class Connection(nn.Module):
    """Static per-feature read/write maps of one connection event ([D, S] each)."""

    def __init__(self, dim: int, slots: int):
        super().__init__()
        self.read_weight = nn.Parameter(torch.full((dim, slots), 1.0 / slots))
        self.write_weight = nn.Parameter(torch.ones(dim, slots))


class Block(nn.Module):
    def __init__(self, dim: int, heads: int, mlp_ratio: float, slots: int):
        super().__init__()
        self.norm1, self.norm2 = RMSNorm(dim), RMSNorm(dim)
        self.attn = Attention(dim, heads)
        self.mlp = SwiGLU(dim, int(dim * mlp_ratio))
        self.ada = nn.Sequential(nn.SiLU(), nn.Linear(dim, 6 * dim))
        self.attention_connection = Connection(dim, slots)
        self.mlp_connection = Connection(dim, slots)

    def attention_update(self, z, mod, cos, sin):
        shift, scale, gate = mod[0], mod[1], mod[2]
        return gate.unsqueeze(1) * self.attn(_modulate(self.norm1(z), shift, scale), cos, sin)

    def mlp_update(self, z, mod):
        shift, scale, gate = mod[3], mod[4], mod[5]
        return gate.unsqueeze(1) * self.mlp(_modulate(self.norm2(z), shift, scale))


class SiHCDenoiser(nn.Module):
    def __init__(self, hidden: int = 1152, depth: int = 28, heads: int = 16, patch: int = 8,
                 stages: tuple[int, ...] = (8, 12, 8), mlp_ratio: float = 4.0, num_classes: int = 1000,
                 image: int = 256, grid: int = 16, schedule: str = "stage", in_context_len: int = 0,
                 in_context_start: int = 4):
        super().__init__()
        if sum(stages) != depth or any(s not in (8, 12) for s in stages):
            raise ValueError("stages must be 8 or 12 blocks each and sum to depth")
        if schedule not in ("stage", "literal"):
            raise ValueError("schedule must be 'stage' or 'literal'")
        if in_context_len < 0:
            raise ValueError(f"in_context_len must be >= 0, got {in_context_len}")
        if in_context_len and not 0 <= in_context_start < depth:
            raise ValueError(f"in_context_start must be in [0, {depth}), got {in_context_start}")
        self.hidden, self.patch, self.image, self.grid = hidden, patch, image, grid
        self.cell = image // patch // grid
        self.slots = self.cell * self.cell
        self.stages, self.schedule = tuple(stages), schedule
        self.freq_dim = 256
        self.t_mlp = nn.Sequential(nn.Linear(self.freq_dim, hidden), nn.SiLU(), nn.Linear(hidden, hidden))
        self.y_table = nn.Embedding(num_classes + 1, hidden)
        self.stem = nn.Linear(3 * patch * patch, hidden)
        self.blocks = nn.ModuleList(Block(hidden, heads, mlp_ratio, self.slots) for _ in range(depth))
        self.final_norm = RMSNorm(hidden)
        self.final_ada = nn.Sequential(nn.SiLU(), nn.Linear(hidden, 2 * hidden))
        self.final = nn.Linear(hidden, patch * patch * 3)
        cos, sin = rope_tables(hidden // heads, grid)
        self.register_buffer("rope_cos", cos, persistent=False)
        self.register_buffer("rope_sin", sin, persistent=False)
        self.in_context_len, self.in_context_start = int(in_context_len), int(in_context_start)
        if self.in_context_len:
            self.in_context_posemb = nn.Parameter(torch.zeros(1, self.in_context_len, hidden))
            # prefix positions are not rotated
            pre = self.in_context_len
            self.register_buffer("rope_cos_ctx", torch.cat([torch.ones(pre, cos.shape[1]), cos]), persistent=False)
            self.register_buffer("rope_sin_ctx", torch.cat([torch.zeros(pre, sin.shape[1]), sin]), persistent=False)
        # routing hooks (None: the HIP ops) and optional timing of routing calls
        self.read = self.triangular = self.write = self.event = None
        self.routing_timer: Optional[list] = None

    def random_init(self, std: float = 0.02, seed: int = 0) -> "SiHCDenoiser":
        """Random weights everywhere (nonzero gates, perturbed connections)."""
        g = torch.Generator(device="cpu").manual_seed(seed)
        with torch.no_grad():
            for name, p in self.named_parameters():
                noise = torch.randn(p.shape, generator=g) * std
                if name.endswith("read_weight") or name.endswith("write_weight") or "norm" in name:
                    p.add_(noise.to(p.device, p.dtype))
                else:
                    p.copy_(noise.to(p.device, p.dtype))
        return self

    # ---- routing with optional HIP-event timing
    def _timed(self, fn, *args):
        if self.routing_timer is None:
            return fn(*args)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        out = fn(*args)
        end.record()
        self.routing_timer.append((start, end))
        return out

    def _update(self, block, part, z, mod, context, index):
        """One sublayer's workspace update (and the prefix tokens' new state): the body
        runs on [prefix, workspace] from block `in_context_start` on (sublayer.py:97-114)."""
        use_context = context is not None and index >= self.in_context_start
        if use_context:
            seq = torch.cat((context, z), dim=1)
            cos, sin = self.rope_cos_ctx.to(z.dtype), self.rope_sin_ctx.to(z.dtype)
        else:
            seq = z
            cos, sin = self.rope_cos.to(z.dtype), self.rope_sin.to(z.dtype)
        dseq = block.attention_update(seq, mod, cos, sin) if part == 0 else block.mlp_update(seq, mod)
        if not use_context:
            return dseq.contiguous(), context
        pre = self.in_context_len
        # removing the prefix leaves a batch-strided view: the routing ops need it packed
        return dseq[:, pre:].contiguous(), context + dseq[:, :pre]

    def _stage_schedule(self, x0, cond, blocks, first, context):
        conns = [c for b in blocks for c in (b.attention_connection, b.mlp_connection)]
        alpha = torch.stack([c.read_weight.to(x0.dtype) for c in conns]).contiguous()
        beta = torch.stack([c.write_weight.to(x0.dtype) for c in conns]).contiguous()
        read = self.read or sublayer_read
        tri = self.triangular or sublayer_triangular
        write = self.write or sublayer_write
        base = self._timed(read, x0, alpha)
        gamma = (alpha[:, None] * beta[None, :]).sum(-1)
        updates = []
        for i, block in enumerate(blocks):
            mod = block.ada(cond).chunk(6, dim=-1)
            for part in range(2):
                e = 2 * i + part
                z = base[e]
                if updates:
                    z = self._timed(tri, z, updates, gamma[e, :e].contiguous())
                dz, context = self._update(block, part, z, mod, context, first + i)
                updates.append(dz)
        return self._timed(write, x0, updates, beta), context

    def _literal_schedule(self, x0, cond, blocks, first, context):
        conns = [c for b in blocks for c in (b.attention_connection, b.mlp_connection)]
        alpha = [c.read_weight.to(x0.dtype).contiguous() for c in conns]
        beta = [c.write_weight.to(x0.dtype).contiguous() for c in conns]
        z = self._timed(self.read or sublayer_read, x0, alpha[0][None])[0]
        x = x0
        e = 0
        for i, block in enumerate(blocks):
            mod = block.ada(cond).chunk(6, dim=-1)
            for part in range(2):
                dz, context = self._update(block, part, z, mod, context, first + i)
                if e + 1 < len(conns):
                    x, z = self._timed(self.event or event_write_read, x, dz, beta[e], alpha[e + 1])
                else:
                    x = self._timed(self.write or sublayer_write, x, [dz], beta[e][None])
                e += 1
        return x, context

    def forward(self, x, t, y):
        b = x.shape[0]
        p, hi = self.patch, self.image // self.patch
        half = self.freq_dim // 2
        freqs = torch.exp(-math.log(10000.0) * torch.arange(half, device=t.device, dtype=torch.float32) / half)
        args = t.float()[:, None] * freqs[None]
        temb = torch.cat([args.cos(), args.sin()], dim=-1).to(self.stem.weight.dtype)
        y_emb = self.y_table(y)
        cond = self.t_mlp(temb) + y_emb
        patches = x.reshape(b, 3, hi, p, hi, p).permute(0, 2, 4, 1, 3, 5).reshape(b, hi, hi, 3 * p * p)
        carrier = self.stem(patches.to(self.stem.weight.dtype)).contiguous()
        context = None
        if self.in_context_len:  # model.py:674-676
            context = (y_emb[:, None].expand(-1, self.in_context_len, -1) + self.in_context_posemb).to(carrier.dtype)
        run = self._stage_schedule if self.schedule == "stage" else self._literal_schedule
        start = 0
        for size in self.stages:
            carrier, context = run(carrier, cond, list(self.blocks[start:start + size]), start, context)
            start += size
        shift, scale = self.final_ada(cond).chunk(2, dim=-1)
        out = self.final(_modulate(self.final_norm(carrier.reshape(b, hi * hi, self.hidden)), shift, scale))
        return out.reshape(b, hi, hi, 3, p, p).permute(0, 3, 1, 4, 2, 5).reshape(b, 3, hi * p, hi * p)


__all__ = ["SiHCDenoiser"]
