"""The allocation-free per-event backward (sihc_event_backward_noalloc) against
sihc_event_backward with a caller workspace, called through the C ABI.

Both entry points run the same kernels with the same reduction order, so every output
must match bit for bit. Two calls in a row on the same GPU (the second with a smaller
input) check that the shared scratch array carries nothing from one call to the next.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from helpers import announce
from sihc_hip import _lib

BF16 = torch.bfloat16


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _inputs(batch, channels, slots, seed, dtype=BF16):
    k = 2 if slots == 4 else 4
    g = torch.Generator(device="cuda").manual_seed(seed)
    r = lambda *shape, m=0.0, sd=1.0: (m + sd * torch.randn(*shape, device="cuda", generator=g)).to(dtype)  # noqa: E731
    carrier = (batch, 16 * k, 16 * k, channels)
    ws = (batch, 256, channels)
    return dict(h=r(*carrier, sd=1e-2), gz=r(*ws, sd=1e-2), xo=r(*carrier), dz=r(*ws),
                beta=r(channels, slots, m=1.0, sd=0.02), alpha=r(channels, slots, m=1.0 / slots, sd=0.02))


def _outputs(inp):
    e = lambda t: torch.full_like(t, float("nan"))  # noqa: E731  (poisoned: every element must be written)
    return dict(gx=e(inp["h"]), gdz=e(inp["dz"]), gb=e(inp["beta"]), ga=e(inp["alpha"]))


def _call(noalloc, inp, out, slots, dtype_code, stream):
    L = _lib.lib()
    b, hh, _, c = inp["h"].shape
    k = 2 if slots == 4 else 4
    args = (_p(inp["h"]), _p(inp["gz"]), _p(inp["xo"]), _p(inp["dz"]), _p(inp["beta"]), _p(inp["alpha"]),
            _p(out["gx"]), _p(out["gdz"]), _p(out["gb"]), _p(out["ga"]), b, hh // k, k, c, None,
            dtype_code, dtype_code)
    if noalloc:
        return L.sihc_event_backward_noalloc(*args, stream)
    nbytes = L.sihc_event_backward_workspace_size(b, hh // k, k, c)
    ws = torch.empty((nbytes + 15) // 16 * 4, device="cuda", dtype=torch.float32)
    rc = L.sihc_event_backward(*args, _p(ws), ws.numel() * 4, stream)
    return rc


CASES = [  # (batch, channels, slots, dtype): the second call of each pair is smaller
    ((8, 1152, 4, BF16), (2, 192, 4, BF16)),
    ((4, 256, 16, BF16), (1, 64, 16, BF16)),
    ((3, 96, 4, torch.float32), (1, 40, 4, torch.float32)),
]


@pytest.mark.gpu
@pytest.mark.parametrize("pair", CASES, ids=lambda p: f"{p[0][0]}x{p[0][1]}s{p[0][2]}-then-{p[1][0]}x{p[1][1]}")
def test_noalloc_matches_workspace_entry_point_twice(pair):
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for call, (batch, channels, slots, dtype) in enumerate(pair):
        announce(f"noalloc event backward call {call}: batch={batch} C={channels} slots={slots} {dtype}")
        code = _lib.DTYPE_F32 if dtype == torch.float32 else _lib.DTYPE_BF16
        inp = _inputs(batch, channels, slots, seed=100 + call, dtype=dtype)
        ref, got = _outputs(inp), _outputs(inp)
        _lib.check(_call(False, inp, ref, slots, code, stream))
        _lib.check(_call(True, inp, got, slots, code, stream))
        torch.cuda.synchronize()
        for name in ref:
            assert not torch.isnan(ref[name]).any(), f"{name}: reference output not fully written"
            assert torch.equal(got[name], ref[name]), f"call {call}: {name} differs from sihc_event_backward"


def test_noalloc_rejects_sizes_beyond_its_scratch():
    # 16 slots, 65,536 tokens, 4096 channels: 256 chunks of 256 tokens x 2 x 16 x 4096 x 4 B
    # = 128 MiB of partial rows, more than the 64 MiB array; rejected from the sizes alone,
    # before any HIP call (so this runs without a GPU)
    L = _lib.lib()
    fake = 0x1000
    need = L.sihc_event_backward_workspace_size(256, 16, 4, 4096)
    assert need == 256 * 2 * 16 * 4096 * 4 > 64 << 20
    rc = L.sihc_event_backward_noalloc(*([fake] * 10), 256, 16, 4, 4096, None, 1, 1, None)
    assert rc == 1 and b"scratch" in L.sihc_last_error() and b"67108864" in L.sihc_last_error()
    # at the benchmark shape (4 slots, 1152 channels) the partial rows fit
    assert L.sihc_event_backward_workspace_size(256, 16, 2, 1152) <= 64 << 20
