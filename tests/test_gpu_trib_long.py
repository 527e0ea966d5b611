"""GPU: the fused triangular backward with more than 64 rows per reduction chunk.

The reduction takes one chunk per 64 rows up to 1,024 chunks, so past 65,536 rows a
chunk covers more rows than one staged gradient sub-tile (64 rows) and the
wave-per-update kernel walks several sub-tiles per chunk, keeping its gamma-gradient
accumulators across them. These shapes reach that mode: 70,000 rows (69 per chunk, a
full sub-tile and a 5-row one) and 131,072 rows (128 per chunk, two full sub-tiles), at
the XL width (1,152 channels, nine 128-channel slices) and at a width whose last slice
is partial (136 channels), in bf16 and fp32, with 4 and 23 updates. The workspace is
filled with NaN first, so a partial row left unwritten shows up in the gamma gradient.

Bars: the update gradients g * gamma_j are one fp32 product rounded once, bit-exact
against the oracle; the fp32 gamma gradient (sums over all rows) meets the fp32 bar
against the oracle's float64 sums.
"""
from __future__ import annotations

import pytest
import torch

from helpers import announce, assert_parity
from oracle import sihc_oracle as O
from sihc_hip import _lib

pytestmark = pytest.mark.gpu
CASES = [  # (rows, channels, updates, dtype)
    (70_000, 1152, 4, torch.bfloat16),
    (70_000, 136, 23, torch.float32),
    (131_072, 136, 23, torch.bfloat16),
    (131_072, 1152, 4, torch.float32),
]


@pytest.mark.parametrize("rows,channels,active,dtype", CASES,
                         ids=[f"r{r}-c{c}-a{a}-{str(d)[6:]}" for r, c, a, d in CASES])
def test_multi_subtile_chunks_match_oracle(rows, channels, active, dtype):
    announce(f"triangular backward multi-sub-tile rows={rows} C={channels} A={active} {dtype}")
    torch.manual_seed(rows % 997 + channels + active)
    grad = torch.randn(rows, channels, device="cuda").to(dtype)
    ups = [torch.randn(rows, channels, device="cuda").to(dtype) for _ in range(active)]
    gamma = 0.05 * torch.randn(active, channels, device="cuda")
    ddz = [torch.empty(rows, channels, device="cuda", dtype=dtype) for _ in range(active)]
    dg = torch.empty(active, channels, device="cuda", dtype=torch.float32)
    L = _lib.lib()
    code = _lib.DTYPE_BF16 if dtype == torch.bfloat16 else _lib.DTYPE_F32
    nbytes = L.sihc_triangular_gamma_grad_workspace_size(active, rows, channels)
    ws = torch.full(((nbytes + 3) // 4 + 64,), float("nan"), device="cuda", dtype=torch.float32)
    _lib.check(L.sihc_triangular_backward(grad.data_ptr(), _lib.ptr_array(u.data_ptr() for u in ups),
                                          gamma.data_ptr(), _lib.ptr_array(d.data_ptr() for d in ddz),
                                          dg.data_ptr(), active, rows, channels, code, _lib.DTYPE_F32,
                                          _lib.DTYPE_F32, ws.data_ptr(), ws.numel() * 4,
                                          torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    # the oracle's torch ops run on the device here (float64 sums; same functions as on the CPU)
    rdz, rdg = O.triangular_backward(grad, ups, gamma)
    for j in range(active):
        assert torch.equal(ddz[j], rdz[j]), f"update gradient {j} not bit-exact"
    assert torch.isfinite(dg).all(), "a partial row was left unwritten"
    assert_parity(dg, rdg, torch.float32, what="dgamma")
