"""GPU: the fused triangular backward when the reduction's last chunk holds no token.

Token chunks are ceil(rows / chunks) long, so for some row counts the last chunks would
start past the last row (1,250 rows in 39 chunks of 33: 38 x 33 >= 1,250). The host
launches and finalizes only the chunks that hold rows, so no partial row is summed that
no block wrote. The workspace is filled with NaN before the call, so a row left unwritten
(or summed without being written) shows up in the gamma gradient. Shapes take the
wave-per-update kernel with one sub-tile per chunk (3+ updates, 16-byte bf16 vectors, at
most 64 rows per chunk).
"""
from __future__ import annotations

import pytest
import torch

from helpers import announce, assert_parity
from oracle import sihc_oracle as O
from sihc_hip import _lib

pytestmark = pytest.mark.gpu
CASES = [(1250, 8, 4), (1250, 64, 11), (1352, 128, 23)]  # (rows, channels, updates)


@pytest.mark.parametrize("rows,channels,active", CASES, ids=[f"r{r}-c{c}-a{a}" for r, c, a in CASES])
def test_empty_last_chunk_writes_zero_partials(rows, channels, active):
    announce(f"triangular backward empty last chunk rows={rows} C={channels} A={active}")
    torch.manual_seed(rows + channels + active)
    bf = torch.bfloat16
    grad = torch.randn(rows, channels, device="cuda").to(bf)
    ups = [torch.randn(rows, channels, device="cuda").to(bf) for _ in range(active)]
    gamma = torch.randn(active, channels, device="cuda")
    ddz = [torch.empty(rows, channels, device="cuda", dtype=bf) for _ in range(active)]
    dg = torch.empty(active, channels, device="cuda", dtype=torch.float32)
    L = _lib.lib()
    nbytes = L.sihc_triangular_gamma_grad_workspace_size(active, rows, channels)
    ws = torch.full(((nbytes + 3) // 4 + 64,), float("nan"), device="cuda", dtype=torch.float32)
    _lib.check(L.sihc_triangular_backward(grad.data_ptr(), _lib.ptr_array(u.data_ptr() for u in ups),
                                          gamma.data_ptr(), _lib.ptr_array(d.data_ptr() for d in ddz),
                                          dg.data_ptr(), active, rows, channels, _lib.DTYPE_BF16, _lib.DTYPE_F32,
                                          _lib.DTYPE_F32, ws.data_ptr(), ws.numel() * 4,
                                          torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    rdz, rdg = O.triangular_backward(grad.cpu(), [u.cpu() for u in ups], gamma.cpu())
    for j in range(active):
        assert torch.equal(ddz[j].cpu(), rdz[j]), f"update gradient {j} not bit-exact"
    assert torch.isfinite(dg).all(), "a partial row was left unwritten"
    # fp32 gamma gradient: the fp32 bar against the oracle's float64 sums
    assert_parity(dg, rdg, torch.float32, what="dgamma")
