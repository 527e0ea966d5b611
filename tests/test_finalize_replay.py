"""CPU: bounds-checked replay of the fixed-order finalize's index arithmetic.

The finalize sums fp32 partial rows part[chunks][R][S][C] into R output rows of [C][S]
(`finalize_outputs` in residual-stream-burden_amd/csrc/sihc_kernels.hip), from three
launch sites: `k_finalize` (weight and gamma gradients; 4 outputs per thread when S*C is
a multiple of 4 and the partial rows are 16-byte aligned, else 1), `k_finalize_batch`
(deferred per-event finalizes, grid.y = event, always 4 per thread) and the trailing
blocks of a chained per-event backward (`run_carry`: blocks nmain, nmain + 1, ... of the
backward's grid). This module restates those index expressions in numpy, for every
thread of every block of a launch, and checks, without a GPU:

* every partial-row load (all NV lanes of a 16-byte load) lies inside part[0, chunks*n);
* the NV outputs of a live thread lie in one row (NV > 1 needs S*C % NV == 0) and every
  store lands inside its destination row [C][S];
* every output is stored exactly once, and the LDS slots stay inside FG x FO x NV;
* the host's choice of NV and block count (launch_finalize, sihc_event_finalize, the
  chained backward's carry_blocks) covers every output.

Shapes: channel counts whose S*C is and is not a multiple of 4 (C = 67, 130, 1152),
S = 1 (gamma gradient), 4 and 16, row counts 1, 2, 3, 24, chunk counts below, at and
above 8 x FG, and events without partial rows (skipped by the batch finalize). A mistake
planted in the replay (a 4-wide load with S*C not a multiple of 4) must be caught.
"""
from __future__ import annotations

import numpy as np
import pytest

FO, FG = 32, 8  # FINALIZE_FO, FINALIZE_FG: output lanes and chunk groups of a 256-thread block


def replay_block_set(n: int, SC: int, S: int, C: int, R: int, pair: bool, chunks: int, nv: int,
                     blocks: np.ndarray, written: np.ndarray) -> None:
    """Replay finalize_outputs<TO, nv> for the given (relative) block indices."""
    tid = np.arange(256)
    o, grp = tid % FO, tid // FO
    b = blocks[:, None]
    i = (b * FO + o[None, :]) * nv                      # this thread's first output (int64)
    live = i < n
    # LDS slots red[grp][o*nv + j]
    lds = grp[None, :, None] * (FO * nv) + o[None, :, None] * nv + np.arange(nv)[None, None, :]
    assert lds.min() >= 0 and lds.max() < FG * FO * nv
    if not live.any():
        return
    il = i[live]
    r = il // SC                                       # the row of the first output
    # all nv outputs of a live thread are in range and in the same row
    last = il + nv - 1
    assert (last < n).all(), "a 4-wide load reads past the partial row"
    assert (last // SC == r).all(), "a thread's outputs straddle two rows"
    # loads: chunk k = grp, grp + FG, ... < chunks; element k*n + i + j
    g_live = np.broadcast_to(grp[None, :], i.shape)[live]
    if chunks > 0:
        kmax = g_live + ((chunks - 1 - g_live) // FG) * FG   # last chunk this thread reads
        has = g_live < chunks
        lo = (g_live[has] * n + il[has])
        hi = (kmax[has] * n + il[has] + nv - 1)
        assert lo.min() >= 0 and hi.max() < chunks * n, "partial-row load out of range"
    # stores: group 0 only
    sel = g_live == 0
    for j in range(nv):
        rem = il[sel] + j - r[sel] * SC
        s = rem // C
        c = rem - s * C
        off = c * S + s
        assert (off >= 0).all() and (off < C * S).all(), "store outside its row"
        rows = r[sel]
        if pair:
            assert (rows <= 1).all()
        np.add.at(written, (rows, off), 1)


def host_nv(S: int, C: int, part_aligned16: bool = True) -> int:
    """launch_finalize: 4 outputs per thread when they never straddle a row and the rows
    are 16-byte aligned."""
    return 4 if (S * C) % 4 == 0 and part_aligned16 else 1


def run_finalize(R: int, S: int, C: int, chunks: int, nv: int, pair: bool = False) -> np.ndarray:
    n, SC = R * S * C, S * C
    blocks = (n + FO * nv - 1) // (FO * nv)
    written = np.zeros((R, C * S), np.int64)
    replay_block_set(n, SC, S, C, R, pair, chunks, nv, np.arange(blocks), written)
    return written


CHUNKS = [1, 7, 8 * FG - 1, 8 * FG, 8 * FG + 1, 512, 1024]


@pytest.mark.parametrize("S", [1, 4, 16])
@pytest.mark.parametrize("C", [67, 130, 1152])
@pytest.mark.parametrize("R", [1, 2, 3, 24])
def test_k_finalize_indexing(S, C, R):
    nv = host_nv(S, C)
    for chunks in CHUNKS:
        w = run_finalize(R, S, C, chunks, nv)
        assert (w == 1).all(), f"outputs not written exactly once (R={R} S={S} C={C} chunks={chunks} nv={nv})"
    if nv == 4:  # the 1-wide form covers the same shapes
        assert (run_finalize(R, S, C, 64, 1) == 1).all()


@pytest.mark.parametrize("S", [4, 16])
@pytest.mark.parametrize("C", [67, 130, 1152])
def test_batch_and_chained_finalize_indexing(S, C):
    # sihc_event_finalize: grid (ceil(2*S*C / 128), events) with 4 outputs per thread; an
    # event whose info lists no partial rows is left out of the batch. The chained
    # backward's trailing blocks use the same count (EV_CARRY_OUTPUTS_PER_BLOCK = 128).
    n = 2 * S * C
    bx = (n + 127) // 128
    for chunks in [0] + CHUNKS:
        written = np.zeros((2, C * S), np.int64)
        if chunks > 0:
            replay_block_set(n, S * C, S, C, 2, True, chunks, 4, np.arange(bx), written)
            assert (written == 1).all()
        # the trailing blocks of a chained launch: block indices nmain .. nmain + bx - 1,
        # each finalizing block (blockIdx.x - nmain)
        nmain = 9 * 1024
        rel = np.arange(nmain, nmain + bx) - nmain
        written2 = np.zeros((2, C * S), np.int64)
        if chunks > 0:
            replay_block_set(n, S * C, S, C, 2, True, chunks, 4, rel, written2)
            assert (written2 == written).all()


def test_planted_wide_load_on_unaligned_rows_is_caught():
    # gamma gradient rows of 67 channels (S = 1): a 4-wide finalize would straddle rows
    with pytest.raises(AssertionError, match="straddle|past the partial row"):
        run_finalize(3, 1, 67, 16, 4)


def logical_block_of(b: np.ndarray, n: int) -> np.ndarray:
    """logical_block_of<true>(n): XCD-contiguous order over the first n blocks."""
    q, r = n >> 3, n & 7
    x, i = b & 7, b >> 3
    return np.where(x < r, x * (q + 1) + i, r * (q + 1) + (x - r) * q + i)


@pytest.mark.parametrize("nmain", [1, 7, 8, 9, 4607, 4608, 9216, 9217])
def test_main_blocks_of_a_chained_launch_map_onto_themselves(nmain):
    # the backward proper of a chained launch (16-slot cells use the XCD order) is the
    # first nmain blocks of a larger grid: its logical block order must be a permutation
    # of 0..nmain-1 whatever the trailing blocks
    lb = logical_block_of(np.arange(nmain), nmain)
    assert np.array_equal(np.sort(lb), np.arange(nmain))
