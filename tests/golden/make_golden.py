"""Write the committed known-answer fixtures (tests/golden/*.npz).

Inputs are drawn with numpy's seeded PCG64 generator; expected outputs come from the
float64 brute-force loops in oracle/sihc_oracle.py (`brute_*`), which index the
carrier through the reference's `_high_offsets` map and share no code with the
PyTorch restatement that the tests check against them.

Run from the repo root: python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import sihc_oracle as O  # noqa: E402

OUT = Path(__file__).resolve().parent

# (name, batch, grid, slots, channels, events, seed)
CASES = [
    ("p8_small", 2, 3, 4, 5, 3, 11),
    ("p4_small", 1, 2, 16, 3, 2, 12),
]


def make_case(name: str, batch: int, grid: int, slots: int, channels: int, events: int, seed: int) -> None:
    rng = np.random.default_rng(seed)
    k = O.cell_edge(slots)
    h = grid * k
    x = rng.standard_normal((batch, h, h, channels)).astype(np.float32)
    alpha = (0.25 + 0.02 * rng.standard_normal((events, channels, slots))).astype(np.float32)
    beta = (1.0 + 0.02 * rng.standard_normal((events, channels, slots))).astype(np.float32)
    updates = rng.standard_normal((events, batch, grid * grid, channels)).astype(np.float32)
    gamma = (0.1 * rng.standard_normal((events, channels))).astype(np.float32)
    index = np.stack([rng.permutation(grid * grid) for _ in range(batch)]).astype(np.int32)
    np.savez(
        OUT / f"{name}.npz",
        x=x, alpha=alpha, beta=beta, updates=updates, gamma=gamma, index=index,
        read=O.brute_read(x, alpha),
        write=O.brute_write(x, updates, beta, add_x=True),
        write_noadd=O.brute_write(x, updates, beta, add_x=False),
        weight_grad=O.brute_weight_grad(x, updates, slots),
        triangular=O.brute_triangular(updates[0], updates[1:], gamma[1:]),
        gather=O.brute_gather(x, index, slots),
    )
    print(f"wrote {name}.npz")


if __name__ == "__main__":
    for case in CASES:
        make_case(*case)
