"""Parity helpers shared by the GPU tests."""
from __future__ import annotations

import os
import sys

import torch

# Slack of the elementwise bf16 bar for results near zero: two fp32 sums of the same
# terms taken in different orders differ by a few fp32 ulps of the terms, which is more
# than one bf16 ulp of a result that cancelled to almost nothing. 2**-16 of the largest
# expected magnitude is 1/256 of the bf16 ulp at that magnitude, so it only matters for
# such near-zero results.
NEAR_ZERO_SLACK = 2.0 ** -16

# (test, what, dtype, kind, max-abs, scale, max ulps, rel-L2) of every check this session,
# summarised at the end of the run (tests/conftest.py) so the margins show in the log.
RECORDS: list[tuple] = []


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.detach().double(), b.detach().double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bfloat16 values at |x| (float64): 2**(floor(log2|x|) - 7) for normal
    magnitudes, the subnormal spacing 2**-133 below 2**-126."""
    _, e = torch.frexp(x.double().abs())  # |x| = m * 2**e, 0.5 <= m < 1
    ulp = torch.ldexp(torch.ones_like(x, dtype=torch.float64), (e - 8).to(torch.int32))
    return torch.where(x.double().abs() < 2.0 ** -126, torch.full_like(ulp, 2.0 ** -133), ulp)


def assert_parity(actual: torch.Tensor, expected: torch.Tensor, dtype: torch.dtype, *, what: str = "",
                  kind: str = "elementwise") -> None:
    """The tier's parity bar. Prints the errors achieved, so margins show in the log.

    fp32 (every kind): max-abs error <= 1e-5 * max|expected| and relative L2 <= 1e-5.
    bf16, kind="elementwise" (an op's own outputs from the same inputs as the oracle's:
          both sides sum exact bf16 x bf16 products in fp32 and round once, so they can
          only land on neighbouring bf16 values): every element within 1 bf16 ulp of the
          oracle value (ulp taken at the larger magnitude of the two), plus
          NEAR_ZERO_SLACK * max|expected| for results that cancelled to almost nothing;
          and relative L2 <= 1e-2.
    bf16, kind="reduced" (sums over all tokens, e.g. weight gradients over 65,536
          tokens: the kernel's fp32 partial sums and the float64 oracle differ by the
          fp32 accumulation error of that many terms, which grows with the token count)
          and kind="chained" (results that pass through several rounding sites, each of
          which may land one ulp apart, e.g. a whole stage or model): max-abs error <=
          2e-2 * max(1, max|expected|) and relative L2 <= 1e-2.
    """
    if kind not in ("elementwise", "reduced", "chained"):
        raise ValueError(f"unknown parity kind {kind!r}")
    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    assert torch.isfinite(a).all() == torch.isfinite(e).all(), f"{what}: finiteness differs"
    scale = float(e.abs().max()) if e.numel() else 0.0
    diff = (a - e).abs()
    err = float(diff.max()) if e.numel() else 0.0
    r = rel_l2(a, e) if e.numel() and float(e.norm()) > 0 else err
    test = os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0]
    if dtype == torch.float32:
        RECORDS.append((test, what, "fp32", "fp32", err, scale, float("nan"), r))
        print(f"[parity] {what}: fp32 max-abs {err:.3e} (scale {scale:.3e}) rel-L2 {r:.3e}", flush=True)
        assert err <= 1e-5 * max(scale, 1e-30), f"{what}: fp32 max-abs {err:.3e} > 1e-5 * {scale:.3e}"
        assert r <= 1e-5, f"{what}: fp32 rel-L2 {r:.3e} > 1e-5"
        return
    ulps = diff / bf16_ulp(torch.maximum(a.abs(), e.abs())) if e.numel() else diff
    max_ulps = float(ulps.max()) if e.numel() else 0.0
    RECORDS.append((test, what, "bf16", kind, err, scale, max_ulps, r))
    print(f"[parity] {what}: bf16 {kind} max-abs {err:.3e} (scale {scale:.3e}) max {max_ulps:.2f} ulp "
          f"rel-L2 {r:.3e}", flush=True)
    assert r <= 1e-2, f"{what}: bf16 rel-L2 {r:.3e} > 1e-2"
    if kind == "elementwise":
        bound = bf16_ulp(torch.maximum(a.abs(), e.abs())) + NEAR_ZERO_SLACK * scale
        bad = diff > bound
        if bad.any():
            i = int(torch.nonzero(bad.flatten())[0])
            raise AssertionError(
                f"{what}: {int(bad.sum())} of {bad.numel()} bf16 elements beyond 1 ulp; first at flat index {i}: "
                f"got {float(a.flatten()[i])!r}, expected {float(e.flatten()[i])!r}")
    else:
        assert err <= 2e-2 * max(1.0, scale), f"{what}: bf16 max-abs {err:.3e} > 2e-2 * max(1, {scale:.3e})"


def assert_close_reference(actual: torch.Tensor, expected: torch.Tensor, *, atol: float, rtol: float,
                           what: str = "") -> None:
    """The reference's own bar (torch.testing.assert_close semantics: |a - e| <= atol +
    rtol * |e| for every element), for checks that mirror one of its tests with its
    tolerances. Prints and records the achieved margin: the worst |a - e| / (atol + rtol*|e|)
    (<= 1 passes) and the relative L2 error."""
    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    assert torch.isfinite(a).all(), f"{what}: non-finite values"
    ratio = float(((a - e).abs() / (atol + rtol * e.abs())).max()) if e.numel() else 0.0
    err = float((a - e).abs().max()) if e.numel() else 0.0
    r = rel_l2(a, e) if e.numel() and float(e.norm()) > 0 else err
    test = os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0]
    RECORDS.append((test, what, "ref", "reference", err, ratio, float("nan"), r))
    print(f"[parity] {what}: reference bar (atol {atol:g}, rtol {rtol:g}) worst {ratio:.3f} of the bar, "
          f"max-abs {err:.3e} rel-L2 {r:.3e}", flush=True)
    assert ratio <= 1.0, f"{what}: {ratio:.3f} x the reference's bar (atol {atol:g}, rtol {rtol:g})"


def announce(msg: str) -> None:
    """Name the case on stdout before a GPU step (survives a box that dies mid-step)."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()
    os.fsync(sys.stdout.fileno()) if hasattr(sys.stdout, "fileno") and _is_file(sys.stdout) else None


def _is_file(stream) -> bool:
    try:
        return os.path.isfile(f"/proc/self/fd/{stream.fileno()}")
    except Exception:
        return False
