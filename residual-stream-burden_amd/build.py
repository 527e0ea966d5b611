"""Build libsihc_hip.so (HIP kernels + C ABI) for gfx950 with hipcc, in-tree.

Usage: python residual-stream-burden_amd/build.py [--verbose]

The library lands next to the Python host package (sihc_hip/libsihc_hip.so) so it
travels with the source tree. Packed-fp32 VALU forms are disabled for all device
code (-packed-fp32-ops); hipcc's host pass warns that it does not know the feature.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO_ROOT = PKG_ROOT.parent
SOURCES = [PKG_ROOT / "csrc" / "sihc_kernels.hip"]
OUTPUT = PKG_ROOT / "sihc_hip" / "libsihc_hip.so"
SELFTEST_SOURCE = PKG_ROOT / "csrc" / "abi_selftest.c"
SELFTEST = PKG_ROOT / "sihc_hip" / "sihc_abi_selftest"
ARCH = "gfx950"


def hipcc_path() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    for cand in (os.path.join(rocm, "bin", "hipcc"), shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the SiHC HIP library cannot be built")


def command(output: Path = OUTPUT) -> list[str]:
    return [
        hipcc_path(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-Wall",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", str(REPO_ROOT / "include"),
        *[str(s) for s in SOURCES],
        "-o", str(output),
    ]


def selftest_command(output: Path = SELFTEST) -> list[str]:
    """A plain C caller of the C ABI, linked against the library next to it."""
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return [
        shutil.which("gcc") or "gcc", "-std=c11", "-O2", "-Wall",
        "-D__HIP_PLATFORM_AMD__",  # selects the AMD runtime API in hip_runtime_api.h
        "-I", os.path.join(rocm, "include"), "-I", str(REPO_ROOT / "include"),
        str(SELFTEST_SOURCE),
        "-L", str(OUTPUT.parent), "-lsihc_hip", "-L", os.path.join(rocm, "lib"), "-lamdhip64",
        "-Wl,-rpath,$ORIGIN", "-Wl,-rpath," + os.path.join(rocm, "lib"), "-lm",
        "-o", str(output),
    ]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"{cmd[0]} failed with exit code {proc.returncode}")
    if verbose and proc.stderr.strip():
        # Keep real diagnostics visible; drop the known host-pass feature notice.
        lines = [l for l in proc.stderr.splitlines() if "packed-fp32-ops" not in l]
        if any(l.strip() for l in lines):
            sys.stderr.write("\n".join(lines) + "\n")


def build(verbose: bool = False) -> Path:
    """Compile the library and the C-ABI self-test (always; atomically replaces an
    existing build)."""
    tmp = OUTPUT.with_suffix(".so.tmp")
    _run(command(tmp), verbose)
    os.replace(tmp, OUTPUT)
    tmp = SELFTEST.with_name(SELFTEST.name + ".tmp")
    _run(selftest_command(tmp), verbose)
    os.replace(tmp, SELFTEST)
    return OUTPUT


if __name__ == "__main__":
    out = build(verbose="--verbose" in sys.argv)
    print(out)
