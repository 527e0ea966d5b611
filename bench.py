#!/usr/bin/env python3
"""Benchmark: SiHC fused read+write, forward + backward, at the SiHC-XL shape.

Workload (benchmark config 2): batch 256, 16x16 workspace tokens (256 per image), 4
slots per token (32x32 carrier), D = 1152, 28 layers x 2 sublayers = 56 connection
events, bf16 storage with fp32 accumulation. One step is the whole read/write path of
one batch: every event's fused write+read forward and its fused backward (carrier,
workspace-update and weight gradients), run as the literal per-event schedule

    z_0 = read(X_0);  X_{i+1}, z_{i+1} = write+read(X_i, dz_i);  ...  X_56 = write(X_55)

with each carrier element crossing HBM once per event. The sublayer bodies are not
part of the path: their outputs dz_i ~ N(0,1) and their input gradients
g_i ~ N(0,1e-2) (and the final carrier gradient ~ N(0,1e-2)) are drawn once before
timing, all inputs resident in HBM. Kernels are launched straight through the C ABI
(libsihc_hip.so) on torch's current HIP stream with preallocated outputs.

Prints one JSON line (see the driver contract). `value` is algorithmic HBM GB/s of
the whole step; tokens/s and the fraction of the 8 TB/s peak ride along.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "residual-stream-burden_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "fused read+write fwd+bwd achieved HBM GB/s (% of peak) + tokens/s at SiHC-XL"
HBM_PEAK_GBS = 8000.0
ELEM = 2  # bf16


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--batch", type=int, default=256)
    p.add_argument("--channels", type=int, default=1152)
    p.add_argument("--events", type=int, default=56)
    p.add_argument("--seed", type=int, default=2)
    p.add_argument("--finalize", choices=("chain", "deferred"), default="chain",
                   help="weight-gradient finalize of the backward: in the next launch's trailing blocks "
                        "(sihc_event_backward_chain), or one deferred launch per 32 events after the last event")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-extra", action="store_true", help="skip the secondary config 1/3/4 figures")
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    p.add_argument("--schedule", choices=("stage", "literal"), default="stage",
                   help="routing schedule of --mode e2e")
    p.add_argument("--slots", type=int, choices=(4, 16), default=4,
                   help="cell slots of --mode kernels: 4 (p8, 32x32 carrier) or 16 (p4, 64x64 carrier)")
    p.add_argument("--size", default="B,XL", help="--mode model: presets among B,L,XL,H")
    p.add_argument("--implementation", default="literal,factored,fused,event",
                   help="--mode model: routing implementations")
    p.add_argument("--phase", default="train,inference", help="--mode model: train and/or inference")
    p.add_argument("--model-batch", type=int, default=128, help="--mode model: images per step")
    p.add_argument("--no-graph", action="store_true", help="--mode model: inference without HIP-graph capture")
    p.add_argument("--compile", action="store_true",
                   help="--mode model: torch.compile the model as the reference's fusion_profile does (train: "
                        "mode='default', inference: mode='reduce-overhead', dynamic=False); --mode stage: compile "
                        "the stage schedule's forward (fullgraph) and run the compiled backward")
    p.add_argument("--tri-backward", choices=("visible", "fused"), default=None,
                   help="--mode model --compile: how the triangular op's traced backward returns the update "
                        "gradients (sihc_hip.sublayer_kernels.COMPILED_TRIANGULAR_BACKWARD)")
    p.add_argument("--mode", choices=("step", "calibrate", "kernels", "e2e", "model", "stage", "ceiling", "valu"),
                   default="step",
                   help="step: the benchmark (default); calibrate: a 1 GiB copy-kernel launch plus single "
                        "event forward/backward launches at the same shape, for HBM counter runs; kernels: "
                        "every HIP kernel timed alone at the benchmark shape (one JSON line per kernel); e2e: "
                        "benchmark config 4, a SiHC-XL denoiser forward on a CFG batch with HIP routing; model: the "
                        "reference's fusion_profile matrix (presets x routing implementation x train/inference); "
                        "stage: benchmark config 2 on the reference's stage API (the drop-in path) only; ceiling: "
                        "the streaming ceiling rows only")
    return p.parse_args()


class LiteralStep:
    """Preallocated buffers and the C-ABI call list of one fwd+bwd step."""

    def __init__(self, batch: int, channels: int, events: int, seed: int, index=None):
        """`index`: an optional int32 [batch, 256] state index (benchmark config 3) passed to
        every launch of the step."""
        import torch

        from sihc_hip import _lib

        self.torch = torch
        self.L = _lib.lib()
        self.check = _lib.check
        self.size_array = _lib.size_array
        dev = torch.device("cuda", 0)
        bf = torch.bfloat16
        g = torch.Generator(device=dev).manual_seed(seed)
        B, C, E, S, G, K = batch, channels, events, 4, 16, 2
        self.B, self.C, self.E, self.S, self.G, self.K = B, C, E, S, G, K
        self.M = B * G * G
        carrier = (B, G * K, G * K, C)
        ws = (B, G * G, C)

        def randn(shape, mean=0.0, std=1.0):
            return (mean + std * torch.randn(shape, device=dev, generator=g)).to(bf)

        # Draw order: X, alpha, beta, dz, upstream grads (the order of benchmark configs 0 and 2).
        self.x = [randn(carrier)] + [torch.empty(carrier, device=dev, dtype=bf) for _ in range(E)]
        self.alpha = torch.stack([randn((S, C), 0.25, 0.02).T.contiguous() for _ in range(E)])  # [E,C,S]
        self.beta = torch.stack([randn((S, C), 1.0, 0.02).T.contiguous() for _ in range(E)])
        self.dz = [randn(ws) for _ in range(E)]
        self.gz = [randn(ws, 0.0, 1e-2) for _ in range(E)]
        self.h_out = randn(carrier, 0.0, 1e-2)
        self.z = [torch.empty(ws, device=dev, dtype=bf) for _ in range(E)]
        self.gx = [torch.empty(carrier, device=dev, dtype=bf) for _ in range(2)]
        self.gdz = [torch.empty(ws, device=dev, dtype=bf) for _ in range(E)]
        self.galpha = torch.empty_like(self.alpha)
        self.gbeta = torch.empty_like(self.beta)
        nws = self.L.sihc_event_backward_workspace_size(B, G, K, C)
        # one workspace per backward call (sihc_event_backward_workspace_size: 1,024 chunks x
        # 2 x 4 slots x 1152 channels x 4 B = 37.7 MB at the benchmark shape); under the
        # deferred schedule each keeps its partial rows until the finalize after the last
        # event (slot E: the first read's adjoint, whose rows must not overwrite event 0's)
        self.work = [torch.empty((nws + 15) // 16 * 4, device=dev, dtype=torch.float32) for _ in range(E + 1)]
        self.info = (ctypes.c_int * (2 * E + 2))()
        self.stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        self.index = index
        self._build(E)

    def _build(self, E):
        L, B, G, K, C = self.L, self.B, self.G, self.K, self.C
        vp = ctypes.c_void_p
        p = lambda t: vp(t.data_ptr())  # noqa: E731
        bf16 = 1
        nwork = self.work[0].numel() * 4
        info = lambda k: ctypes.cast(ctypes.addressof(self.info) + 8 * k, ctypes.POINTER(ctypes.c_int))  # noqa: E731
        U = self.M * C * ELEM
        S = self.S
        # the state index is read once per launch (4 B per token) and counted as such
        ix = None if self.index is None else p(self.index)
        w_bytes = C * S * ELEM
        ixb = 0 if self.index is None else self.M * 4
        fwd, bwd = [], []
        # forward
        outs = (vp * 1)(self.z[0].data_ptr())
        fwd.append(("read", L.sihc_read, (p(self.x[0]), p(self.alpha[0]), outs, 1, B, G, K, C, ix, bf16,
                                           self.stream), (S + 1) * U + w_bytes + ixb))
        for i in range(E):
            last = i == E - 1
            fwd.append(("event_forward_last" if last else "event_forward", L.sihc_event_forward,
                        (p(self.x[i]), p(self.dz[i]), p(self.beta[i]), None if last else p(self.alpha[i + 1]),
                         p(self.x[i + 1]), None if last else p(self.z[i + 1]), B, G, K, C, ix, bf16, self.stream),
                        ((2 * S + 1) if last else (2 * S + 2)) * U + (1 if last else 2) * w_bytes + ixb))
        # backward: last event (write only, carrier gradient aliased), then full events, each
        # with its weight-gradient finalize deferred (sihc_event_backward_partial) ...
        h = self.h_out
        bwd.append(("event_backward_last", L.sihc_event_backward_partial,
                    (p(h), None, None, p(self.dz[E - 1]), p(self.beta[E - 1]), None, None, p(self.gdz[E - 1]),
                     p(self.gbeta[E - 1]), None, B, G, K, C, ix, bf16, bf16, p(self.work[E - 1]), nwork, info(E - 1),
                     self.stream), (S + 2) * U + 2 * w_bytes + ixb))
        for i in range(E - 2, -1, -1):
            dst = self.gx[i % 2]
            bwd.append(("event_backward", L.sihc_event_backward_partial,
                        (p(h), p(self.gz[i + 1]), p(self.x[i + 1]), p(self.dz[i]), p(self.beta[i]),
                         p(self.alpha[i + 1]), p(dst), p(self.gdz[i]), p(self.gbeta[i]), p(self.galpha[i + 1]),
                         B, G, K, C, ix, bf16, bf16, p(self.work[i]), nwork, info(i), self.stream),
                        (3 * S + 3) * U + 4 * w_bytes + ixb))
            h = dst
        # adjoint of the first read (no write part): dX_0 = h + alpha_0 (x) g_0, dalpha_0
        dst = self.gx[1] if h is self.gx[0] else self.gx[0]
        bwd.append(("event_backward_first", L.sihc_event_backward_partial,
                    (p(h), p(self.gz[0]), p(self.x[0]), None, None, p(self.alpha[0]), p(dst), None, None,
                     p(self.galpha[0]), B, G, K, C, ix, bf16, bf16, p(self.work[E]), nwork, info(E),
                     self.stream), (3 * S + 1) * U + 2 * w_bytes + ixb))
        # ... then every event's dbeta / dalpha in one launch per 32 events (same bits)
        self.finalize_args = None
        bwd.append(("event_finalize", self._finalize, (), 0))
        self.fwd, self.bwd = fwd, bwd
        self.bwd_chain = self._chain(bwd[:-1])
        self.bwd_run = self.bwd_chain
        self.bytes_fwd = sum(c[3] for c in fwd)
        self.bytes_bwd = sum(c[3] for c in bwd)

    def use_chain(self, chain: bool) -> None:
        """Backward launches of step(): chained finalizes, or one deferred finalize."""
        self.bwd_run = self.bwd_chain if chain else self.bwd

    def _chain(self, partial_calls):
        """The same backward launches as sihc_event_backward_chain calls: each finalizes the
        previous call's partial rows in its trailing blocks, so only the last call (slot E,
        the first read's adjoint) needs a finalize launch of its own."""
        E, L = self.E, self.L
        vp = ctypes.c_void_p
        gb = [self.gbeta[i] for i in range(E)] + [None]
        ga = [self.galpha[i + 1] for i in range(E - 1)] + [None, self.galpha[0]]
        slots = [E - 1] + list(range(E - 2, -1, -1)) + [E]  # slot of each backward call, in call order
        info = lambda k: ctypes.cast(ctypes.addressof(self.info) + 8 * k, ctypes.POINTER(ctypes.c_int))  # noqa: E731
        p = lambda t: None if t is None else vp(t.data_ptr())  # noqa: E731
        calls = []
        for j, (name, _, args, nbytes) in enumerate(partial_calls):
            k = slots[j - 1]
            prev = (None, 0, None, None, None) if j == 0 else \
                (p(self.work[k]), self.work[k].numel() * 4, info(k), p(gb[k]), p(ga[k]))
            calls.append((name, L.sihc_event_backward_chain, args[:-1] + prev + (args[-1],), nbytes))
        last = slots[-1]
        ptrs = lambda ts: (vp * len(ts))(*(None if t is None else t.data_ptr() for t in ts))  # noqa: E731
        fin = (1, ptrs([self.work[last]]), self.size_array([self.work[last].numel() * 4]), info(last),
               ptrs([gb[last]]), ptrs([ga[last]]), self.K, self.C, 1, self.stream)
        calls.append(("event_finalize", L.sihc_event_finalize, fin, 0))
        return calls

    def _finalize(self):
        """sihc_event_finalize over the E + 1 deferred backward calls: slot i < E holds
        event i's dbeta_i (and dalpha_{i+1}, except the last event's write-only slot); slot
        E the first read's dalpha_0. The info slots were filled by the calls this step."""
        if self.finalize_args is None:
            E = self.E
            ptrs = lambda ts: (ctypes.c_void_p * len(ts))(*(None if t is None else t.data_ptr() for t in ts))  # noqa
            self.finalize_args = (E + 1, ptrs(self.work), self.size_array(w.numel() * 4 for w in self.work), self.info,
                                  ptrs([self.gbeta[i] for i in range(E)] + [None]),
                                  ptrs([self.galpha[i + 1] for i in range(E - 1)] + [None, self.galpha[0]]),
                                  self.K, self.C, 1, self.stream)
        return self.L.sihc_event_finalize(*self.finalize_args)

    def run(self, calls):
        for _, fn, args, _ in calls:
            self.check(fn(*args))

    def spans(self, calls, name):
        """(head, body, tail) of a call list: body is the run of consecutive `name` calls
        (the full per-event launches), head and tail the calls before and after it."""
        idx = [i for i, c in enumerate(calls) if c[0] == name]
        lo, hi = idx[0], idx[-1] + 1
        assert idx == list(range(lo, hi)), f"{name} launches are not consecutive"
        return calls[:lo], calls[lo:hi], calls[hi:]

    def step(self, marks=None):
        """One fwd+bwd step. With `marks` (a list), HIP events on the launch stream are
        recorded only at the ends of the runs of full per-event launches and at the end of
        the forward, appended as (f0, f1, fe, b0, b1, n_fwd, n_bwd): (f1 - f0) spans the
        full forward launches, (b1 - b0) the full backward launches, inter-launch gaps
        included, and fe ends the forward phase. Events between every launch would
        each add a marker packet and an idle gap of several microseconds to the step."""
        if marks is None:
            self.run(self.fwd)
            self.run(self.bwd_run)
            return
        ev = lambda: self.torch.cuda.Event(enable_timing=True)  # noqa: E731
        f0, f1, fe, b0, b1 = ev(), ev(), ev(), ev(), ev()
        fh, fb, ft = self.spans(self.fwd, "event_forward")
        bh, bb, bt = self.spans(self.bwd_run, "event_backward")
        self.run(fh)
        f0.record()
        self.run(fb)
        f1.record()
        self.run(ft)
        fe.record()
        self.run(bh)
        b0.record()
        self.run(bb)
        b1.record()
        self.run(bt)
        marks.append((f0, f1, fe, b0, b1, len(fb), len(bb)))


def measure_step(torch, step: LiteralStep, steps: int, warmup: int) -> dict:
    """Time `steps` steps back to back after `warmup` untimed ones, bracketed by device
    synchronisation, with no HIP event inside (an event record between two launches idles
    the GPU for several microseconds). The average launch times of the full per-event
    kernels and the phase split come from marked one-stream steps run after it: HIP events
    there mark only the phase boundaries and the two runs of full per-event launches."""
    torch.cuda.synchronize()
    for _ in range(warmup):
        step.step()
    torch.cuda.synchronize()
    print(f"[bench] warmup done ({warmup} steps)", file=sys.stderr, flush=True)
    marks: list = []
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    t0 = time.perf_counter()
    for _ in range(steps):
        step.step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    spans = []
    for _ in range(max(2, min(steps, 5))):
        a, c = ev(), ev()
        a.record()
        step.step(marks)
        c.record()
        spans.append((a, c))
    torch.cuda.synchronize()
    return {
        "ms_step": wall / steps * 1e3,
        "marked_ms": statistics.median(a.elapsed_time(c) for a, c in spans),
        "fwd_kernel_ms": statistics.median(f0.elapsed_time(f1) / nf for f0, f1, _, _, _, nf, _ in marks),
        "bwd_kernel_ms": statistics.median(b0.elapsed_time(b1) / nb for _, _, _, b0, b1, _, nb in marks),
        "bwd_launches": sum(mk[6] for mk in marks),
        # phase split from the step's own events: forward = start .. end of the forward tail
        "fwd_ms": statistics.median(a.elapsed_time(mk[2]) for (a, _), mk in zip(spans, marks)),
        "bwd_ms": statistics.median(mk[2].elapsed_time(c) for (_, c), mk in zip(spans, marks)),
    }


def _timed(torch, fn, iters=10, warmup=2):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(iters):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / iters * 1e-3


def stream_ceiling() -> dict:
    """HBM streaming ceiling of this GPU in the same run: the library's calibration stream
    (sihc_stream: one-shot 256-thread blocks that each move one 4 KB unit of every array,
    16-byte vectors, non-temporal loads and stores -- the fastest pattern measured here for
    mixed traffic). Rows: write-only, 1:1 over 2 arrays and 2:1 over 3, at 8-9 GiB per pass;
    and the per-event kernels' own arrays at the benchmark's sizes (shapes 1 and 2:
    carrier-shaped arrays 4 x the 151 MB workspace-shaped ones, as x / x_out / grad x are to
    dz / z_out / grad dz; 1.5 and 2.3 GB per pass, as one launch of those kernels moves).
    The shaped streams slow down as the arrays grow (1 GiB workspace arrays: about 8%
    slower), so they are measured at the size the kernels see. One warm-up pass, then the
    median of 3 runs of back-to-back passes (20 for the kernels' arrays, 4 for the 8-9 GiB
    mixes)."""
    import torch

    from sihc_hip import _lib

    L = _lib.lib()
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    # name: (sources, destinations, shape, workspace-shaped bytes, carrier-shaped sources, destinations)
    mixes = {"write-only (1 array)": (0, 1, 0, 8 << 30, 0, 0), "1:1 (2 arrays)": (1, 1, 0, 4 << 30, 0, 0),
             "2:1 (3 arrays)": (2, 1, 0, 3 << 30, 0, 0),
             "per-event forward's arrays (1:1, 10 units)": (2, 2, 1, 150994944, 1, 1),
             "per-event backward's arrays (2:1, 15 units)": (4, 2, 2, 150994944, 2, 1)}
    out = {"workload": "sihc_stream, one-shot 4 KB units per block, non-temporal loads and stores; generic mixes "
                       "over 8-9 GiB per pass, the per-event kernels' arrays at the benchmark's sizes"}
    for name, (nr, nw, shape, each, r4, w4) in mixes.items():
        srcs_t = [torch.empty((4 if r < r4 else 1) * each, dtype=torch.uint8, device="cuda") for r in range(nr)]
        dsts_t = [torch.empty((4 if w < w4 else 1) * each, dtype=torch.uint8, device="cuda") for w in range(nw)]
        for t in srcs_t:
            t.fill_(1)
        total = sum(t.numel() for t in srcs_t + dsts_t)
        srcs = (ctypes.c_void_p * max(nr, 1))(*[t.data_ptr() for t in srcs_t])
        dsts = (ctypes.c_void_p * nw)(*[t.data_ptr() for t in dsts_t])
        # back-to-back passes, as the step runs its kernels (a single pass after an idle
        # synchronisation runs up to ~8% faster than the same pass in a back-to-back run)
        reps = 4 if shape == 0 else 20
        _lib.check(L.sihc_stream(srcs, nr, dsts, nw, each, shape, st))
        passes = []
        for _ in range(3):
            a0, b0 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a0.record()
            for _ in range(reps):
                _lib.check(L.sihc_stream(srcs, nr, dsts, nw, each, shape, st))
            b0.record()
            torch.cuda.synchronize()
            passes.append(a0.elapsed_time(b0) * 1e-3 / reps)
        sec = statistics.median(passes)
        out[name] = {"GB/s": round(total / sec / 1e9, 1), "frac_of_peak": round(total / sec / 1e9 / HBM_PEAK_GBS, 4),
                     "bytes_per_pass": total, "ms": round(sec * 1e3, 3)}
        del srcs_t, dsts_t
        torch.cuda.empty_cache()
    return out


def valu_rate() -> None:
    """Sustained vector-ALU rates without packed fp32 (sihc_fma_rate): 4, 8 or 16 independent
    chains per thread, 4 steps per iteration, 20,000 iterations, on 8 to 32 blocks of 256
    threads per CU, in four instruction forms: fp32 fma with register operands (v_fma_f32),
    with literal constants (v_fmamk_f32), the bf16 pair dot (v_dot2c_f32_bf16, 2 lane-FMAs
    each) and the accumulating fma (v_fmac_f32, the form of the kernels' sums). One warm-up launch, then the median of 5
    launches timed with HIP events. Prints one JSON line per case."""
    import torch

    from sihc_hip import _lib

    L = _lib.lib()
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    iters = 20000
    forms = {0: "v_fma_f32 (register operands)", 1: "v_fmamk_f32 (literal constants)", 2: "v_dot2c_f32_bf16",
             3: "v_fmac_f32 (accumulating)"}
    cases = [(0, 4, 8), (0, 4, 32), (0, 8, 32), (0, 16, 32), (1, 8, 32), (1, 16, 32), (2, 8, 32), (2, 16, 32),
             (3, 8, 32), (3, 16, 32)]
    for form, chains, per_cu in cases:
        blocks = cus * per_cu
        out = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
        run = lambda: _lib.check(L.sihc_fma_rate(ctypes.c_void_p(out.data_ptr()), chains, form, blocks, iters, st))  # noqa
        run()
        torch.cuda.synchronize()
        ts = []
        for _ in range(5):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            run()
            b.record()
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b) * 1e-3)
        sec = statistics.median(ts)
        fmas = blocks * 256 * iters * 4 * chains * (2 if form == 2 else 1)
        print(json.dumps({"form": forms[form], "chains": chains, "blocks_per_cu": per_cu, "cus": cus,
                          "ms": round(sec * 1e3, 3), "lane_fma_per_s": fmas / sec,
                          "lane_fma_per_cu_clock_2p4ghz": round(fmas / sec / cus / 2.4e9, 1),
                          "finite": bool(torch.isfinite(out).all())}), flush=True)


def extra_configs(seed: int) -> dict:
    """Secondary figures on benchmark configs 1 and 3 (not the headline `value`).

    config 1: SiHC-B shape (batch 256, D=768), forward only, one 24-event stage, as the
      per-event fused schedule and as the reference's stage API (read E=24, triangular
      with 1..23 active updates, write E=24). Sublayer outputs pre-drawn.
    config 3: spatially indexed variant (batch 128, D=1152, group-of-5 index): the
      per-event fused forward and backward through the index, and the explicit bit-exact
      gather/scatter of every token's state.
    """
    import torch

    from sihc_hip import launch
    from sihc_hip.indexed import group_index

    dev = torch.device("cuda", 0)
    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(seed)
    r = lambda shape, m=0.0, sd=1.0: (m + sd * torch.randn(shape, device=dev, generator=g)).to(bf)  # noqa: E731
    out = {}
    # ---- config 1
    B, C, E, S = 256, 768, 24, 4
    U = B * 256 * C * ELEM
    x0 = r((B, 32, 32, C))
    alpha = r((E, C, S), 0.25, 0.02)
    beta = r((E, C, S), 1.0, 0.02)
    dz = [r((B, 256, C)) for _ in range(E)]
    gamma = (alpha[:, None].float() * beta[None, :].float()).sum(-1).to(bf)
    xs = [x0] + [torch.empty_like(x0) for _ in range(E)]

    def literal():
        launch.read(x0, alpha[:1])
        for i in range(E):
            launch.event_forward(xs[i], dz[i], beta[i], alpha[i + 1] if i + 1 < E else None)

    def stage():
        base = launch.read(x0, alpha)
        for i in range(1, E):
            launch.triangular(base[i], dz[:i], gamma[i, :i].contiguous())
        launch.write(x0, dz, beta)

    lit_bytes = ((S + 1) + (E - 1) * (2 * S + 2) + (2 * S + 1)) * U
    stage_bytes = ((S + E) + sum(i + 2 for i in range(1, E)) + (2 * S + E)) * U
    t_lit, t_stage = _timed(torch, literal, iters=5), _timed(torch, stage, iters=5)
    out["config1_forward"] = {
        "workload": "batch 256, D=768, 24 events (12 layers x 2 sublayers), forward only, bf16",
        "per_event_fused": {"ms": round(t_lit * 1e3, 3), "GB/s": round(lit_bytes / t_lit / 1e9, 1),
                            "bytes": lit_bytes, "tokens_per_s": round(B * 256 / t_lit, 1)},
        "stage_api": {"ms": round(t_stage * 1e3, 3), "GB/s": round(stage_bytes / t_stage / 1e9, 1),
                      "bytes": stage_bytes, "tokens_per_s": round(B * 256 / t_stage, 1)},
    }
    del xs, dz, x0
    torch.cuda.empty_cache()
    # ---- 16-slot cells (patch 4, 64x64 carrier): the same 24-event forward at D=1152
    B, C, E, S = 256, 1152, 24, 16
    U = B * 256 * C * ELEM
    x0 = r((B, 64, 64, C))
    alpha = r((E, C, S), 1.0 / S, 0.02)
    beta = r((E, C, S), 1.0, 0.02)
    dz = [r((B, 256, C)) for _ in range(E)]
    gamma = (alpha[:, None].float() * beta[None, :].float()).sum(-1).to(bf)
    xs = [x0, torch.empty_like(x0), torch.empty_like(x0)]

    def literal16():
        launch.read(x0, alpha[:1])
        for i in range(E):
            src = x0 if i == 0 else xs[1 + (i - 1) % 2]
            launch.event_forward(src, dz[i], beta[i], alpha[i + 1] if i + 1 < E else None)

    def stage16():
        base = launch.read(x0, alpha)
        for i in range(1, E):
            launch.triangular(base[i], dz[:i], gamma[i, :i].contiguous())
        launch.write(x0, dz, beta)

    lit_bytes = ((S + 1) + (E - 1) * (2 * S + 2) + (2 * S + 1)) * U
    stage_bytes = ((S + E) + sum(i + 2 for i in range(1, E)) + (2 * S + E)) * U
    t_lit, t_stage = _timed(torch, literal16, iters=3), _timed(torch, stage16, iters=3)
    out["p4_forward"] = {
        "workload": "16-slot cells: batch 256, 64x64 carrier, D=1152, 24 events, forward only, bf16",
        "per_event_fused": {"ms": round(t_lit * 1e3, 3), "GB/s": round(lit_bytes / t_lit / 1e9, 1),
                            "bytes": lit_bytes, "tokens_per_s": round(B * 256 / t_lit, 1)},
        "stage_api": {"ms": round(t_stage * 1e3, 3), "GB/s": round(stage_bytes / t_stage / 1e9, 1),
                      "bytes": stage_bytes, "tokens_per_s": round(B * 256 / t_stage, 1)},
    }
    del xs, dz, x0
    torch.cuda.empty_cache()
    out["config3_indexed"] = config3_indexed(seed)
    return out


def config3_indexed(seed: int) -> dict:
    """Benchmark config 3 (batch 128, D=1152, bf16, the seeded group-of-5 state index):
    the per-event fused forward and backward through the index and without it, and the
    explicit bit-exact gather/scatter of every token's state."""
    import torch

    from sihc_hip import launch
    from sihc_hip.indexed import group_index

    dev = torch.device("cuda", 0)
    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(seed + 3)
    r = lambda shape, m=0.0, sd=1.0: (m + sd * torch.randn(shape, device=dev, generator=g)).to(bf)  # noqa: E731
    # ---- config 3: preallocated buffers, launches through the C ABI (as the config-2 step),
    # the backward with its own finalize launch (sihc_event_backward)
    from sihc_hip import _lib

    L3 = _lib.lib()
    st3 = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    vp = ctypes.c_void_p
    B, C, S = 128, 1152, 4
    U = B * 256 * C * ELEM
    x = r((B, 32, 32, C))
    idx = group_index(B, 16, 5, seed=3).to(dev)
    d = r((B, 256, C))
    bw, aw = r((C, S), 1.0, 0.02), r((C, S), 0.25, 0.02)
    h, gz = r((B, 32, 32, C), 0.0, 1e-2), r((B, 256, C), 0.0, 1e-2)
    xo, zo, gx3 = torch.empty_like(x), torch.empty_like(d), torch.empty_like(x)
    gdz3, gb3, ga3 = torch.empty_like(d), torch.empty_like(bw), torch.empty_like(aw)
    nws3 = L3.sihc_event_backward_workspace_size(B, 16, 2, C)
    ws3 = torch.empty(nws3, dtype=torch.uint8, device=dev)
    p3 = lambda t: vp(t.data_ptr())  # noqa: E731

    def fwd3(ix):
        _lib.check(L3.sihc_event_forward(p3(x), p3(d), p3(bw), p3(aw), p3(xo), p3(zo), B, 16, 2, C,
                                         None if ix is None else p3(ix), 1, st3))

    def bwd3(ix):
        _lib.check(L3.sihc_event_backward(p3(h), p3(gz), p3(xo), p3(d), p3(bw), p3(aw), p3(gx3), p3(gdz3),
                                          p3(gb3), p3(ga3), B, 16, 2, C, None if ix is None else p3(ix), 1, 1,
                                          p3(ws3), nws3, st3))

    fwd3(idx)
    cells = launch.gather_cells(x, idx, S)
    # fresh buffers: the first few dozen launches over them run several % slower, so both
    # the indexed and the unindexed launches warm up before either is timed
    for _ in range(10):
        fwd3(idx), bwd3(idx), fwd3(None), bwd3(None)
    fwd3(idx)
    t_f, t_b = _timed(torch, lambda: fwd3(idx), iters=20), _timed(torch, lambda: bwd3(idx), iters=20)
    t_g = _timed(torch, lambda: launch.gather_cells(x, idx, S))
    t_s = _timed(torch, lambda: launch.scatter_cells(cells, idx))
    # the same launches without the index, for the cost of the index at this batch
    t_fu, t_bu = _timed(torch, lambda: fwd3(None), iters=20), _timed(torch, lambda: bwd3(None), iters=20)
    per_call = {
        "schedule": "one event's forward, then its backward with its own finalize launch (sihc_event_backward), "
                    "the same buffers every call",
        "event_forward_GB/s": round(10 * U / t_f / 1e9, 1), "event_backward_GB/s": round(15 * U / t_b / 1e9, 1),
        "unindexed_event_forward_GB/s": round(10 * U / t_fu / 1e9, 1),
        "unindexed_event_backward_GB/s": round(15 * U / t_bu / 1e9, 1),
    }
    out = {"gather_GB/s": round(2 * S * U / t_g / 1e9, 1), "scatter_GB/s": round(2 * S * U / t_s / 1e9, 1)}
    del x, d, h, gz, xo, zo, gx3, gdz3, ws3, cells
    torch.cuda.empty_cache()
    # ---- the config-2 step at config 3's shape: 56 events (28 layers x 2 sublayers) on
    # per-event buffers, the backward as a chain of sihc_event_backward_chain calls, every
    # launch through the state index; then the same step without it. Per-launch rates are
    # the span averages of the full per-event launches (measure_step).
    steps = {}
    for name, ix in (("indexed", idx), ("unindexed", None)):
        st = LiteralStep(B, C, 56, seed + 3, index=ix)
        st.use_chain(True)
        m = measure_step(torch, st, steps=5, warmup=2)
        fwd_b = next(c[3] for c in st.fwd if c[0] == "event_forward")
        bwd_b = next(c[3] for c in st.bwd if c[0] == "event_backward")
        steps[name] = {"ms_per_step": round(m["ms_step"], 3),
                       "GB/s": round((st.bytes_fwd + st.bytes_bwd) / (m["ms_step"] * 1e-3) / 1e9, 1),
                       "tokens_per_s": round(B * 256 / (m["ms_step"] * 1e-3), 1),
                       "event_forward_GB/s": round(fwd_b / (m["fwd_kernel_ms"] * 1e-3) / 1e9, 1),
                       "event_backward_GB/s": round(bwd_b / (m["bwd_kernel_ms"] * 1e-3) / 1e9, 1),
                       "event_backward_avg_ms": round(m["bwd_kernel_ms"], 4)}
        del st
        torch.cuda.empty_cache()
    return {
        "workload": "batch 128, D=1152, int32 state index (seeded groups of 5), bf16, C-ABI launches on "
                    "preallocated buffers: the config-2 step's schedule at this shape (56 events, chained "
                    "backward finalizes; 'step'), and single events with their own finalize launch ('per_call')",
        "event_forward_GB/s": steps["indexed"]["event_forward_GB/s"],
        "event_backward_GB/s": steps["indexed"]["event_backward_GB/s"],
        "unindexed_event_forward_GB/s": steps["unindexed"]["event_forward_GB/s"],
        "unindexed_event_backward_GB/s": steps["unindexed"]["event_backward_GB/s"],
        "step": steps, "per_call": per_call, **out,
        "event_fwd_bwd_tokens_per_s": round(B * 256 / (t_f + t_b), 1),
    }


def stage_api_config2(seed: int, steps: int = 3, compiled: bool = False) -> dict:
    """Benchmark config 2 on the reference's own schedule (sublayer.py:52-72), the drop-in
    path: per stage of 8/12/8 blocks (16/24/16 events) read -> triangular -> write through
    the sihc:: custom ops, then torch autograd back through them, batch 256, D = 1152, bf16.
    As in the per-event leg the sublayer bodies are not part of the path: the updates dz_i
    are pre-drawn leaves and the bodies' input gradients g_i = dL/dz_i are pre-drawn upstream
    gradients of the read outputs z_i. Bytes: the algorithmic bytes of the kernel ops
    launched (read (S+E), triangular i (i+2), write (2S+E); backward: update reads and the
    weight gradients (S+E) each, fused triangular backward (1+2i)); the time also covers
    autograd's own work. Eagerly, autograd adds up each update's gradient contributions
    (one from the write's adjoint, one from every later triangular op of its stage) in
    bf16, E(E-1)/2 adds of 3 U per stage: that traffic is reported apart
    (accumulation_units) and in the all-traffic rate. With `compiled`, the schedule's
    forward is compiled by Inductor (mode="default", fullgraph) and autograd runs the
    compiled backward, where the triangular update gradients stay visible to Inductor and
    are fused with that accumulation."""
    import torch

    from sihc_hip.sublayer_kernels import sublayer_read, sublayer_triangular, sublayer_write

    dev = torch.device("cuda", 0)
    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(seed)
    r = lambda shape, m=0.0, sd=1.0: (m + sd * torch.randn(shape, device=dev, generator=g)).to(bf)  # noqa: E731
    B, C, S = 256, 1152, 4
    U = B * 256 * C * ELEM
    stages = (16, 24, 16)
    x0 = r((B, 32, 32, C)).requires_grad_()
    alphas = [r((e, C, S), 0.25, 0.02).requires_grad_() for e in stages]
    betas = [r((e, C, S), 1.0, 0.02).requires_grad_() for e in stages]
    dzs = [[r((B, 256, C)).requires_grad_() for _ in range(e)] for e in stages]
    gzs = [[r((B, 256, C), 0.0, 1e-2) for _ in range(e)] for e in stages]
    g_out = r((B, 32, 32, C), 0.0, 1e-2)

    def forward(x, alphas, betas, dzs):
        outs = []
        for alpha, beta, dz in zip(alphas, betas, dzs):
            base = sublayer_read(x, alpha)
            gamma = (alpha[:, None] * beta[None, :]).sum(-1)
            for i in range(len(dz)):
                outs.append(base[i] if i == 0 else sublayer_triangular(base[i], dz[:i], gamma[i, :i].contiguous()))
            x = sublayer_write(x, dz, beta)
        return outs, x

    fwd = forward
    if compiled:
        torch._dynamo.reset()
        fwd = torch.compile(forward, mode="default", fullgraph=True)
    flat_gz = [g for gs in gzs for g in gs]

    def run():
        outs, x = fwd(x0, alphas, betas, dzs)
        torch.autograd.backward(outs + [x], flat_gz + [g_out])

    fwd_u = sum((S + e) + sum(i + 2 for i in range(1, e)) + (2 * S + e) for e in stages)
    bwd_u = sum(4 * (S + e) + sum(1 + 2 * i for i in range(1, e)) for e in stages)
    acc_u = sum(3 * e * (e - 1) // 2 for e in stages)  # eager autograd: bf16 a + b per extra contribution
    tc = time.perf_counter()
    for _ in range(1):
        run()
    if compiled:
        torch.cuda.synchronize()
        print(f"[bench] stage API compiled: first step {time.perf_counter() - tc:.1f} s", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        for t in [x0, *alphas, *betas, *(d for ds in dzs for d in ds)]:
            t.grad = None
        run()
    torch.cuda.synchronize()
    sec = (time.perf_counter() - t0) / steps
    nbytes = (fwd_u + bwd_u) * U
    out = {"workload": "benchmark config 2 on the reference's stage schedule (read -> triangular -> write, stages "
                       "8/12/8) through the sihc:: custom ops, fwd + autograd bwd, batch 256, D=1152, bf16"
                       + (", forward compiled by Inductor (fullgraph), compiled backward" if compiled else ", eager"),
           "ms_per_step": round(sec * 1e3, 3), "kernel_op_bytes": nbytes, "fwd_units": fwd_u, "bwd_units": bwd_u,
           "GB/s": round(nbytes / sec / 1e9, 1), "frac_of_peak": round(nbytes / sec / 1e9 / HBM_PEAK_GBS, 4),
           "tokens_per_s": round(B * 256 / sec, 1)}
    if compiled:
        # traffic of the compiled backward: the gamma reduction (1 + i) U per triangular op
        # instead of the fused (1 + 2i) U, and one fused pass per update gradient (the later
        # read gradients, the write adjoint's contribution and the result: E - 1 - j + 2)
        cb = sum(4 * (S + e) + sum(1 + i for i in range(1, e)) + sum(e - 1 - j + 2 for j in range(e)) for e in stages)
        out.update({"compiled_bwd_units": cb, "compiled_traffic_GB/s": round((fwd_u + cb) * U / sec / 1e9, 1)})
    else:
        allb = nbytes + acc_u * U
        out.update({"accumulation_units": acc_u, "all_traffic_bytes": allb,
                    "all_traffic_GB/s": round(allb / sec / 1e9, 1),
                    "all_traffic_frac_of_peak": round(allb / sec / 1e9 / HBM_PEAK_GBS, 4)})
    del x0, alphas, betas, dzs, gzs, g_out
    torch.cuda.empty_cache()
    return out


def cpu_baseline(budget_s: float) -> dict:
    """benchmark config 0 on the host: the oracle's unfused PyTorch read/write (fp32,
    batch 8, 256 tokens, 4 slots, D=768, one event) forward + autograd backward."""
    import torch

    from oracle import sihc_oracle as O

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    torch.manual_seed(0)
    x = torch.randn(8, 32, 32, 768)
    alpha = (0.25 + 0.02 * torch.randn(4, 768)).T.contiguous()
    beta = (1.0 + 0.02 * torch.randn(4, 768)).T.contiguous()
    y = torch.randn(8, 256, 768)
    gxp = 1e-2 * torch.randn(8, 32, 32, 768)
    gz = 1e-2 * torch.randn(8, 256, 768)
    leaves = [t.clone().requires_grad_() for t in (x, alpha, beta, y)]

    def once():
        t0 = time.perf_counter()
        z = O.read_torch(leaves[0], leaves[1])
        xp = O.write_torch(leaves[0], [leaves[3]], [leaves[2]])
        t1 = time.perf_counter()
        torch.autograd.grad((xp * gxp).sum() + (z * gz).sum(), leaves)
        t2 = time.perf_counter()
        return t1 - t0, t2 - t1

    for _ in range(3):
        once()
    fwd, bwd = [], []
    t_start = time.perf_counter()
    while len(fwd) < 20 and (time.perf_counter() - t_start < budget_s or len(fwd) < 3):
        f, b = once()
        fwd.append(f)
        bwd.append(b)
    U = 8 * 256 * 768 * 4
    byt = 14 * U + 20 * U  # unfused single event: forward 14 U, backward 20 U (fp32)
    t = statistics.median(fwd) + statistics.median(bwd)
    return {
        "value": round(byt / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "tokens_per_s": round(8 * 256 / t, 1),
        "fwd_ms": round(statistics.median(fwd) * 1e3, 3), "bwd_ms": round(statistics.median(bwd) * 1e3, 3),
        "runs": len(fwd),
        "sample": ("benchmark config 0 on the host: oracle/ restatement of the reference's unfused PyTorch "
                   "read_torch/write_torch + autograd, fp32, batch 8 x 256 tokens, 4 slots, D=768, one event "
                   "fwd+bwd, median of up to 20 runs after 3 warmups; GB/s from the same algorithmic bytes "
                   "(14 U fwd + 20 U bwd, U = one fp32 workspace tensor)"),
    }


def traffic_from_profiles() -> float | None:
    """HBM bytes per dominant-kernel launch measured by rocprofv3 counters, if committed."""
    f = ROOT / "profiles" / "event_backward_traffic.json"
    if not f.exists():
        return None
    try:
        return float(json.loads(f.read_text())["bytes_per_launch"])
    except Exception:
        return None


def calibrate(args) -> None:
    """Launches for rocprofv3 counter runs: the library's copy kernel over a known byte
    count (the FETCH_SIZE/WRITE_SIZE scale), 3 per-event forwards, then 4 full per-event
    backwards at the benchmark shape as the step launches them: a first
    sihc_event_backward_partial, then 3 sihc_event_backward_chain calls, each finalizing the
    previous call's partial rows in its trailing blocks (the dispatches 2-4 are the ones the
    step repeats 54 times)."""
    import torch

    step = LiteralStep(args.batch, args.channels, 2, args.seed)
    L, check = step.L, step.check
    copy_bytes = 1 << 30
    src = torch.empty(copy_bytes, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    src.fill_(1)
    torch.cuda.synchronize()
    fwd = next(c for c in step.fwd if c[0] == "event_forward")
    for _ in range(3):
        check(L.sihc_copy(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), copy_bytes, step.stream))
    # full backward of event 0 (reads grad of x_1 and z_1, x_1, dz_0; writes grad_x_0, grad_dz_0)
    vp = ctypes.c_void_p
    p = lambda t: vp(t.data_ptr())  # noqa: E731
    B, G, K, C = step.B, step.G, step.K, step.C
    nwork = step.work[0].numel() * 4
    info = (ctypes.c_int * 8)()
    slot = lambda k: ctypes.cast(ctypes.addressof(info) + 8 * k, ctypes.POINTER(ctypes.c_int))  # noqa: E731
    grads = [(torch.empty_like(step.gbeta[0]), torch.empty_like(step.galpha[1])) for _ in range(4)]
    works = [step.work[0], step.work[1]]

    def bwd_args(k):
        return (p(step.h_out), p(step.gz[1]), p(step.x[1]), p(step.dz[0]), p(step.beta[0]), p(step.alpha[1]),
                p(step.gx[0]), p(step.gdz[0]), p(grads[k][0]), p(grads[k][1]), B, G, K, C, None, 1, 1,
                p(works[k % 2]), nwork, slot(k))

    for _ in range(3):
        check(fwd[1](*fwd[2]))
    check(L.sihc_event_backward_partial(*bwd_args(0), step.stream))
    for k in range(1, 4):
        prev = (p(works[(k - 1) % 2]), nwork, slot(k - 1), p(grads[k - 1][0]), p(grads[k - 1][1]))
        check(L.sihc_event_backward_chain(*bwd_args(k), *prev, step.stream))
    torch.cuda.synchronize()
    U = step.M * C * ELEM
    rows = info[6] * 2 * step.S * C * 4  # partial rows of one launch
    print(json.dumps({"copy_bytes_read": copy_bytes, "copy_bytes_written": copy_bytes,
                      "event_forward_bytes": fwd[3], "event_backward_bytes": 15 * U + 4 * C * 4 * ELEM,
                      "event_forward_read": 5 * U, "event_forward_written": 5 * U,
                      "event_backward_read": 10 * U, "event_backward_written": 5 * U,
                      "event_backward_partial_rows_bytes": rows}), flush=True)


def kernels(args) -> None:
    """Each library kernel alone at the SiHC-XL shape (batch 256, D=1152, bf16), including
    the stage-API ops the reference's sublayer.py calls (events 16/24, active prefixes up to
    23) and the config-3 gather/scatter (batch 128). GB/s = algorithmic bytes / mean time."""
    import torch

    from sihc_hip import launch
    from sihc_hip.indexed import group_index

    dev = torch.device("cuda", 0)
    bf = torch.bfloat16
    B, C, S = args.batch, args.channels, args.slots
    edge = 32 if S == 4 else 64
    g = torch.Generator(device=dev).manual_seed(args.seed)
    r = lambda shape, m=0.0, sd=1.0: (m + sd * torch.randn(shape, device=dev, generator=g)).to(bf)  # noqa: E731
    x = r((B, edge, edge, C))
    ws = [r((B, 256, C)) for _ in range(25)]
    alpha = r((24, C, S), 1.0 / S, 0.02)
    beta = r((24, C, S), 1.0, 0.02)
    gamma = (0.05 * torch.randn(24, C, device=dev, generator=g))
    U = B * 256 * C * ELEM

    def timed(fn, iters=10):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(iters):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / iters * 1e-3

    cases = []
    for e in (1, 16, 24):
        cases.append((f"read E={e}", (S + e) * U, lambda e=e: launch.read(x, alpha[:e])))
    for e in (1, 16, 24):
        cases.append((f"write E={e}", (2 * S + e) * U, lambda e=e: launch.write(x, ws[:e], beta[:e])))
    cases.append(("write_impl (add_x=False) E=24", (S + 24) * U, lambda: launch.write(x, ws[:24], alpha, add_x=False)))
    for e in (16, 24):
        cases.append((f"weight_grad E={e}", (S + e) * U, lambda e=e: launch.weight_grad(x, ws[:e], beta[:e])))
    for a in (1, 12, 23):
        cases.append((f"triangular A={a}", (a + 2) * U, lambda a=a: launch.triangular(ws[24], ws[:a], gamma[:a])))
    for a in (12, 23):
        cases.append((f"triangular_gamma_grad A={a}", (a + 1) * U,
                      lambda a=a: launch.triangular_gamma_grad(ws[24], ws[:a], gamma[:a])))
    for a in (1, 11, 23):
        cases.append((f"triangular_backward A={a}", (2 * a + 1) * U,
                      lambda a=a: launch.triangular_backward(ws[24], ws[:a], gamma[:a])))
    cases.append(("event_forward", (2 * S + 2) * U, lambda: launch.event_forward(x, ws[0], beta[0], alpha[1])))
    h = r((B, edge, edge, C), 0.0, 1e-2)
    cases.append(("event_backward", (3 * S + 3) * U,
                  lambda: launch.event_backward(h, ws[1], x, ws[0], beta[0], alpha[1])))
    xb = x[: B // 2].contiguous()
    idx = group_index(B // 2, 16, 5, seed=3).to(dev)
    cells = launch.gather_cells(xb, idx, S)
    cases.append(("gather_cells (config 3)", 2 * S * U // 2, lambda: launch.gather_cells(xb, idx, S)))
    cases.append(("scatter_cells (config 3)", 2 * S * U // 2, lambda: launch.scatter_cells(cells, idx)))
    # Reference point of each op: the one-shot calibration stream over the op's own arrays
    # (sihc_stream_mix: carrier-shaped sources, workspace-shaped sources, carrier-shaped
    # destinations, workspace-shaped destinations), the same bytes as the op moves.
    mixes = {"event_forward": (1, 1, 1, 1), "event_backward": (2, 2, 1, 1),
             "write_impl (add_x=False) E=24": (0, 24, 1, 0),
             "gather_cells (config 3)": (1, 0, 1, 0), "scatter_cells (config 3)": (1, 0, 1, 0)}
    for e in (1, 16, 24):
        mixes[f"read E={e}"] = (1, 0, 0, e)
        mixes[f"write E={e}"] = (1, e, 1, 0)
        mixes[f"weight_grad E={e}"] = (1, e, 0, 0)
    for a in (1, 11, 12, 23):
        mixes[f"triangular A={a}"] = (0, a + 1, 0, 1)
        mixes[f"triangular_gamma_grad A={a}"] = (0, a + 1, 0, 0)
        mixes[f"triangular_backward A={a}"] = (0, a + 1, 0, a)
    from sihc_hip import _lib

    Lk = _lib.lib()
    stv = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    car_src = [torch.empty(S * U, dtype=torch.uint8, device=dev) for _ in range(2)]
    car_dst = torch.empty(S * U, dtype=torch.uint8, device=dev)
    ws_dst = [torch.empty(U, dtype=torch.uint8, device=dev) for _ in range(24)]
    sink = torch.empty(U // 64, dtype=torch.uint8, device=dev)
    arr = lambda ts: (ctypes.c_void_p * max(1, len(ts)))(*[t.data_ptr() for t in ts])  # noqa: E731

    def stream_of(name):
        ncs, nws, ncd, nwd = mixes[name]
        half = name.endswith("(config 3)")  # gather / scatter run at half the batch
        srcs = arr(car_src[:ncs] + ws[:nws])
        dsts = arr(([car_dst] if ncd else []) + ws_dst[:nwd])
        nb = U // 2 if half else U
        return lambda: _lib.check(Lk.sihc_stream_mix(srcs, ncs + nws, ncs, dsts, ncd + nwd, ncd, S, nb,
                                                     ctypes.c_void_p(sink.data_ptr()), stv))

    for name, nbytes, fn in cases:
        t = timed(fn)
        row = {"kernel": name, "us": round(t * 1e6, 1), "bytes": nbytes,
               "GB/s": round(nbytes / t / 1e9, 1), "frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)}
        if name in mixes:
            ts = timed(stream_of(name))
            row["stream_us"] = round(ts * 1e6, 1)
            row["of_stream"] = round(ts / t, 4)
        print(json.dumps(row),
              flush=True)


def e2e_config4(seed: int, schedules=("stage", "literal"), steps: int = 5) -> dict:
    """benchmark config 4: SiHC-XL sublayer denoiser (p8, D=1152, 28 blocks, 16 heads,
    MLP ratio 4, stages 8/12/8), bf16, random init; one forward of 64 class-conditional
    + 64 unconditional (label 1000) samples from N(0,1) images, t ~ U(0,1). Routing on
    the HIP ops; bodies on PyTorch-ROCm. Reports samples/s, images/s per CFG step and
    the share of the forward spent in routing (HIP events around each routing call)."""
    import torch

    from sihc_hip.e2e import SiHCDenoiser

    dev = torch.device("cuda", 0)
    torch.manual_seed(seed)
    model = SiHCDenoiser().random_init(seed=seed).to(dev, torch.bfloat16).eval()
    x = torch.randn(128, 3, 256, 256, device=dev).to(torch.bfloat16)
    t = torch.rand(128, device=dev)
    y = torch.cat([torch.randint(0, 1000, (64,), device=dev), torch.full((64,), 1000, device=dev)])
    out = {"workload": "benchmark config 4: SiHC-XL sublayer denoiser forward, CFG batch 64+64, bf16, random init"}
    for schedule in schedules:
        model.schedule = schedule
        with torch.no_grad():
            for _ in range(2):
                model(x, t, y)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                y_hat = model(x, t, y)
            torch.cuda.synchronize()
            fwd = (time.perf_counter() - t0) / steps
            model.routing_timer = []
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            model(x, t, y)
            b.record()
            torch.cuda.synchronize()
            routing = sum(s.elapsed_time(e) for s, e in model.routing_timer) * 1e-3
            total = a.elapsed_time(b) * 1e-3
            model.routing_timer = None
        assert torch.isfinite(y_hat.float()).all(), "non-finite output"
        out[schedule] = {"forward_ms": round(fwd * 1e3, 3), "samples_per_s": round(128 / fwd, 1),
                         "images_per_s_per_cfg_step": round(64 / fwd, 1), "routing_ms": round(routing * 1e3, 3),
                         "routing_share": round(routing / total, 4)}
    return out


# ---- model-level benchmark (the reference's sihc/bench/fusion_profile.py matrix)
# Presets of sihc/presets.py:9-23: (depth, hidden, heads, stage sizes, in-context start);
# every preset is patch 4 (16-slot cells) with 32 in-context prefix tokens.
MODEL_PRESETS = {
    "B": (12, 768, 12, (12,), 4),
    "L": (24, 1024, 16, (12, 12), 8),
    "XL": (40, 1024, 16, (8, 8, 8, 8, 8), 8),
    "H": (32, 1280, 16, (8, 12, 12), 8),
}


def _torch_controls():
    """The reference's PyTorch routing controls (sihc/bench/fusion_controls.py:14-38),
    run on the GPU as the unfused baselines of the model benchmark: NHWC reshapes,
    fp32 products, one cast. Benchmark controls only; the library never calls them."""

    def read(x, alpha_cs):
        b, h, _, c = x.shape
        k = int(round(alpha_cs.shape[1] ** 0.5))
        g = h // k
        cells = x.reshape(b, g, k, g, k, c)
        w = alpha_cs.T.reshape(1, 1, k, 1, k, c)
        return (cells.float() * w.float()).sum((2, 4)).reshape(b, g * g, c).to(x.dtype)

    def write(x, updates, betas):
        b, h, _, c = x.shape
        k = int(round(betas[0].shape[1] ** 0.5))
        g = h // k
        value = x.reshape(b, g, k, g, k, c).float()
        for dz, beta in zip(updates, betas):
            value = value + dz.reshape(b, g, 1, g, 1, c).float() * beta.T.reshape(1, 1, k, 1, k, c).float()
        return value.reshape_as(x).to(x.dtype)

    def triangular(base, updates, gamma):
        value = base.float()
        for j, dz in enumerate(updates):
            value = value + dz.float() * gamma[j].float()
        return value.to(base.dtype)

    return read, write, triangular


def model_step(size: str, implementation: str, phase: str, batch: int, steps: int, warmup: int,
               graph: bool, seed: int, compile_model: bool = False) -> dict:
    """One fusion_profile cell on this GPU: the compact SiHC sublayer denoiser of
    sihc_hip.e2e at a reference preset, FP32 parameters under BF16 autocast, batch
    `batch`. train: forward, loss, backward, fused AdamW (lr 2e-4, betas 0.9/0.95) and
    two FP32 EMAs; inference: one forward (HIP-graph captured with `graph`). Routing:
    fused = HIP stage API (reference "fused"), event = HIP per-event schedule,
    factored / literal = the PyTorch controls (reference "factored" / "literal").
    Bodies run eager unless `compile_model`: then the whole model is compiled as in
    fusion_profile.py:103 (train mode="default", inference mode="reduce-overhead",
    dynamic=False; the reference's single-rank DDP wrapper is not reproduced) and the
    inference step is not captured into a HIP graph by hand."""
    import torch

    from sihc_hip.e2e import SiHCDenoiser

    depth, hidden, heads, stages, ctx_start = MODEL_PRESETS[size]
    schedule = "stage" if implementation in ("fused", "factored") else "literal"
    dev = torch.device("cuda", 0)
    torch.manual_seed(seed)
    torch.cuda.reset_peak_memory_stats()
    model = SiHCDenoiser(hidden=hidden, depth=depth, heads=heads, patch=4, stages=stages, schedule=schedule,
                         in_context_len=32, in_context_start=ctx_start).random_init(seed=seed).to(dev)
    if implementation in ("factored", "literal"):
        read, write, tri = _torch_controls()
        model.read = lambda x, alpha: [read(x, a) for a in alpha.unbind(0)]
        model.triangular = tri
        model.write = lambda x, ups, beta: write(x, ups, list(beta.unbind(0)))
        model.event = lambda x, dz, b, a: (lambda xo: (xo, read(xo, a)))(write(x, [dz], [b]))
    g = torch.Generator(device=dev).manual_seed(seed + 1)
    x = torch.randn(batch, 3, 256, 256, device=dev, generator=g)
    t = torch.full((batch,), 0.5, device=dev)
    y = torch.arange(batch, device=dev) % 1000
    out = {"size": size, "implementation": implementation, "phase": phase, "batch": batch,
           "params": sum(p.numel() for p in model.parameters()), "compiled": compile_model}
    runner = model
    if compile_model:
        import torch._inductor.config as inductor_config

        torch._dynamo.config.cache_size_limit = 128
        inductor_config.compile_threads = min(8, inductor_config.compile_threads)  # bounded worker pool
        runner = torch.compile(model, mode="default" if phase == "train" else "reduce-overhead", dynamic=False)
        graph = False
    if phase == "train":
        model.train()
        target = torch.randn(batch, 3, 256, 256, device=dev, generator=g)
        params = [p for p in model.parameters() if p.requires_grad]
        opt = torch.optim.AdamW(params, lr=2e-4, betas=(0.9, 0.95), weight_decay=0, fused=True)
        emas = [[p.detach().clone() for p in params] for _ in range(2)]

        def run(first=False):
            opt.zero_grad(set_to_none=True)
            tc = time.perf_counter()
            with torch.autocast("cuda", dtype=torch.bfloat16):
                loss = (runner(x, t, y).float() - target).square().flatten(1).mean(1).mean()
            if first:
                torch.cuda.synchronize()
                print(f"[bench] {size} {implementation} train: first forward {time.perf_counter() - tc:.1f} s",
                      file=sys.stderr, flush=True)
            loss.backward()
            opt.step()
            with torch.no_grad():
                for copies, decay in zip(emas, (0.9999, 0.9996)):
                    torch._foreach_mul_(copies, decay)
                    torch._foreach_add_(copies, params, alpha=1 - decay)
            return loss
    else:
        model.eval().requires_grad_(False)
        if graph:
            static = [x.clone(), t.clone(), y.clone()]
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            # autocast's weight-cast cache off: the casts are recorded into the graph
            amp = dict(device_type="cuda", dtype=torch.bfloat16, cache_enabled=False)
            with torch.inference_mode(), torch.cuda.stream(side), torch.autocast(**amp):
                for _ in range(2):
                    model(*static)
            torch.cuda.current_stream().wait_stream(side)
            hg = torch.cuda.CUDAGraph()
            with torch.inference_mode(), torch.cuda.graph(hg), torch.autocast(**amp):
                result = model(*static)

            def run():
                hg.replay()
                return result
        else:
            def run():
                if compile_model:
                    torch.compiler.cudagraph_mark_step_begin()
                with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
                    return runner(x, t, y)
    last = None
    tc = time.perf_counter()
    for i in range(warmup):
        last = run(first=True) if i == 0 and phase == "train" and compile_model else run()
        if i == 0 and compile_model:
            torch.cuda.synchronize()
            print(f"[bench] {size} {implementation} {phase}: first (compiling) step {time.perf_counter() - tc:.1f} s",
                  file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        last = run()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    finite = bool(torch.isfinite(last.float()).all())
    out.update({"ms_per_step": round(dt * 1e3, 2), "images_per_s": round(batch / dt, 1),
                "peak_allocated_gib": round(torch.cuda.max_memory_allocated() / 2**30, 2), "finite": finite,
                "hip_graph": bool(graph and phase == "inference")})
    return out


def model_bench(args) -> None:
    if args.tri_backward:
        from sihc_hip import sublayer_kernels

        sublayer_kernels.COMPILED_TRIANGULAR_BACKWARD = args.tri_backward
    for size in args.size.split(","):
        for phase in args.phase.split(","):
            for impl in args.implementation.split(","):
                import torch
                try:
                    r = model_step(size, impl, phase, args.model_batch, args.steps, args.warmup,
                                   not args.no_graph, args.seed, args.compile)
                    if args.compile and args.tri_backward:
                        r["tri_backward"] = args.tri_backward
                except torch.OutOfMemoryError:
                    r = {"size": size, "implementation": impl, "phase": phase, "status": "oom"}
                print(json.dumps(r), flush=True)
                torch.cuda.empty_cache()


def e2e(args) -> None:
    print(json.dumps(e2e_config4(args.seed, (args.schedule,), max(1, min(args.steps, 10)))), flush=True)


def main():
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this build runs no "
              "multi-GPU path: the read/write path shards along batch with no collective.", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (MI355X); none is visible", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    if args.mode == "calibrate":
        calibrate(args)
        return
    if args.mode == "kernels":
        kernels(args)
        return
    if args.mode == "e2e":
        e2e(args)
        return
    if args.mode == "model":
        model_bench(args)
        return
    if args.mode == "stage":
        print(json.dumps(stage_api_config2(args.seed, max(1, args.steps), args.compile)), flush=True)
        return
    if args.mode == "ceiling":
        print(json.dumps(stream_ceiling()), flush=True)
        return
    if args.mode == "valu":
        valu_rate()
        return
    print(f"[bench] building step: batch={args.batch} C={args.channels} events={args.events}", file=sys.stderr,
          flush=True)
    step = LiteralStep(args.batch, args.channels, args.events, args.seed)
    step.use_chain(args.finalize == "chain")
    m = measure_step(torch, step, args.steps, args.warmup)
    ms_step, marked_ms, fwd_ms, bwd_ms = m["ms_step"], m["marked_ms"], m["fwd_ms"], m["bwd_ms"]
    avg_kernel_ms, avg_fwd_kernel_ms, n_bwd_launches = m["bwd_kernel_ms"], m["fwd_kernel_ms"], m["bwd_launches"]
    print(f"[bench] timed {args.steps} steps: {ms_step:.3f} ms/step", file=sys.stderr, flush=True)

    total_bytes = step.bytes_fwd + step.bytes_bwd
    gbs = total_bytes / (ms_step * 1e-3) / 1e9
    dom_bytes = next(c[3] for c in step.bwd if c[0] == "event_backward")
    achieved = dom_bytes / (avg_kernel_ms * 1e-3) / 1e9
    fwd_bytes = next(c[3] for c in step.fwd if c[0] == "event_forward")
    fwd_rate = fwd_bytes / (avg_fwd_kernel_ms * 1e-3) / 1e9
    traffic = traffic_from_profiles()
    result = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "benchmark config 2: SiHC-XL-shape fused read/write fwd+bwd, literal per-event schedule",
            "batch": args.batch, "tokens": 256, "slots": 4, "channels": args.channels,
            "events": args.events, "schedule": "per-event fused (write+read, one carrier pass per event)",
            "parallelism": "single GPU",
            "finalize": {"chain": "each backward launch finalizes the previous event's weight gradients in its "
                                  "trailing blocks (sihc_event_backward_chain)",
                         "deferred": "one deferred finalize launch per 32 events after the last event"}[args.finalize],
        },
        "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
        "tokens_per_s": round(args.batch * 256 / (ms_step * 1e-3), 1),
        "fwd_kernel_GBps": round(fwd_rate, 1),
        "fwd_kernel_avg_ms": round(avg_fwd_kernel_ms, 4),
        "fwd_ms": round(fwd_ms, 3),
        "bwd_ms": round(bwd_ms, 3),
        "marked_step_ms": round(marked_ms, 3),
        "algorithmic_bytes_per_step": total_bytes,
        "roofline": {
            "kernel": ("k_event_bwd (sihc_event_backward_chain, full event, with the previous event's "
                       "weight-gradient finalize in its trailing blocks)") if args.finalize == "chain" else
                      ("k_event_bwd (sihc_event_backward_partial, full event; the step's deferred finalize of "
                       "all events is outside the launch)"),
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": ("committed profiles/event_backward_traffic.json: rocprofv3 FETCH_SIZE + WRITE_SIZE "
                               "of bench.py --mode calibrate, scaled by the same counters on the library's copy "
                               "of 1 GiB; not measured in this run") if traffic is not None else None,
            "bytes_per_launch": dom_bytes,
            "avg_launch_ms": round(avg_kernel_ms, 4),
            "launches": n_bwd_launches,
        },
    }
    if not args.no_extra:
        del step
        torch.cuda.empty_cache()
        print("[bench] secondary configs 1 and 3", file=sys.stderr, flush=True)
        result["extra"] = extra_configs(args.seed)
        print("[bench] config 2 on the stage API (drop-in path), eager and compiled", file=sys.stderr, flush=True)
        result["extra"]["config2_stage_api"] = stage_api_config2(args.seed)
        try:
            result["extra"]["config2_stage_api_compiled"] = stage_api_config2(args.seed, compiled=True)
        except Exception as exc:  # the headline line must not depend on the compiler
            result["extra"]["config2_stage_api_compiled"] = {"error": f"{type(exc).__name__}: {exc}"[:300]}
        result["extra"]["stream_ceiling"] = ceiling = stream_ceiling()
        fw_rate = result["fwd_kernel_GBps"]
        result["extra"]["fraction_of_stream_ceiling"] = {
            "k_event_fwd_rows vs the per-event forward's arrays":
                round(fw_rate / ceiling["per-event forward's arrays (1:1, 10 units)"]["GB/s"], 4),
            "k_event_bwd vs the per-event backward's arrays":
                round(achieved / ceiling["per-event backward's arrays (2:1, 15 units)"]["GB/s"], 4)}
        torch.cuda.empty_cache()
        print("[bench] config 4 end-to-end forward", file=sys.stderr, flush=True)
        result["extra"]["config4_e2e"] = e2e_config4(args.seed)
    if not args.no_cpu_baseline:
        print("[bench] CPU baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
