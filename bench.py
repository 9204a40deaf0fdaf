"""Throughput of the isotonic hot path on one MI355X, against the HBM roofline, with the
reference CPU solver timed beside it.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]

Prints ONE JSON line. The headline ``value`` is BASELINE config C2: a forward
``torchisotonic_amd.isotonic`` of float32 y[1e6, 16] = -0.1 i + N(0, 1), unweighted,
decreasing, inputs resident in HBM, K back-to-back calls of the public API between device
synchronisations (Gelem/s = 1.6e7 K / seconds). ``extra`` holds the metric's other legs:
C2 forward+backward (dy), and C4 (one row of 1e8, weighted) forward and forward+backward when
the long-row path is built.

``roofline`` is for the dominant kernel of the headline step, timed live with HIP events
recorded on the launch stream around each launch (raw C-ABI calls on preallocated buffers):
achieved = algorithmic bytes per launch / mean kernel time; peak = 8 TB/s. ``traffic`` is null
unless --traffic-factor data from rocprofv3 PMC runs is supplied.

``cpu_baseline`` times the reference's own pava.h (compiled from the reference checkout into
oracle/_ref/libti_ref.so; kind "reference") or, if that library is absent, the C restatement
(kind "port") on the host's cores over a bounded sample of C2 rows.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import torchisotonic_amd  # noqa: E402
from torchisotonic_amd import _ext  # noqa: E402

PEAK_GBPS = 8000.0
METRIC = "Gelem/s fwd & fwd+bwd, % HBM roofline; 1e6×16 and 1×1e8 f32"


def log(*a: object) -> None:
    print(*a, file=sys.stderr, flush=True)


def c2_inputs(device: str) -> tuple[torch.Tensor, torch.Tensor]:
    rng = np.random.default_rng(0)
    b, n = 1_000_000, 16
    y = (-0.1 * np.arange(n) + rng.standard_normal((b, n))).astype(np.float32)
    g = np.random.default_rng(1).standard_normal((b, n)).astype(np.float32)
    return torch.from_numpy(y).to(device), torch.from_numpy(g).to(device)


def timed_calls(fn, steps: int, warmup: int) -> float:
    """Seconds per call over `steps` back-to-back calls, bracketed by synchronisations."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def kernel_ms(launch, reps: int) -> float:
    """Mean device time of one launch: HIP events recorded on the launch stream right before
    and after each raw launch."""
    stream = torch.cuda.current_stream()
    pairs = []
    for _ in range(reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        launch()
        e1.record(stream)
        pairs.append((e0, e1))
    torch.cuda.synchronize()
    return float(np.mean([a.elapsed_time(b) for a, b in pairs]))


def warm_gpu() -> None:
    # An idle GPU clocks down; keep it busy briefly first (the reference's method,
    # bench/bench.py:51-55).
    x = torch.empty(1 << 26, device="cuda")
    for _ in range(20):
        x.mul_(1.0)
    torch.cuda.synchronize()


def bench_c2(steps: int, warmup: int) -> dict:
    y, g = c2_inputs("cuda")
    b, n = y.shape
    elems = b * n
    # forward through the public API
    fwd = lambda: torchisotonic_amd.isotonic(y, increasing=False)  # noqa: E731
    t_fwd = timed_calls(fwd, steps, warmup)
    # forward + backward (dy) through the public API
    yr = y.clone().requires_grad_()

    def fwd_bwd() -> None:
        out = torchisotonic_amd.isotonic(yr, increasing=False)
        torch.autograd.grad(out, (yr,), g)

    t_fb = timed_calls(fwd_bwd, steps, warmup)
    # the raw kernels, for the roofline
    lib = _ext.load()
    out = torch.empty_like(y)
    starts = torch.empty(_ext.starts_words(b, n), dtype=torch.int32, device="cuda")
    gy = torch.empty_like(y)
    stream = torch.cuda.current_stream().cuda_stream

    def launch_fwd() -> None:
        lib.ti_fwd(y.data_ptr(), None, out.data_ptr(), None, None, b, n, _ext.F32, 0, 0.0, 0.0, None, 0, stream)

    def launch_fwd_starts() -> None:
        lib.ti_fwd(y.data_ptr(), None, out.data_ptr(), starts.data_ptr(), None, b, n, _ext.F32, 0, 0.0, 0.0, None, 0, stream)

    def launch_bwd() -> None:
        lib.ti_bwd(starts.data_ptr(), g.data_ptr(), None, None, gy.data_ptr(), None, b, n, _ext.F32, 1, 0.0, 0.0, None, 0, stream)

    for f in (launch_fwd, launch_fwd_starts, launch_bwd):
        f()
    torch.cuda.synchronize()
    k_fwd = kernel_ms(launch_fwd, 50)
    k_fwd_s = kernel_ms(launch_fwd_starts, 50)
    k_bwd = kernel_ms(launch_bwd, 50)
    return {
        "elems": elems,
        "t_fwd": t_fwd,
        "t_fb": t_fb,
        "k_fwd_ms": k_fwd,
        "k_fwd_starts_ms": k_fwd_s,
        "k_bwd_ms": k_bwd,
    }


def cpu_baseline(budget_s: float = 12.0) -> dict:
    import oracle

    rng = np.random.default_rng(0)
    b, n = 1_000_000, 16
    y = (-0.1 * np.arange(n) + rng.standard_normal((b, n))).astype(np.float32)
    threads = min(16, os.cpu_count() or 1)
    kind = "reference" if oracle.ref_lib() is not None else "port"
    impl = "reference" if kind == "reference" else "oracle"
    oracle.pava(y[:1000], None, increasing=False, threads=threads, impl=impl, with_starts=False)
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        oracle.pava(y, None, increasing=False, threads=threads, impl=impl, with_starts=False)
        times.append(time.perf_counter() - t0)
        if len(times) >= 200:
            break
    med = float(np.median(times))
    return {
        "value": b * n / med / 1e9,
        "unit": "Gelem/s",
        "cores": threads,
        "kind": kind,
        "sample": f"C2 [1e6,16] f32 decreasing unweighted, forward, median of {len(times)} calls "
        f"({sum(times):.1f} s), rows over {threads} OpenMP threads",
    }


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(
            "bench.py measures one GPU: rows are independent and this build runs on a single "
            "MI355X; multi-GPU sharding is design-only (see DESIGN.md). Run with --gpus 1.",
            file=sys.stderr,
        )
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    warm_gpu()
    c2 = bench_c2(args.steps, args.warmup)
    elems = c2["elems"]
    fwd_gelem = elems / c2["t_fwd"] / 1e9
    fb_gelem = elems / c2["t_fb"] / 1e9
    bytes_fwd = 8 * elems  # y in, fit out (f32)
    achieved = bytes_fwd / (c2["k_fwd_ms"] * 1e-3) / 1e9
    extra = {
        "c2_fwd_gelem_s": fwd_gelem,
        "c2_fwd_bwd_gelem_s": fb_gelem,
        "c2_fwd_ms": c2["t_fwd"] * 1e3,
        "c2_fwd_bwd_ms": c2["t_fb"] * 1e3,
        "c2_fwd_pct_roofline": 100 * 8 * elems / c2["t_fwd"] / 1e9 / PEAK_GBPS,
        "c2_fwd_bwd_pct_roofline": 100 * 16 * elems / c2["t_fb"] / 1e9 / PEAK_GBPS,
        "kernel_ms": {
            "short_fit (no starts)": c2["k_fwd_ms"],
            "short_fit (with starts)": c2["k_fwd_starts_ms"],
            "short_grad (dy)": c2["k_bwd_ms"],
        },
    }
    line = {
        "metric": METRIC,
        "value": fwd_gelem,
        "unit": "Gelem/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": c2["t_fwd"] * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (f64 sums and hull tests)",
        "data": "synthetic: y[b,i] = -0.1 i + N(0,1), seed 0",
        "config": {
            "workload": "C2: isotonic forward, y f32 [1000000, 16], unweighted, increasing=False",
            "batch": 1_000_000,
            "n": 16,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": PEAK_GBPS,
            "unit": "GB/s",
            "frac": achieved / PEAK_GBPS,
            "traffic": None,
            "kernel": "short_fit_kernel<float,16,false>",
            "algorithmic_bytes_per_launch": bytes_fwd,
        },
        "extra": extra,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
