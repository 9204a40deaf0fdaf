"""Throughput of the isotonic hot path on one MI355X, against the HBM roofline, with the
reference CPU solver timed beside it.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs c2,c4,c5,c1,c3,next,hull[,grid]] [--no-cpu]

Prints ONE JSON line. The headline ``value`` is BASELINE config C2: a forward
``torchisotonic_amd.isotonic`` of float32 y[1e6, 16] = -0.1 i + N(0, 1), unweighted,
decreasing, inputs resident in HBM, K back-to-back calls of the public API between device
synchronisations (Gelem/s = 1.6e7 K / seconds). ``extra`` holds the metric's other legs - C2
forward+backward (dy), C4 (one row of 1e8, weighted 0/1 labels, integer counts) forward and
forward+backward (dy, dw) - the other BASELINE configs (C5 bootstrap, C1, C3), and the rows
either side of the path (``next``: C2's rows at their own lengths with offsets, soft ranks,
calibration), and hull-heavy rows (``hull``: one row of 1e8 rising with noise). With
``--configs ...,grid`` (not in the default run) ``extra.grid`` also times the reference's own
README table: its (batch, n) grid and data, each call synchronised, median and best of ten.

Bytes per element (algorithmic, float32, each API tensor moved once): forward 8 unweighted
(y in, fit out), 12 weighted (+w); backward 8 for dy alone (g in, gy out), 24 for dy and dw
(g, w, y, fit in; gy, gw out). ``%roofline`` = bytes * Gelem/s / 8000 GB/s.

``roofline`` is for the dominant kernel of the headline step, timed live with one HIP event
pair on the launch stream around K back-to-back raw C-ABI launches on preallocated buffers:
achieved = algorithmic bytes per launch / (interval / K); peak = 8 TB/s. ``copy_ceiling`` is a
128 MB device copy timed the same way in the same run. ``traffic`` is that kernel's
HBM bytes per launch from the rocprofv3 FETCH_SIZE and WRITE_SIZE passes summarised in
profiles/short_rows_kernel_c2_traffic.json (each counter scaled by what it reads for a copy-like
kernel of known size), or null where that summary is absent.

``cpu_baseline`` times the reference's own pava.h (compiled from the reference checkout into
oracle/_ref/libti_ref.so; kind "reference") or, if that library is absent, the C restatement
(kind "port") on the host's cores over C2's rows.
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


def sync() -> None:
    torch.cuda.synchronize()


SLEEP_CYCLES = 100_000  # torch.cuda._sleep: about 40 us at this part's shader clock (longer spins let it clock down)


def timed_calls(fn, steps: int, warmup: int) -> float:
    """Seconds per call over exactly `steps` back-to-back calls, bracketed by synchronisations:
    after a short clock-raising load and `warmup` untimed calls, a spin kernel that touches no
    memory (torch.cuda._sleep, about 40 us) holds the stream while the host queues the calls,
    and one HIP event pair on the stream around them times them on the GPU. The window holds
    the calls and every gap between them (a host slower than the GPU shows as idle time in it),
    but not the first launch's latency nor the final synchronisation's, which a wall clock
    around 20 calls of 30 us spreads over them as a few per cent (wall_calls)."""
    warm_gpu(0.05)
    for _ in range(warmup):
        fn()
    sync()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(SLEEP_CYCLES)
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    sync()
    return e0.elapsed_time(e1) * 1e-3 / steps


def wall_calls(fn, steps: int, warmup: int) -> float:
    """Seconds per call by the host's clock over `steps` back-to-back calls between two
    synchronisations: the GPU time plus the first launch's and the last synchronisation's
    latency, divided by `steps`."""
    warm_gpu(0.05)
    for _ in range(warmup):
        fn()
    sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    sync()
    return (time.perf_counter() - t0) / steps


def kernel_ms(launch, reps: int, repeats: int = 3) -> float:
    """Device time of `launch` per launch: one HIP event pair recorded on the launch stream
    around `reps` back-to-back launches, divided by reps; the best of `repeats` such intervals,
    each after a short clock-raising load. The launches queue behind a spin kernel that touches
    no memory, so the GPU never waits for the host between them, no earlier kernel's write-back
    is timed, and the interval holds kernel time only (an event pair per launch would add its
    own overhead to every interval)."""
    stream = torch.cuda.current_stream()
    best = float("inf")
    launch()  # (first-call set-up outside the intervals)
    for _ in range(repeats):
        warm_gpu(0.03)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(SLEEP_CYCLES)
        e0.record(stream)
        for _ in range(reps):
            launch()
        e1.record(stream)
        sync()
        best = min(best, e0.elapsed_time(e1) / reps)
    return best


def copy_ceiling(mbytes: int = 128, reps: int = 50) -> dict:
    """A device-to-device copy of `mbytes` MB (half read, half written) timed like the kernels:
    the bandwidth a plain streaming kernel reaches on this box."""
    half = mbytes * 1_000_000 // 2 // 4
    src = torch.empty(half, dtype=torch.float32, device="cuda").normal_()
    dst = torch.empty_like(src)
    ms = kernel_ms(lambda: dst.copy_(src), reps)
    return {"gbps": mbytes * 1e6 / (ms * 1e-3) / 1e9, "bytes": mbytes * 1_000_000, "ms": ms}


_BUSY: torch.Tensor | None = None


def warm_gpu(seconds: float = 0.3) -> None:
    # An idle GPU clocks down; keep it busy first (the reference's method, bench/bench.py:51-55).
    # A few milliseconds are not enough on this part: kernel times keep falling for about a
    # tenth of a second of load (C2's forward kernel 33.5 -> 31.3 us).
    global _BUSY
    if _BUSY is None:
        _BUSY = torch.empty(1 << 26, device="cuda")
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(10):
            _BUSY.mul_(1.0)
        sync()


def rate(elems: int, seconds: float, bytes_per_elem: float) -> dict:
    g = elems / seconds / 1e9
    return {"ms": seconds * 1e3, "gelem_s": g, "pct_roofline": 100 * g * bytes_per_elem / PEAK_GBPS}


def fwd_bwd_fn(y: torch.Tensor, w: torch.Tensor | None, g: torch.Tensor, want_w: bool, **kw):
    yr = y.detach().requires_grad_()
    wr = None if w is None else (w.detach().requires_grad_(want_w))
    inputs = (yr, wr) if (wr is not None and want_w) else (yr,)

    def f() -> None:
        out = torchisotonic_amd.isotonic(yr, wr, **kw)
        torch.autograd.grad(out, inputs, g)

    return f


# --- C2: [1e6, 16] ------------------------------------------------------------------------


def bench_c2(steps: int, warmup: int) -> dict:
    rng = np.random.default_rng(0)
    b, n = 1_000_000, 16
    y = torch.from_numpy((-0.1 * np.arange(n) + rng.standard_normal((b, n))).astype(np.float32)).cuda()
    g = torch.from_numpy(np.random.default_rng(1).standard_normal((b, n)).astype(np.float32)).cuda()
    elems = b * n
    t_fwd = timed_calls(lambda: torchisotonic_amd.isotonic(y, increasing=False), steps, warmup)
    t_fb = timed_calls(fwd_bwd_fn(y, None, g, False, increasing=False), steps, warmup)
    t_fwd_wall = wall_calls(lambda: torchisotonic_amd.isotonic(y, increasing=False), steps, warmup)
    t_fb_wall = wall_calls(fwd_bwd_fn(y, None, g, False, increasing=False), steps, warmup)
    lib = _ext.load()
    out = torch.empty_like(y)
    starts = torch.empty(_ext.starts_words(b, n), dtype=torch.int32, device="cuda")
    gy = torch.empty_like(y)
    s = torch.cuda.current_stream().cuda_stream
    fwd = lambda: lib.ti_fwd(y.data_ptr(), None, out.data_ptr(), None, None, b, n, 0, 0, 0.0, 0.0, None, 0, s)  # noqa: E731
    fwd_s = lambda: lib.ti_fwd(y.data_ptr(), None, out.data_ptr(), starts.data_ptr(), None, b, n, 0, 0, 0.0, 0.0, None, 0, s)  # noqa: E731
    bwd = lambda: lib.ti_bwd(starts.data_ptr(), None, 0, g.data_ptr(), None, None, gy.data_ptr(), None, b, n, 0, 0, 0.0, 0.0, None, 0, s)  # noqa: E731
    for f in (fwd, fwd_s, bwd):
        assert f() == 0
    sync()
    return {
        "elems": elems,
        "fwd": rate(elems, t_fwd, 8),
        "fwd_bwd": rate(elems, t_fb, 16),
        "fwd_wall_clock": rate(elems, t_fwd_wall, 8),
        "fwd_bwd_wall_clock": rate(elems, t_fb_wall, 16),
        "kernel_ms": {
            "short_rows_kernel<float,16,unweighted> (no starts)": kernel_ms(fwd, 100),
            "short_rows_kernel<float,16,unweighted> (with starts)": kernel_ms(fwd_s, 100),
            "short_grad_rows_kernel<float,16,unweighted> (dy)": kernel_ms(bwd, 100),
        },
    }


# --- C4: one row of 1e8, weighted -------------------------------------------------------------


def c4_inputs(n: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    rng = np.random.default_rng(0)
    s = np.sort(rng.standard_normal(n) * 1.5)
    y = (rng.random(n) < 1.0 / (1.0 + np.exp(-s))).astype(np.float32)
    del s
    w = rng.integers(1, 6, n).astype(np.float32)
    g = np.random.default_rng(1).standard_normal(n).astype(np.float32)
    return torch.from_numpy(y).cuda(), torch.from_numpy(w).cuda(), torch.from_numpy(g).cuda()


def bench_c4(steps: int, warmup: int, n: int = 100_000_000) -> dict:
    y, w, g = c4_inputs(n)
    t_fwd = timed_calls(lambda: torchisotonic_amd.isotonic(y, w), steps, warmup)
    t_fb = timed_calls(fwd_bwd_fn(y, w, g, True), steps, warmup)
    t_fb_dy = timed_calls(fwd_bwd_fn(y, w, g, False), steps, warmup)
    # raw forward pipeline on preallocated buffers (no API host work, no weight-flag sync)
    lib = _ext.load()
    yy, ww = y.view(1, n), w.view(1, n)
    out = torch.empty_like(yy)
    ws = _ext._workspace("fwd", 1, n, 0, True, y.device)
    s = torch.cuda.current_stream().cuda_stream
    fwd = lambda: lib.ti_fwd(yy.data_ptr(), ww.data_ptr(), out.data_ptr(), None, None, 1, n, 0, 1, 0.0, 0.0, ws.data_ptr(), ws.numel(), s)  # noqa: E731
    assert fwd() == 0
    sync()
    return {
        "elems": n,
        "fwd": rate(n, t_fwd, 12),
        "fwd_bwd": rate(n, t_fb, 36),
        "fwd_bwd_dy_only": rate(n, t_fb_dy, 24),
        "fwd_pipeline_ms": kernel_ms(fwd, 20),
    }


# --- C5: bootstrap [1000, 65536] ----------------------------------------------------------------


def bench_c5(steps: int, warmup: int) -> dict:
    b, n = 1000, 65536
    rng = np.random.default_rng(0)
    y0 = (rng.random(n) < 1 / (1 + np.exp(-np.linspace(-4, 4, n)))).astype(np.float32)
    y = torch.from_numpy(y0).cuda().expand(b, n).contiguous()
    w = torch.from_numpy(np.maximum(rng.exponential(1.0, (b, n)), 1e-6).astype(np.float32)).cuda()
    g = torch.from_numpy(np.random.default_rng(1).standard_normal((b, n)).astype(np.float32)).cuda()
    t_fwd = timed_calls(lambda: torchisotonic_amd.isotonic(y, w), steps, warmup)
    t_fb = timed_calls(fwd_bwd_fn(y, w, g, True), steps, warmup)
    return {"elems": b * n, "fwd": rate(b * n, t_fwd, 12), "fwd_bwd": rate(b * n, t_fb, 36)}


# --- C1 and C3: [1000, 5000] ----------------------------------------------------------------


def bench_c1_c3(steps: int, warmup: int) -> dict:
    b, n = 1000, 5000
    rng = np.random.default_rng(0)
    y1 = torch.from_numpy((0.001 * np.arange(n) + rng.standard_normal((b, n))).astype(np.float32)).cuda()
    res = {"c1_fwd": rate(b * n, timed_calls(lambda: torchisotonic_amd.isotonic(y1), steps, warmup), 8)}
    base = 1 / (1 + np.exp(-(np.linspace(-4, 4, n) + 0.5 * rng.standard_normal((b, n)))))
    wnp = rng.random((b, n)) + 0.1
    gnp = np.random.default_rng(1).standard_normal((b, n))
    kw = dict(increasing=False, y_min=0.0, y_max=1.0)
    for name, dt in (("f32", np.float32), ("f64", np.float64)):
        y, w, g = (torch.from_numpy(a.astype(dt)).cuda() for a in (base, wnp, gnp))
        bpe = 12 if dt == np.float32 else 24
        res[f"c3_{name}_fwd"] = rate(b * n, timed_calls(lambda: torchisotonic_amd.isotonic(y, w, **kw), steps, warmup), bpe)
        res[f"c3_{name}_fwd_bwd"] = rate(b * n, timed_calls(fwd_bwd_fn(y, w, g, True, **kw), steps, warmup), 3 * bpe)
    return res


# --- the rows either side of the path: ragged rows, soft ranks, calibration -------------------


def bench_hull(steps: int, warmup: int) -> dict:
    """Hull-heavy rows: one float32 row of 1e8 rising with noise, y = i / n + s N(0, 1) (float64,
    rounded once to float32; seed 0), unweighted, increasing, forward through the public API,
    for s = 1e-9 (about 3.8e7 blocks: nearly every point a hull vertex) and 1e-7 (about 1.6e7),
    with the fit's block count. Their upper merge levels have one or two parents each, whose
    survivors survivors_kernel writes."""
    n = 100_000_000
    res: dict = {}
    gen = torch.Generator(device="cuda").manual_seed(0)
    for noise in (1e-9, 1e-7):
        i = torch.arange(n, device="cuda", dtype=torch.float64)
        y = (i / n + noise * torch.randn(n, device="cuda", dtype=torch.float64, generator=gen)).float().view(1, n)
        del i
        fit = torchisotonic_amd.isotonic(y)
        blocks = int(torch.unique_consecutive(fit).numel())
        del fit
        r = rate(n, timed_calls(lambda y=y: torchisotonic_amd.isotonic(y), max(5, min(steps, 10)), 2), 8)
        r["blocks"] = blocks
        res[f"rising_1e8_noise_{noise:g}"] = r
        del y
    return res


def bench_next(steps: int, warmup: int) -> dict:
    """The consumers around the fit, timed like the configs above (back-to-back calls of the
    public API between synchronisations): C2's rows at their own lengths (len ~ U{4..16}, seed 2;
    the padded variant is the C2 forward above), packed with offsets, forward and forward+backward
    (8 and 16 B per element); 1e5 rows of lengths U{1..2000}, packed and padded; soft ranks at the reference's shapes and strengths (reference
    paper/soft_rank.py:23-28; x, g ~ N(0, 1) float32); and calibration (fit over pooled keys,
    then interpolation) of 6.5 million float32 scores, about one day of the reference's Criteo
    example (examples/ctr_calibration/calibrate.py:171-187)."""
    res: dict = {}
    rng = np.random.default_rng(0)
    b, n = 1_000_000, 16
    y = (-0.1 * np.arange(n) + rng.standard_normal((b, n))).astype(np.float32)
    lens = np.random.default_rng(2).integers(4, n + 1, b)
    packed = torch.from_numpy(y[np.arange(n)[None, :] < lens[:, None]]).cuda()
    off = torch.from_numpy(np.r_[0, np.cumsum(lens)]).cuda()
    g = torch.randn_like(packed)
    elems = packed.numel()
    fwd = lambda: torchisotonic_amd.isotonic_ragged(packed, off, increasing=False)  # noqa: E731
    pr = packed.detach().requires_grad_()

    def fb() -> None:
        torch.autograd.grad(torchisotonic_amd.isotonic_ragged(pr, off, increasing=False), pr, g)

    # with the rows' length bound (the padded length, 16) the fit starts before the plan's wait
    fwd16 = lambda: torchisotonic_amd.isotonic_ragged(packed, off, increasing=False, max_len=n)  # noqa: E731

    def fb16() -> None:
        torch.autograd.grad(torchisotonic_amd.isotonic_ragged(pr, off, increasing=False, max_len=n), pr, g)

    lib = _ext.load()
    out = torch.empty_like(packed)
    bits = torch.zeros((elems + 31) // 32, dtype=torch.int32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    raw = lambda: lib.ti_fwd_ragged(packed.data_ptr(), None, out.data_ptr(), None, None, off.data_ptr(), b, elems, n, 0, 0, 0.0, 0.0, s)  # noqa: E731
    assert raw() == 0
    # the backward's kernel, from the bits of a forward that wrote them
    gy = torch.empty_like(packed)
    assert lib.ti_fwd_ragged(packed.data_ptr(), None, out.data_ptr(), bits.data_ptr(), None, off.data_ptr(), b, elems, n, _ext.F32, 0, 0.0, 0.0, s) == 0
    rawb = lambda: lib.ti_bwd_ragged(bits.data_ptr(), g.data_ptr(), None, None, gy.data_ptr(), None, off.data_ptr(), b, elems, n, _ext.F32, 0, 0.0, 0.0, s)  # noqa: E731
    assert rawb() == 0
    plan = torch.zeros(_ext.RAGGED_PLAN_WORDS, dtype=torch.int64, device="cuda")  # (plans fold into it: a timing)
    keys = torch.empty(b, dtype=torch.uint8, device="cuda")
    rawp = lambda: lib.ti_ragged_plan(off.data_ptr(), b, elems, plan.data_ptr(), keys.data_ptr(), s)  # noqa: E731
    assert rawp() == 0
    res["c2_ragged"] = {
        "elems": elems,
        "fwd": rate(elems, timed_calls(fwd, steps, warmup), 8),
        "fwd_bwd": rate(elems, timed_calls(fb, steps, warmup), 16),
        "fwd_max_len": rate(elems, timed_calls(fwd16, steps, warmup), 8),
        "fwd_bwd_max_len": rate(elems, timed_calls(fb16, steps, warmup), 16),
        "kernel_ms": {
            "ragged_fit_kernel<float,16,unweighted> (no starts)": kernel_ms(raw, 100),
            "ragged_grad_kernel<float,16,unweighted> (dy)": kernel_ms(rawb, 100),
            "ragged_plan_kernel": kernel_ms(rawp, 100),
        },
    }
    del bits, gy
    # 1e5 rows of lengths U{1..2000} (seed 31; about 1e8 elements), increasing, float32, packed
    # with offsets, against the same rows padded to 2000 elements (each beyond its own maximum,
    # the reference's padding rule) and fitted dense; rates in the rows' own elements
    rb, rl = 100_000, 2000
    lens2 = torch.from_numpy(np.random.default_rng(31).integers(1, rl + 1, rb)).cuda()
    off2 = torch.zeros(rb + 1, dtype=torch.int64, device="cuda")
    off2[1:] = torch.cumsum(lens2, 0)
    tot2 = int(off2[-1])
    rowid = torch.repeat_interleave(torch.arange(rb, device="cuda"), lens2)
    col = torch.arange(tot2, device="cuda") - off2[:-1][rowid]
    gen = torch.Generator(device="cuda").manual_seed(31)
    packed2 = 0.001 * col.float() + torch.randn(tot2, device="cuda", generator=gen)
    g2 = torch.randn(tot2, device="cuda", generator=gen)
    rmax = torch.full((rb,), -float("inf"), device="cuda").scatter_reduce(0, rowid, packed2, "amax")
    padded = (rmax + 1.0)[:, None].expand(rb, rl).contiguous()
    padded[rowid, col] = packed2
    gpad = torch.zeros(rb, rl, device="cuda")
    gpad[rowid, col] = g2
    del rowid, col, rmax
    pr2 = packed2.detach().requires_grad_()
    pp2 = padded.detach().requires_grad_()
    k2 = max(3, min(steps, 10))

    def rfb() -> None:
        torch.autograd.grad(torchisotonic_amd.isotonic_ragged(pr2, off2), pr2, g2)

    def pfb() -> None:
        torch.autograd.grad(torchisotonic_amd.isotonic(pp2), pp2, gpad)

    res["ragged_long"] = {
        "rows": rb,
        "elems": tot2,
        "padded_elems": rb * rl,
        "fwd": rate(tot2, timed_calls(lambda: torchisotonic_amd.isotonic_ragged(packed2, off2), k2, 2), 8),
        "fwd_bwd": rate(tot2, timed_calls(rfb, k2, 2), 16),
        "padded_fwd": rate(tot2, timed_calls(lambda: torchisotonic_amd.isotonic(padded), k2, 2), 8),
        "padded_fwd_bwd": rate(tot2, timed_calls(pfb, k2, 2), 16),
    }
    del packed2, g2, padded, gpad, pr2, pp2
    soft = {}
    for sb, sn in ((1024, 100), (256, 1000), (64, 10_000), (8, 100_000), (1, 1_000_000)):
        torch.manual_seed(0)
        x = torch.randn(sb, sn, device="cuda")
        gx = torch.randn(sb, sn, device="cuda")
        for name, eps in (("1", 1.0), ("1/n", 1.0 / sn)):
            xr = x.detach().requires_grad_()

            def sfb(xr=xr, eps=eps, gx=gx) -> None:
                torch.autograd.grad(torchisotonic_amd.soft_rank(xr, eps), xr, gx)

            soft[f"{sb}x{sn} eps={name}"] = {
                "fwd_ms": 1e3 * timed_calls(lambda x=x, eps=eps: torchisotonic_amd.soft_rank(x, eps), steps, warmup),
                "fwd_bwd_ms": 1e3 * timed_calls(sfb, steps, warmup),
            }
    res["soft_rank"] = soft
    m = 6_500_000
    cr = np.random.default_rng(3)
    logit = cr.normal(-1.2, 1.5, m)
    scores = torch.from_numpy((1 / (1 + np.exp(-logit))).astype(np.float32)).cuda()
    labels = torch.from_numpy((cr.random(m) < 1 / (1 + np.exp(-(logit * 0.8 + 0.3)))).astype(np.float32)).cuda()
    t_fit = timed_calls(lambda: torchisotonic_amd.calibration_fit(scores, labels), max(5, steps // 4), 1)
    xp, fp = torchisotonic_amd.calibration_fit(scores, labels)
    q = scores.double()
    interp_out = torch.empty_like(q)
    index = _ext.interp_index(xp)
    xlaunch = lambda: lib.ti_interp_index(xp.data_ptr(), xp.numel(), _ext.F64, index.data_ptr(), index.numel(), s)  # noqa: E731
    ilaunch = lambda: lib.ti_interp_indexed(q.data_ptr(), xp.data_ptr(), fp.data_ptr(), index.data_ptr(), index.numel(),  # noqa: E731
                                            interp_out.data_ptr(), m, xp.numel(), _ext.F64, s)
    flaunch = lambda: lib.ti_interp(q.data_ptr(), xp.data_ptr(), fp.data_ptr(), interp_out.data_ptr(), m, xp.numel(), _ext.F64, s)  # noqa: E731
    assert xlaunch() == 0 and ilaunch() == 0 and flaunch() == 0
    k = kernel_ms(ilaunch, 50)
    kx = kernel_ms(xlaunch, 50)
    kf = kernel_ms(flaunch, 20)
    cal = torchisotonic_amd.IsotonicCalibrator()
    cal.xp, cal.fp, cal.index = xp, fp, index

    def torch_interp() -> torch.Tensor:  # the reference's tensor formula (calibrate.py:163-168)
        i = torch.searchsorted(xp, q).clamp(1, xp.numel() - 1)
        x0, x1, f0, f1 = xp[i - 1], xp[i], fp[i - 1], fp[i]
        return f0 + ((q - x0) / (x1 - x0).clamp_min(1e-300)).clamp(0, 1) * (f1 - f0)

    res["calibration"] = {
        "scores": m,
        "knots": xp.numel(),
        "fit_ms": 1e3 * t_fit,
        "predict": rate(m, timed_calls(lambda: torchisotonic_amd.calibration_predict(q, xp, fp), steps, warmup), 16),
        "predict_kept_index": rate(m, timed_calls(lambda: cal.predict(q), steps, warmup), 16),
        "interp_kernel_ms": k,
        "interp_kernel_pct_roofline": 100 * 16 * m / (k * 1e-3) / 1e9 / PEAK_GBPS,
        "interp_index_kernel_ms": kx,
        "interp_full_search_kernel_ms": kf,
        "interp_torch_formula_ms": 1e3 * timed_calls(torch_interp, steps, warmup),
    }
    return res


# The reference's README table: its grid (reference bench/bench.py:31-33) and data (:108-110):
# float32 rows of a noisy trend, reversed, fitted decreasing and unweighted.
GRID = [(1_000_000, 16), (100_000, 128), (10_000, 1_000), (1_000, 10_000), (100, 100_000),
        (10, 1_000_000), (1, 10_000_000), (100, 1_000), (10, 10_000), (1, 100_000),
        (1, 1_000_000), (1, 100_000_000)]  # fmt: skip


def bench_grid(repeats: int = 10) -> dict:
    """Per (batch, n): seconds per call of the public API, each call followed by a device
    synchronisation (the reference's method, bench/bench.py:47-64), median and best."""
    out = {}
    for b, n in GRID:
        rng = np.random.default_rng(0)
        trend = np.linspace(0, 3, n, dtype=np.float32)
        data = (trend + rng.standard_normal((b, n), dtype=np.float32))[:, ::-1].copy()
        x = torch.from_numpy(data).cuda()
        del data
        torchisotonic_amd.isotonic(x, increasing=False)  # warm-up (first call's allocations)
        warm_gpu()
        times = []
        for _ in range(repeats):
            t0 = time.perf_counter()
            torchisotonic_amd.isotonic(x, increasing=False)
            sync()
            times.append(time.perf_counter() - t0)
        out[f"{b}x{n}"] = {"median_ms": float(np.median(times)) * 1e3, "best_ms": float(np.min(times)) * 1e3}
        log(f"  grid {b} x {n}: {out[f'{b}x{n}']['median_ms']:.3f} ms")
        del x
        torch.cuda.empty_cache()
    return out


# --- CPU baseline ---------------------------------------------------------------------------


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
        f"({sum(times):.1f} s), rows over {threads} OpenMP threads of {os.cpu_count()} "
        f"({cpu_model()})",
    }


def cpu_c4(n: int = 10_000_000) -> dict:
    """The reference CPU solver on a 1e7-element prefix-shaped sample of C4 (one row: the
    reference runs a row on one thread, ops.cpp:30)."""
    import oracle

    rng = np.random.default_rng(0)
    s = np.sort(rng.standard_normal(n) * 1.5)
    y = (rng.random(n) < 1.0 / (1.0 + np.exp(-s))).astype(np.float32)[None]
    w = rng.integers(1, 6, n).astype(np.float32)[None]
    impl = "reference" if oracle.ref_lib() is not None else "oracle"
    t0 = time.perf_counter()
    oracle.pava(y, w, threads=1, impl=impl, with_starts=False)
    t = time.perf_counter() - t0
    return {"gelem_s": n / t / 1e9, "cores": 1, "kind": "reference" if impl == "reference" else "port",
            "sample": f"C4-shaped row of {n} elements, f32 weighted, one thread"}


def measured_traffic() -> float | None:
    """HBM bytes per launch of the headline kernel, from the committed counter summary."""
    f = ROOT / "profiles" / "short_rows_kernel_c2_traffic.json"
    try:
        t = json.loads(f.read_text())
        kib = t["fetch_size_kib"] * t["fetch_scale"] + t["write_size_kib"] * t["write_scale"]
        return kib * 1024.0
    except (OSError, KeyError, ValueError):
        return None


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--configs", default="c2,c4,c5,c1,c3,next,hull")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(
            "bench.py measures one GPU: rows are independent and this build runs on a single "
            "MI355X; multi-GPU sharding is design-only. Run with --gpus 1.",
            file=sys.stderr,
        )
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    configs = set(args.configs.split(","))
    warm_gpu()
    log("C2 ...")
    c2 = bench_c2(args.steps, args.warmup)
    ceiling = copy_ceiling()
    extra: dict = {"c2": c2}
    if "c4" in configs:
        log("C4 ...")
        extra["c4"] = bench_c4(max(20, args.steps), 2)
    if "c5" in configs:
        log("C5 ...")
        extra["c5"] = bench_c5(max(20, args.steps), 2)
    if "c1" in configs or "c3" in configs:
        log("C1/C3 ...")
        extra["c1_c3"] = bench_c1_c3(max(20, args.steps), 2)
    if "next" in configs:
        log("ragged rows, soft ranks, calibration ...")
        extra.update(bench_next(args.steps, args.warmup))
    if "hull" in configs:
        log("hull-heavy rows ...")
        extra["hull_heavy"] = bench_hull(args.steps, args.warmup)
    if "grid" in configs:
        log("README grid ...")
        extra["grid"] = bench_grid()
    elems = c2["elems"]
    k = c2["kernel_ms"]["short_rows_kernel<float,16,unweighted> (no starts)"]
    achieved = 8 * elems / (k * 1e-3) / 1e9
    if k > c2["fwd"]["ms"]:
        log(f"warning: kernel time {k:.4f} ms exceeds the API's {c2['fwd']['ms']:.4f} ms per call")
    line = {
        "metric": METRIC,
        "value": c2["fwd"]["gelem_s"],
        "unit": "Gelem/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": c2["fwd"]["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64",
        "data": "synthetic: C2 y[b,i] = -0.1 i + N(0,1), seed 0",
        "config": {
            "workload": "C2: isotonic forward, y f32 [1000000, 16], unweighted, increasing=False "
            "(float32 in and out; sums, hull tests and slopes in float64)",
            "batch": 1_000_000,
            "n": 16,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": PEAK_GBPS,
            "unit": "GB/s",
            "frac": achieved / PEAK_GBPS,
            "traffic": measured_traffic(),
            "kernel": "short_rows_kernel<float,16,unweighted>",
            "kernel_ms": k,
            "algorithmic_bytes_per_launch": 8 * elems,
            "copy_ceiling": ceiling,
            "frac_of_copy": achieved / ceiling["gbps"],
        },
        "extra": extra,
    }
    if not args.no_cpu:
        log("CPU baseline ...")
        line["cpu_baseline"] = cpu_baseline()
        if "c4" in configs:
            extra["c4_cpu"] = cpu_c4()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
