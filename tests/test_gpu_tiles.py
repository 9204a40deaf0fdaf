"""Rows longer than 32 elements (the span kernel, merges and tiled expansion) on the GPU against
the oracle: the reference's lane/chunk edge shapes and adversarial patterns (reference
tests/test_cuda.py:31-134, 224-265) restated for the HIP path."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from gpu_util import check_fit, gpu_fit, tolerance

pytestmark = pytest.mark.gpu

# Rows over 32 elements take the span kernel and the merges; the expansion and the backward work
# in tiles of 4096 elements unweighted, 2048 weighted, so these shapes cross their edges.
SHAPES = [33, 63, 64, 65, 100, 255, 256, 511, 1000, 1023, 1024, 1025, 2047, 2048, 2049, 4095, 4096]
LONG_SHAPES = [4097, 8193, 20_000, 100_000]
MULTI_TILE = True  # rows longer than one tile


def fits(n: int, weighted: bool) -> bool:
    return MULTI_TILE or n <= (2048 if weighted else 4096)


def data(batch: int, n: int, dtype: type, seed: int) -> tuple[np.ndarray, np.ndarray]:
    rng = np.random.default_rng(seed)
    y = (np.linspace(0, 3, n) + rng.standard_normal((batch, n))).astype(dtype)
    w = (rng.random((batch, n)) + 0.1).astype(dtype)
    return y, w


@pytest.mark.parametrize("n", SHAPES)
@pytest.mark.parametrize("batch", [1, 3, 70])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_tile_shapes(n: int, batch: int, dtype: type) -> None:
    print(f"tiles n={n} batch={batch} dtype={np.dtype(dtype).name}", flush=True)
    y, w = data(batch, n, dtype, n + batch)
    check_fit(y)
    check_fit(y, None, increasing=False, y_min=-0.5, y_max=2.0)
    if fits(n, True):
        check_fit(y, w, increasing=False)
        check_fit(y, w, increasing=True, y_min=0.0, y_max=2.5)


PATTERNS = ["increasing", "decreasing", "saw", "cliff", "walk", "constant", "valley", "zeros_ones"]


def pattern(name: str, n: int, rng: np.random.Generator) -> np.ndarray:
    i = np.arange(n, dtype=np.float64)
    if name == "increasing":  # every point is a vertex
        return i
    if name == "decreasing":  # one block
        return -i
    if name == "saw":  # convex runs with drops, not aligned to threads or tiles
        return i % 7 + (i % 1500) * 0.1
    if name == "cliff":  # one bridge across almost everything
        return np.where(i == n - 1, -1e9, i)
    if name == "walk":
        return rng.standard_normal(n).cumsum()
    if name == "constant":  # collinear points everywhere
        return np.ones(n)
    if name == "zeros_ones":  # exact ties in means
        return (rng.random(n) < 1 / (1 + np.exp(-np.linspace(-3, 3, n)))).astype(np.float64)
    return (i - n / 3) ** 2  # valley: falls, then rises


@pytest.mark.parametrize("name", PATTERNS)
@pytest.mark.parametrize("n", [700, 1025, 2048, 3000, 4096])
def test_tile_patterns(name: str, n: int) -> None:
    print(f"pattern {name} n={n}", flush=True)
    rng = np.random.default_rng(n)
    y = pattern(name, n, rng)[None]
    w = rng.random((1, n)) + 0.1
    ties = name in ("constant", "zeros_ones", "saw")
    check_fit(y, check_starts=not ties)
    if fits(n, True):
        check_fit(y, w, check_starts=not ties)
        check_fit(y, w, increasing=False, check_starts=not ties)
    check_fit(y.astype(np.float32), check_starts=False)


@pytest.mark.parametrize("n", [40, 2048, 4096])
def test_exact_ties_partition(n: int) -> None:
    # 0/1 labels with integer weights: every sum is an exact integer, so the partition must be
    # the exact one (long-double oracle), ties pooled.
    rng = np.random.default_rng(n)
    y = (rng.random((20, n)) < 1 / (1 + np.exp(-np.linspace(-3, 3, n)))).astype(np.float32)
    w = rng.integers(1, 6, (20, n)).astype(np.float32)
    for ww in (None, w):
        if not fits(n, ww is not None):
            continue
        got, starts = gpu_fit(y, ww)
        want, want_starts = oracle.pava(y, ww, acc="f64x")
        assert np.abs(got - want).max() <= tolerance(y)
        np.testing.assert_array_equal(starts, want_starts)


@pytest.mark.parametrize("n", [100, 500, 3000])
def test_nan_rows_long(n: int) -> None:
    # (rows of 100 and 500: several rows a wave of the span kernel, NaN rows among them)
    rng = np.random.default_rng(1)
    y = rng.standard_normal((40, n))
    y[3, 17] = np.nan
    y[39, n - 1] = np.nan
    y[20, 0] = np.nan
    check_fit(y)
    check_fit(y.astype(np.float32), increasing=False)


@pytest.mark.parametrize("big", [1e3, 1e6, 1e12])
@pytest.mark.parametrize("n", [500, 2048])
def test_cancelling_sums(n: int, big: float) -> None:
    # reference tests/test_cuda.py:243-265: per 64 elements, 32 of +big, one of -32 big, then
    # small near-collinear values; coordinates are differences of far larger terms.
    rng = np.random.default_rng(n)
    k = np.arange(n) % 64
    y = np.where(k < 32, big, 1.0)
    y[k == 32] = -32 * big
    y = y + 1e-3 * (-1.0) ** k * (k > 32) + 1e-6 * rng.standard_normal(n)
    for w in (None, rng.random(n) + 0.1):
        for dtype, step, dev in ((np.float64, 8 * 2.0**-52, 1e-14), (np.float32, 0, 1e-7)):
            yy = y.astype(dtype)[None]
            ww = None if w is None else w.astype(dtype)[None]
            want, _ = oracle.pava(yy.astype(np.float64), None if ww is None else ww.astype(np.float64))
            got, _ = gpu_fit(yy, ww, with_starts=False)
            got = got.astype(np.float64)
            scale = float(np.abs(yy.astype(np.float64)).max())
            assert float((got[:, :-1] - got[:, 1:]).max()) <= step * scale
            assert float(np.abs(got - want).max()) <= dev * scale


@pytest.mark.parametrize("name", ["collinear", "offset", "consecutive"])
def test_float32_fit_is_monotone_long(name: str) -> None:
    rng = np.random.default_rng(2)
    n = 4096
    i = np.arange(n, dtype=np.float64)
    one = np.float32(1.0).view(np.int32)
    y = {
        "collinear": 1e6 + 1e-3 * i + 1e-9 * rng.standard_normal(n),
        "offset": 1e6 + rng.standard_normal(n),
        "consecutive": (one + np.arange(n, dtype=np.int32)).view(np.float32).astype(np.float64),
    }[name].astype(np.float32)[None]
    u = rng.random((1, n))
    for w in (None, (u + 0.1).astype(np.float32), np.exp(8 * u).astype(np.float32)):
        if w is not None:
            yy, ww = y[:, :2048], w[:, :2048]
        else:
            yy, ww = y, None
        got, _ = gpu_fit(np.ascontiguousarray(yy), None if ww is None else np.ascontiguousarray(ww), with_starts=False)
        assert (np.diff(got, axis=1) >= 0).all()


def grad_rows(batch: int, n: int, seed: int, dtype=np.float64):
    rng = np.random.default_rng(seed)
    y = (np.linspace(0, 3, n) + rng.standard_normal((batch, n))).astype(dtype)
    w = (rng.random((batch, n)) + 0.1).astype(dtype)
    c = rng.standard_normal((batch, n)).astype(dtype)
    return y, w, c


def gpu_grads(y, w, c, **kw):
    import torch

    import torchisotonic_amd

    yy = torch.from_numpy(y).cuda().requires_grad_()
    ww = None if w is None else torch.from_numpy(w).cuda().requires_grad_()
    fit = torchisotonic_amd.isotonic(yy, ww, **kw)
    inputs = (yy,) if ww is None else (yy, ww)
    gs = torch.autograd.grad((fit * torch.from_numpy(c).cuda()).sum(), inputs)
    return [x.cpu().numpy() for x in gs], fit.detach().cpu().numpy()


@pytest.mark.parametrize(("batch", "n"), [(70, 33), (9, 64), (9, 65), (7, 128), (5, 512), (5, 513),
                                          (5, 1000), (5, 1024), (3, 1025), (3, 2048), (3, 4096),
                                          (3, 4097), (2, 9000), (2, 70_000)])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_tile_gradients_match_oracle(batch: int, n: int, dtype: type) -> None:
    # reference tests/test_cuda.py:137-157: the gradient against the CPU's closed form on the
    # oracle's partition (tie-free data), weighted (when one tile holds the row) and not.
    print(f"tile grad batch={batch} n={n} dtype={np.dtype(dtype).name}", flush=True)
    y, w, c = grad_rows(batch, n, n, dtype)
    tol = 1e-12 if dtype == np.float64 else 2e-5
    for inc in (True, False):
        for weights in (w, None):
            if weights is not None and not fits(n, True):
                continue
            gs, _ = gpu_grads(y, weights, c, increasing=inc)
            fit, starts = oracle.pava(y, weights, increasing=inc, acc="f64")
            ey, ew = oracle.block_grad(
                starts, c.astype(np.float64), None if weights is None else weights.astype(np.float64),
                y.astype(np.float64), fit, want_w=weights is not None,
            )
            np.testing.assert_allclose(gs[0], ey, rtol=tol, atol=tol)
            if weights is not None:
                scale = tol * (1 + float(np.abs(y).max()))
                np.testing.assert_allclose(gs[1], ew, rtol=tol, atol=scale)


@pytest.mark.parametrize("name", PATTERNS)
@pytest.mark.parametrize("n", [100, 333, 1024, 1025, 2048, 3000, 9000, 70_000])
def test_tile_gradient_is_block_average(name: str, n: int) -> None:
    # reference tests/test_cuda.py:160-183: whatever the data (ties included) the gradient is
    # the block average over the blocks the GPU's fit reports.
    import torch

    from torchisotonic_amd import _ext

    rng = np.random.default_rng(n)
    y = np.broadcast_to(pattern(name, n, rng), (3, n)).copy()
    w = rng.random((3, n)) + 0.1
    c = rng.standard_normal((3, n))
    for weights in (w, None):
        if weights is not None and not fits(n, True):
            continue
        gs, fit = gpu_grads(y, weights, c)
        _, starts = _ext.isotonic_tiles(
            torch.from_numpy(y).cuda(), None if weights is None else torch.from_numpy(weights).cuda(),
            True, True, True,
        )  # the same fit again: its partition
        s = starts.cpu().numpy().astype(np.uint8)
        ey, ew = oracle.block_grad(s, c, weights, y, fit, want_w=weights is not None)
        np.testing.assert_allclose(gs[0], ey, rtol=1e-9, atol=1e-9)
        if weights is not None:
            np.testing.assert_allclose(gs[1], ew, rtol=1e-9, atol=1e-9 * (1 + np.abs(y).max()))


@pytest.mark.parametrize("n", [100, 2048, 9000])
def test_tile_clamp_gradient_matches_torch_clamp(n: int) -> None:
    import torch

    import torchisotonic_amd

    rng = np.random.default_rng(n)
    y = np.round(rng.standard_normal((20, n)) * 2) / 2
    w = rng.random(y.shape) + 0.1
    c = rng.standard_normal(y.shape)
    for lo, hi in ((-0.5, 0.5), (0.0, None), (None, 1.0), (1.0, -1.0)):
        yy = torch.from_numpy(y).cuda().requires_grad_()
        ww = torch.from_numpy(w).cuda().requires_grad_()
        out = torchisotonic_amd.isotonic(yy, ww, y_min=lo, y_max=hi)
        gy, gw = torch.autograd.grad((out * torch.from_numpy(c).cuda()).sum(), (yy, ww))
        yy2 = torch.from_numpy(y).cuda().requires_grad_()
        ww2 = torch.from_numpy(w).cuda().requires_grad_()
        out2 = torchisotonic_amd.isotonic(yy2, ww2).clamp(min=lo, max=hi)
        gy2, gw2 = torch.autograd.grad((out2 * torch.from_numpy(c).cuda()).sum(), (yy2, ww2))
        torch.testing.assert_close(out, out2, rtol=0, atol=0)
        torch.testing.assert_close(gy, gy2, rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(gw, gw2, rtol=1e-12, atol=1e-12)


def test_tile_gradcheck() -> None:
    import torch
    from torch.autograd import gradcheck

    import torchisotonic_amd

    g = torch.Generator().manual_seed(0)
    y = torch.randn(2, 40, generator=g, dtype=torch.float64).cuda().requires_grad_()
    w = (torch.rand(2, 40, generator=g, dtype=torch.float64) + 0.1).cuda().requires_grad_()
    for kw in ({}, {"increasing": False}, {"y_min": -0.3, "y_max": 0.5}):
        assert gradcheck(lambda y, w: torchisotonic_amd.isotonic(y, w, **kw), (y, w))
        assert gradcheck(lambda y: torchisotonic_amd.isotonic(y, **kw), (y,))


@pytest.mark.parametrize("n", LONG_SHAPES)
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_long_rows(n: int, dtype: type) -> None:
    # rows of several tiles: the cross-tile merge and the expansion
    print(f"long rows n={n} dtype={np.dtype(dtype).name}", flush=True)
    batch = 3
    y, w = data(batch, n, dtype, n)
    check_fit(y)
    check_fit(y, w, increasing=False)
    check_fit(y, None, increasing=False, y_min=-0.5, y_max=2.0)


@pytest.mark.parametrize("name", PATTERNS)
@pytest.mark.parametrize("n", [9000, 70_000, 300_000])
def test_long_patterns(name: str, n: int) -> None:
    print(f"long pattern {name} n={n}", flush=True)
    rng = np.random.default_rng(n)
    y = pattern(name, n, rng)[None]
    w = rng.random((1, n)) + 0.1
    ties = name in ("constant", "zeros_ones", "saw")
    check_fit(y, check_starts=not ties)
    check_fit(y, w, check_starts=not ties)
    check_fit(y, w, increasing=False, check_starts=not ties)
    check_fit(y.astype(np.float32), check_starts=False)


@pytest.mark.parametrize("n", [300_000, 5_000_000])
def test_long_exact_ties(n: int) -> None:
    # calibration-shaped rows (0/1 labels, integer counts): exact partitions across merges
    rng = np.random.default_rng(n)
    s = np.sort(rng.standard_normal(n) * 1.5)
    y = (rng.random(n) < 1 / (1 + np.exp(-s))).astype(np.float32)[None]
    w = rng.integers(1, 6, n).astype(np.float32)[None]
    got, starts = gpu_fit(y, w)
    want, want_starts = oracle.pava(y, w, acc="f64x")
    assert np.abs(got - want).max() <= tolerance(y)
    np.testing.assert_array_equal(starts, want_starts)


@pytest.mark.parametrize("n", [100, 1500, 9000])
def test_long_nan_row_gradients(n: int) -> None:
    # a NaN row is one block: gy is the row's average gradient, gw NaN; through a clamp, zero
    # (rows of 100: both rows in one workgroup of the packed backward)
    rng = np.random.default_rng(5)
    y = rng.standard_normal((2, n))
    y[0, n // 2 - 1] = np.nan
    w = rng.random((2, n)) + 0.1
    c = rng.standard_normal((2, n))
    (gy, gw), _ = gpu_grads(y, w, c)
    np.testing.assert_allclose(gy[0], w[0] * c[0].sum() / w[0].sum(), rtol=1e-10)
    assert np.isnan(gw[0]).all()
    fit, starts = oracle.pava(y[1:], w[1:])
    ey, _ = oracle.block_grad(starts, c[1:], w[1:])
    np.testing.assert_allclose(gy[1:], ey, rtol=1e-10, atol=1e-12)
    (gy, gw), _ = gpu_grads(y, w, c, y_min=-0.5)
    assert (gy[0] == 0).all() and np.isnan(gw[0]).all()


@pytest.mark.parametrize("n", [1000, 5000, 70_000])
@pytest.mark.parametrize("dtype", ["float32", "float64"])
def test_weight_check_every_path(n: int, dtype: str) -> None:
    # a non-positive or NaN weight anywhere in a row of one tile or of several raises (the
    # long-row forward returns once its first kernel has read w, before the fit is done), and a
    # valid call right after is unaffected by the failed one
    import torch

    import torchisotonic_amd

    print(f"weight check n={n} dtype={dtype}", flush=True)
    rng = np.random.default_rng(n)
    y = torch.from_numpy(rng.standard_normal((2, n))).to(getattr(torch, dtype)).cuda()
    good = torch.from_numpy(rng.random((2, n)) + 0.1).to(y.dtype).cuda()
    for bad_value in (0.0, -2.0, float("nan")):
        for row, col in ((0, 0), (1, n // 2), (1, n - 1)):
            w = good.clone()
            w[row, col] = bad_value
            with pytest.raises(ValueError, match="strictly positive"):
                torchisotonic_amd.isotonic(y, w)
    got = torchisotonic_amd.isotonic(y, good).cpu().numpy()
    want, _ = oracle.pava(y.cpu().double().numpy(), good.cpu().double().numpy())
    assert np.abs(got - want).max() <= tolerance(y.cpu().numpy())


def check_many_rows(batch: int, n: int) -> None:
    rng = np.random.default_rng(n)
    y = (np.linspace(0, 2, n) + rng.standard_normal((batch, n))).astype(np.float32)
    w = (rng.random((batch, n)) + 0.1).astype(np.float32)
    check_fit(y)
    check_fit(y, w, increasing=False)
    check_fit(y.astype(np.float64), w.astype(np.float64), y_min=-0.2, y_max=1.5)
    if batch <= 10_000:
        c = rng.standard_normal((batch, n))
        (gy, gw), fit = gpu_grads(y.astype(np.float64), w.astype(np.float64), c)
        want, starts = oracle.pava(y.astype(np.float64), w.astype(np.float64))
        ey, ew = oracle.block_grad(starts, c, w.astype(np.float64), y.astype(np.float64), want, want_w=True)
        np.testing.assert_allclose(gy, ey, rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(gw, ew, rtol=1e-9, atol=1e-9)
        # float32, unweighted, decreasing, through a clamp: the clamp's mask from the GPU's fit
        cf = c.astype(np.float32)
        (gy,), _ = gpu_grads(y, None, cf, increasing=False, y_min=0.0, y_max=1.2)
        (_,), raw = gpu_grads(y, None, cf, increasing=False)  # the fit before the clamp
        want, starts = oracle.pava(y.astype(np.float64), None, increasing=False)
        inside = ((raw >= 0.0) & (raw <= 1.2)).astype(np.float64)
        ey, _ = oracle.block_grad(starts, cf.astype(np.float64), None)
        # the mask is constant over a block (one fit value a block)
        np.testing.assert_allclose(gy, ey * inside, rtol=2e-5, atol=2e-5)


@pytest.mark.parametrize(("batch", "n"), [(1, 2**24 + 5), (1_100_000, 16)])
def test_weight_check_large(batch: int, n: int, monkeypatch: pytest.MonkeyPatch) -> None:
    # past 2^24 elements the fit's own first kernel checks the weights as it reads them (smaller
    # fits check them in a kernel of their own first): a bad weight anywhere still raises
    monkeypatch.setenv("TI_KEEP_MIN_BYTES", str(256 << 20))  # (the kept-hulls path under autograd)
    import torch

    import torchisotonic_amd

    print(f"weight check large batch={batch} n={n}", flush=True)
    rng = np.random.default_rng(7)
    y = torch.from_numpy(rng.standard_normal((batch, n)).astype(np.float32)).cuda()
    good = torch.from_numpy((rng.random((batch, n)) + 0.1).astype(np.float32)).cuda()
    for bad_value in (0.0, float("nan")):
        for row, col in ((0, 0), (batch - 1, n // 2), (batch - 1, n - 1)):
            w = good.clone()
            w[row, col] = bad_value
            with pytest.raises(ValueError, match="strictly positive"):
                torchisotonic_amd.isotonic(y, w)
            # under autograd (past 256 MB of workspace the node keeps only the final hulls, and the
            # host waits for their vertex bound, not for the weights' own mark)
            with pytest.raises(ValueError, match="strictly positive"):
                torchisotonic_amd.isotonic(y.detach().requires_grad_(), w)
    got = torchisotonic_amd.isotonic(y, good).cpu().numpy()
    want, _ = oracle.pava(y.cpu().double().numpy(), good.cpu().double().numpy())
    assert np.abs(got - want).max() <= tolerance(y.cpu().numpy())


@pytest.mark.parametrize(("batch", "n"), [(10_000, 33), (9_000, 64), (40_000, 256), (140_000, 40)])
def test_many_rows_of_one_span(batch: int, n: int) -> None:
    # batches of thousands of rows of at most 256 elements (at most 64 below 32768 rows): one
    # span per row, one row per lane and 64 rows a wave, the span hulls the final hulls (no
    # merge level)
    print(f"one span a row batch={batch} n={n}", flush=True)
    check_many_rows(batch, n)


@pytest.mark.parametrize(("batch", "n"), [(9_000, 100), (8_192, 256), (2_000, 512), (3_000, 1000), (5_000, 1500)])
def test_several_rows_a_wave(batch: int, n: int) -> None:
    # rows of at most 2048 elements: several rows a wave of the span kernel, a power-of-two
    # number of spans each, merged per row in the wave
    print(f"rows a wave batch={batch} n={n}", flush=True)
    check_many_rows(batch, n)


# (batch, n) of one merge level, one row a wave: the wave that builds a row's final hull also
# writes its tile records, start bits and fit. Rows with a vertex at every element have more
# edges than the wave's table of edge values holds (about 3.5k-4.8k), so it is restaged within
# the row; n = 2049 is one element past the packed expansion's rows.
ONE_LEVEL_SHAPES = [(600, 10_000), (700, 5_000), (2_100, 2_049)]


@pytest.mark.parametrize(("batch", "n"), ONE_LEVEL_SHAPES)
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("weighted", [False, True])
def test_one_level_rows_expanded_by_their_wave(batch: int, n: int, dtype: type, weighted: bool) -> None:
    from torchisotonic_amd import _ext

    print(f"one-level rows batch={batch} n={n} dtype={np.dtype(dtype).name} weighted={weighted}", flush=True)
    geo = _ext.geometry(batch, n, weighted)
    assert geo["levels"] == 1 and geo["rows_per_wave"] == 1, geo
    rng = np.random.default_rng(n + batch + weighted)
    y = np.linspace(0, 3, n) + rng.standard_normal((batch, n))
    mono = np.arange(0, batch, 3)
    y[mono] = 1e-3 * np.arange(n) + rng.random((mono.size, 1))  # a vertex at every element
    y[5, n // 2] = np.nan
    y = y.astype(dtype)
    w = (rng.random((batch, n)) + 0.1).astype(dtype) if weighted else None
    got, starts = check_fit(y, w)
    assert starts[mono].all()
    check_fit(y, w, increasing=False, y_min=0.5, y_max=2.0)
    # both gradients through the wave's tile records and start bits (rows without the NaN)
    ok = ~np.isnan(y).any(axis=1)
    c = rng.standard_normal((batch, n)).astype(dtype)
    gs, _ = gpu_grads(y, w, c)
    fit, st = oracle.pava(y[ok], None if w is None else w[ok], acc="f64")
    ey, ew = oracle.block_grad(
        st, c[ok].astype(np.float64), None if w is None else w[ok].astype(np.float64),
        y[ok].astype(np.float64), fit, want_w=w is not None,
    )
    tol = 1e-12 if dtype == np.float64 else 2e-5
    np.testing.assert_allclose(gs[0][ok], ey, rtol=tol, atol=tol)
    if w is not None:
        np.testing.assert_allclose(gs[1][ok], ew, rtol=tol, atol=tol * (1 + float(np.nanmax(np.abs(y)))))


# Rows whose hulls keep most of their points as vertices (rising data with a drop every 997
# elements) at sizes whose upper merge levels work by reference to the children's vertices
# (more than LDS holds) and move hundreds of thousands of survivors in place, each child's by a
# shift that grows with every drop before it.
@pytest.mark.parametrize(("batch", "n"), [(1, 3_000_000), (3, 700_000), (20, 150_000)])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("weighted", [False, True])
def test_near_monotone_rows_many_survivors(batch: int, n: int, dtype: type, weighted: bool) -> None:
    from torchisotonic_amd import _ext

    print(f"near-monotone rows batch={batch} n={n} dtype={np.dtype(dtype).name} weighted={weighted}", flush=True)
    assert _ext.geometry(batch, n, weighted)["levels"] >= 2
    rng = np.random.default_rng(n + batch + weighted)
    i = np.arange(n)
    y = 1e-3 * i + 1e-5 * rng.standard_normal((batch, n)) - 0.3 * (i % 997 == 0)
    y = y.astype(dtype)
    w = (rng.random((batch, n)) + 0.5).astype(dtype) if weighted else None
    check_fit(y, w)


# (batch, n): rows of two merge levels in batches of 256 or more, whose final merge launch has a
# workgroup a row: that workgroup also writes the row's tile records, start bits and fit. Rows
# with a vertex at every element have more edges than the workgroup's table of edge values holds,
# so it is restaged within the row.
LAST_MERGE_SHAPES = [(256, 20_000), (300, 40_000)]


@pytest.mark.parametrize(("batch", "n"), LAST_MERGE_SHAPES)
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("weighted", [False, True])
def test_rows_expanded_by_their_last_merge(batch: int, n: int, dtype: type, weighted: bool) -> None:
    from torchisotonic_amd import _ext

    print(f"last-merge rows batch={batch} n={n} dtype={np.dtype(dtype).name} weighted={weighted}", flush=True)
    assert _ext.geometry(batch, n, weighted)["levels"] == 2
    rng = np.random.default_rng(n + batch + weighted)
    y = np.linspace(0, 3, n) + rng.standard_normal((batch, n))
    mono = np.arange(0, batch, 5)
    y[mono] = 1e-3 * np.arange(n) + rng.random((mono.size, 1))  # a vertex at every element
    y[7, n // 3] = np.nan
    y = y.astype(dtype)
    w = (rng.random((batch, n)) + 0.1).astype(dtype) if weighted else None
    got, starts = check_fit(y, w)
    assert starts[mono].all()
    check_fit(y, w, increasing=False, y_min=0.5, y_max=2.0)
    ok = ~np.isnan(y).any(axis=1)
    c = rng.standard_normal((batch, n)).astype(dtype)
    gs, _ = gpu_grads(y, w, c)
    fit, st = oracle.pava(y[ok], None if w is None else w[ok], acc="f64")
    ey, ew = oracle.block_grad(
        st, c[ok].astype(np.float64), None if w is None else w[ok].astype(np.float64),
        y[ok].astype(np.float64), fit, want_w=w is not None,
    )
    tol = 1e-12 if dtype == np.float64 else 2e-5
    np.testing.assert_allclose(gs[0][ok], ey, rtol=tol, atol=tol)
    if w is not None:
        np.testing.assert_allclose(gs[1][ok], ew, rtol=tol, atol=tol * (1 + float(np.nanmax(np.abs(y)))))


# Six rows of 300000 elements: spans of 32, so the second merge level has three parents a row,
# each over 131072 elements (18 in the batch), and the third one a row (6): both levels write
# their hulls into the other vertex store than their children's, the second store and then the
# first again. Rows with a vertex at every element (0, 3) have parents of more than 4096
# survivors, which survivors_kernel writes; a near-monotone row with drops (2) some of either;
# noisy rows (1, 5) only parents that write their own; row 4 rises too but holds a NaN. Fit,
# start bits and both gradients against the oracle, increasing, and decreasing with clamps.
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("weighted", [False, True])
def test_deferred_survivors_mixed_rows(dtype: type, weighted: bool) -> None:
    from torchisotonic_amd import _ext

    batch, n = 6, 300_000
    print(f"deferred survivors batch={batch} n={n} dtype={np.dtype(dtype).name} weighted={weighted}", flush=True)
    geo = _ext.geometry(batch, n, weighted)
    assert geo["span0"] == 32 and geo["levels"] == 3
    rng = np.random.default_rng(7 + weighted)
    i = np.arange(n)
    y = np.linspace(0, 3, n) + rng.standard_normal((batch, n))
    for r in (0, 3, 4):
        y[r] = 1e-3 * i + rng.random()
    y[2] = 1e-3 * i + 1e-5 * rng.standard_normal(n) - 0.3 * (i % 997 == 0)
    y[4, n // 3] = np.nan  # (a rising row with a NaN: its parents defer as well)
    y = y.astype(dtype)
    w = (rng.random((batch, n)) + 0.1).astype(dtype) if weighted else None
    got, starts = check_fit(y, w)
    assert starts[0].all() and starts[3].all()
    check_fit(y, w, increasing=False, y_min=0.5, y_max=2.0)
    ok = ~np.isnan(y).any(axis=1)
    c = rng.standard_normal((batch, n)).astype(dtype)
    gs, _ = gpu_grads(y, w, c)
    fit, st = oracle.pava(y[ok], None if w is None else w[ok], acc="f64")
    ey, ew = oracle.block_grad(
        st, c[ok].astype(np.float64), None if w is None else w[ok].astype(np.float64),
        y[ok].astype(np.float64), fit, want_w=w is not None,
    )
    tol = 1e-12 if dtype == np.float64 else 2e-5
    np.testing.assert_allclose(gs[0][ok], ey, rtol=tol, atol=tol)
    if w is not None:
        np.testing.assert_allclose(gs[1][ok], ew, rtol=tol, atol=tol * (1 + float(np.nanmax(np.abs(y)))))


def chord_rows(rows: int, n: int, dtype: type, weighted: bool, seed: int) -> tuple[np.ndarray, np.ndarray | None, np.ndarray]:
    """Rows that put points on and near the chords of their neighbours, in four kinds by row
    (index mod 4): small integers (exact ties, points exactly on chords), noise over 24 decades,
    noise rounded to 1/64 plus a trace of noise (near ties), a trend with noise."""
    rng = np.random.default_rng(seed)
    kind = np.arange(rows) % 4
    y = np.empty((rows, n))
    y[kind == 0] = rng.integers(0, 4, ((kind == 0).sum(), n))
    y[kind == 1] = rng.standard_normal(((kind == 1).sum(), n)) * 10.0 ** rng.uniform(-12, 12, ((kind == 1).sum(), n))
    q = rng.standard_normal(((kind == 2).sum(), n))
    y[kind == 2] = np.round(q * 64) / 64 + 1e-9 * rng.standard_normal(q.shape)
    y[kind == 3] = np.linspace(0, 3, n) + rng.standard_normal(((kind == 3).sum(), n))
    w = None
    if weighted:
        w = rng.random((rows, n)) + 0.1
        w[kind == 0] = rng.integers(1, 5, ((kind == 0).sum(), n))
        w = w.astype(dtype)
    return y.astype(dtype), w, kind


@pytest.mark.parametrize("increasing", [True, False])
@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_candidate_filter_same_bits(dtype: type, weighted: bool, increasing: bool) -> None:
    # A grid of at most two waves a SIMD (600 rows of 5000: 600 waves) runs the span kernel's
    # stronger candidate test, which drops points lying clearly above the chord of their
    # neighbours two elements away; 3000 rows (3000 waves, the same spans of 80) run without it. The same rows through
    # both give the same bits, and the oracle's fit (and, but for the rows over 24 decades, whose
    # sums round differently in any order, its partition).
    from torchisotonic_amd import _ext

    n, small, big = 5000, 600, 3000
    print(f"candidate filter dtype={np.dtype(dtype).name} weighted={weighted} increasing={increasing}", flush=True)
    assert _ext.geometry(small, n, weighted) == _ext.geometry(big, n, weighted)
    y, w, kind = chord_rows(small, n, dtype, weighted, 11 + weighted + 2 * increasing)
    yb, wb, _ = chord_rows(big, n, dtype, weighted, 5)
    yb[:small] = y
    if w is not None:
        wb[:small] = w
    got, starts = gpu_fit(y, w, increasing)
    got_b, starts_b = gpu_fit(yb, wb, increasing)
    np.testing.assert_array_equal(got_b[:small].view(np.uint8), got.view(np.uint8))
    np.testing.assert_array_equal(starts_b[:small], starts)
    exact = kind != 1
    check_fit(y[exact], None if w is None else w[exact], increasing)
    # (rows over 24 decades: the float64 oracle's fit only; a float32 sum of them is no reference)
    want, _ = oracle.pava(y[~exact], None if w is None else w[~exact], increasing=increasing, acc="f64")
    assert float(np.abs(got[~exact].astype(np.float64) - want).max()) <= tolerance(y[~exact])
