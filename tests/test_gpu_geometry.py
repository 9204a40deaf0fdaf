"""The kernel geometries bench.py times, at their real sizes, and exact-arithmetic cases across the
merge levels, on the GPU against the oracle.

- C4 (one weighted row of 1e8, BASELINE's recipe: 0/1 labels, integer counts): spans of 256
  elements and four merge launches; the fit, the exact partition (long-double oracle) and both
  gradients.
- C5 (1000 rows of 65536, BASELINE's recipe): spans of 256 and the fused first merge level; fit
  and gradients.
- One row of 2^25 elements: spans of 256 at batch 1.
- Cancelling sums (reference tests/test_cuda.py:243-265, which runs n = 100000 to reach merged
  chunks) at 100000 and 5e6 elements, so the merge kernel's double-double child offsets run
  under cancellation.
- Exact ties whose cross products are not representable (non-integer sums): every test of
  collinear points must pool them, on the short, span, merge paths.
- The golden fixtures (scipy) on the span path: rows of 33-60 elements and of 20000.

Each test prints its case before the GPU work starts.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
import torchisotonic_amd
from gpu_util import check_fit, gpu_fit, tolerance
from torchisotonic_amd import _ext

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def say(*a: object) -> None:
    print(*a, flush=True)


def autograd(y: np.ndarray, w: np.ndarray | None, g: np.ndarray, **kw) -> tuple[np.ndarray, list[np.ndarray]]:
    """The fit and its gradients through the public API (autograd), as numpy arrays."""
    yt = torch.from_numpy(y).cuda().requires_grad_()
    wt = None if w is None else torch.from_numpy(w).cuda().requires_grad_()
    fit = torchisotonic_amd.isotonic(yt, wt, **kw)
    inputs = (yt,) if wt is None else (yt, wt)
    gs = torch.autograd.grad(fit, inputs, torch.from_numpy(g).cuda())
    return fit.detach().cpu().numpy(), [x.cpu().numpy() for x in gs]


def close_grad(got: np.ndarray, want: np.ndarray, rtol: float) -> None:
    scale = max(float(np.abs(want).max()), 1e-300)
    np.testing.assert_allclose(got, want, rtol=rtol, atol=rtol * scale)


# --- the configurations bench.py times, at full size --------------------------------------------


def c4_data(n: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    # BASELINE C4 (bench.py c4_inputs): s = sort(1.5 N(0, 1)), y = Bernoulli(sigmoid(s)) as 0/1
    # float32, w = randint(1, 6) as float32, seed 0; upstream gradient N(0, 1), seed 1
    rng = np.random.default_rng(0)
    s = np.sort(rng.standard_normal(n) * 1.5)
    y = (rng.random(n) < 1.0 / (1.0 + np.exp(-s))).astype(np.float32)
    del s
    w = rng.integers(1, 6, n).astype(np.float32)
    g = np.random.default_rng(1).standard_normal(n).astype(np.float32)
    return y, w, g


def test_c4_full_size() -> None:
    n = 100_000_000
    geo = _ext.geometry(1, n, True)
    say(f"config c4 n={n} geometry {geo}")
    assert geo["span0"] == 256 and geo["levels"] == 4 and geo["rows_per_wave"] == 1
    y, w, g = c4_data(n)
    got, starts = gpu_fit(y[None], w[None])
    say("c4: GPU fit done; oracle (long double) ...")
    want, want_starts = oracle.pava(y, w, acc="f64x")
    # every sum is an exact integer: the partition is the exact one, ties pooled
    assert float(np.abs(got[0] - want).max()) <= tolerance(y)
    np.testing.assert_array_equal(starts[0], want_starts)
    del got, starts
    say("c4: forward + backward ...")
    fit, (gy, gw) = autograd(y, w, g)
    assert float(np.abs(fit - want).max()) <= tolerance(y)
    ey, ew = oracle.block_grad(want_starts, g.astype(np.float64), w.astype(np.float64), y.astype(np.float64),
                               want, want_w=True)
    close_grad(gy, ey, 1e-5)
    close_grad(gw, ew, 1e-5)


def test_c5_full_size() -> None:
    b, n = 1000, 65536
    geo = _ext.geometry(b, n, True)
    say(f"config c5 {b}x{n} geometry {geo}")
    assert geo["span0"] == 256 and geo["rows_per_wave"] == 1
    # BASELINE C5 (bench.py bench_c5): shared labels, per-row Exponential(1) weights floored at
    # 1e-6, seed 0; upstream gradient N(0, 1), seed 1
    rng = np.random.default_rng(0)
    y0 = (rng.random(n) < 1 / (1 + np.exp(-np.linspace(-4, 4, n)))).astype(np.float32)
    y = np.broadcast_to(y0, (b, n)).copy()
    w = np.maximum(rng.exponential(1.0, (b, n)), 1e-6).astype(np.float32)
    g = np.random.default_rng(1).standard_normal((b, n)).astype(np.float32)
    # runs of equal labels tie at rounding level (their sums are formed differently by the two
    # sides), so the fit is compared, and the gradients over the GPU's own partition
    check_fit(y, w, check_starts=False)
    _, starts = gpu_fit(y, w)
    fit, (gy, gw) = autograd(y, w, g)
    ey, ew = oracle.block_grad(starts, g.astype(np.float64), w.astype(np.float64), y.astype(np.float64),
                               fit.astype(np.float64), want_w=True)
    close_grad(gy, ey, 1e-5)
    close_grad(gw, ew, 1e-5)


@pytest.mark.parametrize("weighted", [False, True])
def test_span256_one_row(weighted: bool) -> None:
    n = 2**25
    geo = _ext.geometry(1, n, weighted)
    say(f"one row of 2^25, weighted={weighted}, geometry {geo}")
    assert geo["span0"] == 256 and geo["levels"] == 3
    rng = np.random.default_rng(25)
    y = (np.linspace(0, 3, n) + rng.standard_normal(n)).astype(np.float32)[None]
    w = (rng.random((1, n)) + 0.1).astype(np.float32) if weighted else None
    check_fit(y, w)
    g = rng.standard_normal((1, n)).astype(np.float32)
    fit, gs = autograd(y, w, g)
    want, starts = oracle.pava(y, w, acc="f64")
    w64 = None if w is None else w.astype(np.float64)
    ey, ew = oracle.block_grad(starts, g.astype(np.float64), w64, y.astype(np.float64), want, want_w=weighted)
    close_grad(gs[0], ey, 1e-5)
    if weighted:
        close_grad(gs[1], ew, 1e-5)


# --- cancelling sums across merge levels ---------------------------------------------------------


@pytest.mark.parametrize("big", [1e3, 1e6, 1e12])
@pytest.mark.parametrize("n", [100_000, 5_000_000])
def test_cancelling_sums_merged(n: int, big: float) -> None:
    # reference tests/test_cuda.py:243-265 (its n = 100000 reaches merged chunks): per 64
    # elements, 32 of +big, one of -32 big, then small near-collinear values
    geo = _ext.geometry(1, n, False)
    say(f"cancelling sums n={n} big={big:g} geometry {geo}")
    assert geo["levels"] >= 2
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


def test_float32_store_rounding_keeps_the_fit_monotone() -> None:
    # Float32 rows keep hull sums rounded to float64 between merge levels; where points are
    # nearly collinear the rounding can leave a final hull slightly non-convex in those values,
    # and the check after the last merge removes such vertices (on this row, about 3000 of them in
    # one pass). The fit must stay monotone and within float32 accuracy of the exact fit.
    n = 4_000_000
    say(f"float32 store rounding: one weighted near-collinear row of {n}")
    rng = np.random.default_rng(7)
    rng.standard_normal(1_000_000)  # (the draws before this row in the search that found it)
    rng.random(1_000_000)
    i = np.arange(n, dtype=np.float64)
    y = (1e3 + 1e-3 * i + 1e-7 * rng.standard_normal(n)).astype(np.float32)[None]
    w = np.exp(8 * rng.random(n)).astype(np.float32)[None]
    assert _ext.geometry(1, n, True)["levels"] >= 2
    got, starts = gpu_fit(y, w)
    assert (np.diff(got, axis=1) >= 0).all()
    want, _ = oracle.pava(y.astype(np.float64), w.astype(np.float64))
    assert float(np.abs(got - want).max()) <= tolerance(y)
    g = rng.standard_normal(n).astype(np.float32)[None]
    fit, (gy, gw) = autograd(y, w, g)
    np.testing.assert_array_equal(fit, got)
    ey, ew = oracle.block_grad(starts, g.astype(np.float64), w.astype(np.float64), y.astype(np.float64),
                               fit.astype(np.float64), want_w=True)
    close_grad(gy, ey, 1e-5)
    close_grad(gw, ew, 1e-5)


# (batch, n, merge levels): rows through two merge levels, fewer or more than 256 of them, and
# rows whose final hulls the span kernel makes, one row a wave (merged by reference to the span
# hulls, which do not fit the wave's LDS) or two rows a wave (the overflowing waves' rows merged
# by the first merge launch)
STORE_ROUNDING_SHAPES = [(80, 100_000, 2), (300, 40_000, 2), (1100, 20_000, 2), (600, 10_000, 1), (3000, 1000, 1)]


@pytest.mark.parametrize(("batch", "n", "levels"), STORE_ROUNDING_SHAPES)
def test_float32_store_rounding_many_rows(batch: int, n: int, levels: int) -> None:
    # The same near-collinear data over many rows: with 256 rows or more the last merge launch's
    # workgroups (256 and 64 threads here, one a row) make their rows' hulls convex in the stored
    # values themselves, and so do the span kernel's waves where they make the final hulls; with
    # fewer rows of two levels, the check and repair launches do.
    say(f"float32 store rounding: {batch} weighted near-collinear rows of {n}")
    rng = np.random.default_rng(11)
    i = np.arange(n, dtype=np.float64)
    y = (1e3 + 1e-3 * i + 1e-7 * rng.standard_normal((batch, n))).astype(np.float32)
    w = np.exp(8 * rng.random((batch, n))).astype(np.float32)
    assert _ext.geometry(batch, n, True)["levels"] == levels
    got, starts = gpu_fit(y, w)
    assert (np.diff(got, axis=1) >= 0).all()
    want, _ = oracle.pava(y.astype(np.float64), w.astype(np.float64))
    assert float(np.abs(got - want).max()) <= tolerance(y)


@pytest.mark.parametrize(("batch", "n"), [(1, 4_000_000), (300, 40_000), (600, 10_000), (3000, 1000), (9000, 100)])
def test_float32_repair_chain_gives_the_same_hulls(batch: int, n: int) -> None:
    # The repair finishes a row with a sequential monotone chain after a cascade of removals
    # longer than its pass limit; the REPAIR_CHAIN hint takes that form at once (through the
    # check and repair launches for one row, in the last merge launch for 300, in the span
    # kernel's waves or the first merge launch for 600 x 10000 (one row a wave), 3000 x 1000 (two
    # rows a wave) and 9000 x 100 (eight)). Both keep the lower hull of the stored points, so fit
    # and partition are the passes' bit for bit.
    say(f"float32 repair chain: {batch} weighted near-collinear rows of {n}")
    rng = np.random.default_rng(13)
    i = np.arange(n, dtype=np.float64)
    y = torch.from_numpy((1e3 + 1e-3 * i + 1e-7 * rng.standard_normal((batch, n))).astype(np.float32)).cuda()
    w = torch.from_numpy(np.exp(8 * rng.random((batch, n))).astype(np.float32)).cuda()
    a, sa, bad_a, _ = _ext.fit(y, w, True, True, True)
    b, sb, bad_b, _ = _ext.fit(y, w, True, True, True, hints=_ext.REPAIR_CHAIN)
    assert bad_a is False and bad_b is False
    assert torch.equal(a, b)
    assert torch.equal(_ext.starts_to_bool(sa, batch, n), _ext.starts_to_bool(sb, batch, n))
    assert bool((b[:, 1:] >= b[:, :-1]).all())


# --- exact ties with inexact cross products ------------------------------------------------------

# (batch, n): short rows, one row a lane ("packed"), several rows a wave, one row a wave, and rows
# whose spans go through one, two and three merge launches
TIE_SHAPES = [(5, 6), (5, 30), (9000, 60), (300, 600), (3, 3000), (1, 100_002), (1, 3 * 2**20)]


@pytest.mark.parametrize(("batch", "n"), TIE_SHAPES)
def test_exact_ties_inexact_products(batch: int, n: int) -> None:
    # Three patterns, each pooling into ONE block in exact arithmetic (every block [a, 0, 0] has
    # the same mean): the sums are exact, but the cross products of the hull tests are not
    # representable, so a test that counts a product's rounding error twice (an fma contracted
    # into the exact predicate) splits the row.
    #  - float64, unweighted, a = 1 + 2^-30: sums k a exact, products k a m inexact;
    #  - float64 decreasing, the pattern reversed;
    #  - float32 weighted, y in {0, 1}, w = 1 + 2^-23: products k m w^2 inexact.
    say(f"exact ties, inexact products: {batch} x {n}")
    a = 1 + 2.0**-30
    cases = [
        (np.tile([a, 0.0, 0.0], (batch, n // 3)), None, True),
        (np.tile([0.0, 0.0, a], (batch, n // 3)), None, False),
        (np.tile(np.float32([1, 0, 0]), (batch, n // 3)), np.full((batch, n // 3 * 3), np.float32(1 + 2.0**-23)), True),
    ]
    rng = np.random.default_rng(n)
    for y, w, inc in cases:
        want, want_starts = oracle.pava(y, w, increasing=inc, acc="f64")
        assert int(want_starts.sum()) == batch  # one block a row
        got, starts = gpu_fit(y, w, inc)
        assert float(np.abs(got - want).max()) <= tolerance(y)
        np.testing.assert_array_equal(starts, want_starts)
        g = rng.standard_normal(y.shape).astype(y.dtype)
        _, gs = autograd(y, w, g, increasing=inc)
        w64 = None if w is None else w.astype(np.float64)
        ey, _ = oracle.block_grad(want_starts, g.astype(np.float64), w64)
        close_grad(gs[0], ey, 1e-12 if y.dtype == np.float64 else 1e-5)


def test_advisor_example_short_row() -> None:
    # float64 [0.1, 0, 0, 0.1, 0, 0]: both halves have dS = 0.1, dW = 3, an exact tie whose
    # product 0.3 is inexact; the reference's PAVA pools all six (pava.h:46-55)
    say("exact tie [0.1, 0, 0, 0.1, 0, 0]")
    y = np.array([[0.1, 0, 0, 0.1, 0, 0]])
    got, starts = gpu_fit(y)
    np.testing.assert_array_equal(starts, [[1, 0, 0, 0, 0, 0]])
    _, (gy,) = autograd(y, None, np.eye(6)[:1])
    np.testing.assert_allclose(gy, np.full((1, 6), 1 / 6), rtol=1e-15)


# --- the golden fixtures on the span path -------------------------------------------------------


def test_scipy_golden_vectors_span_path() -> None:
    say("scipy golden vectors, rows of 33-60")
    d = np.load(GOLDEN / "scipy_fits.npz", allow_pickle=False)
    off, bo = d["offsets"], d["block_offsets"]
    seen = 0
    for k in range(len(off) - 1):
        sl = slice(off[k], off[k + 1])
        if off[k + 1] - off[k] <= 32:
            continue
        seen += 1
        y = d["y"][sl][None]
        w = d["w"][sl][None] if d["weighted"][k] else None
        got, starts = gpu_fit(y, w, bool(d["increasing"][k]))
        np.testing.assert_allclose(got[0], d["x"][sl], rtol=1e-12, atol=1e-9)
        blocks = np.concatenate([np.flatnonzero(starts[0]), [y.shape[1]]])
        np.testing.assert_array_equal(blocks, d["blocks"][bo[k] : bo[k + 1]])
    assert seen > 100


def test_scipy_long_golden_span_path() -> None:
    say("scipy golden vectors, rows of 20000")
    data = np.load(GOLDEN / "scipy_long.npz", allow_pickle=False)
    for y, x in zip(data["y"], data["x"]):
        got, _ = gpu_fit(y[None], with_starts=False)
        np.testing.assert_allclose(got[0], x, rtol=1e-12, atol=1e-9)
