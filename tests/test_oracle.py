"""The CPU oracle (oracle/ti_oracle.c) pinned before anything is compared with it:

- against the third-party solvers the reference's own tests use (scipy's
  isotonic_regression for fits and blocks, scikit-learn's for clipping), through the golden
  vectors committed under tests/golden/ (reference tests/test_isotonic.py:30-81, 103-117);
- against the reference's own pava.h compiled in place (oracle/_ref), bit for bit, where it
  was built;
- against what the mathematics fixes: brute force over all partitions on small rows, closed
  forms, the KKT certificate (reference paper/accuracy.py:72-81), exact rational arithmetic
  for the long-double mode, finite differences for the backward;
- and with planted mistakes, to show that these checks catch the plausible ones.
"""

from __future__ import annotations

import itertools
import math
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def blocks_of(starts: np.ndarray) -> np.ndarray:
    n = len(starts)
    return np.concatenate([np.flatnonzero(starts), [n]]).astype(np.int64)


def golden_problems(name: str):
    d = np.load(GOLDEN / name, allow_pickle=False)
    off = d["offsets"]
    for k in range(len(off) - 1):
        sl = slice(off[k], off[k + 1])
        yield k, d, sl


def clamp(x: np.ndarray, lo: float, hi: float) -> np.ndarray:
    """torch.clamp / numpy.clip semantics (upper bound applied last)."""
    out = x.copy()
    if not math.isnan(lo):
        out = np.where(out < lo, lo, out)
    if not math.isnan(hi):
        out = np.where(out > hi, hi, out)
    return out


# --- golden vectors ----------------------------------------------------------------------


def test_matches_scipy_golden_fits_and_blocks() -> None:
    d = np.load(GOLDEN / "scipy_fits.npz", allow_pickle=False)
    off, boff = d["offsets"], d["block_offsets"]
    checked = 0
    for k in range(len(off) - 1):
        y = d["y"][off[k] : off[k + 1]]
        if len(y) == 0:
            continue
        w = d["w"][off[k] : off[k + 1]] if d["weighted"][k] else None
        inc = bool(d["increasing"][k])
        fit, starts = oracle.pava(y, w, increasing=inc)
        np.testing.assert_allclose(fit, d["x"][off[k] : off[k + 1]], rtol=1e-12, atol=1e-9)
        np.testing.assert_array_equal(blocks_of(starts), d["blocks"][boff[k] : boff[k + 1]])
        checked += 1
    assert checked > 500


def test_matches_sklearn_golden_clip() -> None:
    d = np.load(GOLDEN / "sklearn_clip.npz", allow_pickle=False)
    off = d["offsets"]
    for k in range(len(off) - 1):
        y = d["y"][off[k] : off[k + 1]]
        w = d["w"][off[k] : off[k + 1]] if d["weighted"][k] else None
        fit, _ = oracle.pava(y, w, increasing=bool(d["increasing"][k]))
        got = clamp(fit, float(d["y_min"][k]), float(d["y_max"][k]))
        np.testing.assert_allclose(got, d["x"][off[k] : off[k + 1]], rtol=1e-12, atol=1e-9)


def test_matches_scipy_long_patterns() -> None:
    data = np.load(GOLDEN / "scipy_long.npz", allow_pickle=False)
    for y, x in zip(data["y"], data["x"]):
        fit, _ = oracle.pava(y)
        np.testing.assert_allclose(fit, x, rtol=1e-12, atol=1e-9)


# --- the reference's own solver, compiled in place ----------------------------------------

needs_ref = pytest.mark.skipif(oracle.ref_lib() is None, reason="reference pava.h not built here")


@needs_ref
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("increasing", [True, False])
def test_bit_identical_to_reference_pava(dtype: type, weighted: bool, increasing: bool) -> None:
    rng = np.random.default_rng(7)
    y = (np.linspace(0, 3, 333) + rng.standard_normal((64, 333))).astype(dtype)
    y[5] = np.round(y[5])  # exact ties
    y[9] = 1.0  # constant
    y[11, 17] = np.nan
    w = (rng.random((64, 333)) + 0.1).astype(dtype) if weighted else None
    a, sa = oracle.pava(y, w, increasing=increasing)
    b, sb = oracle.pava(y, w, increasing=increasing, impl="reference")
    np.testing.assert_array_equal(a.view(np.uint8), b.view(np.uint8))
    np.testing.assert_array_equal(sa, sb)


# --- what the mathematics fixes ------------------------------------------------------------


def brute_force(y: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Least-squares monotone fit by enumerating every partition into contiguous blocks whose
    weighted means do not decrease (the optimum is one of them)."""
    n = len(y)
    best, best_obj = None, math.inf
    for cuts in itertools.product([0, 1], repeat=n - 1):
        edges = [0] + [i + 1 for i, c in enumerate(cuts) if c] + [n]
        means = [np.average(y[a:b], weights=w[a:b]) for a, b in itertools.pairwise(edges)]
        if any(m2 < m1 for m1, m2 in itertools.pairwise(means)):
            continue
        fit = np.concatenate([np.full(b - a, m) for (a, b), m in zip(itertools.pairwise(edges), means)])
        obj = float(np.sum(w * (fit - y) ** 2))
        if obj < best_obj:
            best, best_obj = fit, obj
    assert best is not None
    return best


def test_matches_brute_force_on_small_rows() -> None:
    rng = np.random.default_rng(3)
    for trial in range(300):
        n = int(rng.integers(1, 9))
        y = rng.standard_normal(n) if trial % 3 else rng.integers(-2, 3, n).astype(float)
        w = rng.random(n) + 0.1 if trial % 2 else np.ones(n)
        fit, _ = oracle.pava(y, w)
        np.testing.assert_allclose(fit, brute_force(y, w), rtol=1e-12, atol=1e-12)


def kkt_violation(y: np.ndarray, w: np.ndarray, fit: np.ndarray) -> float:
    """Largest violation of the optimality conditions, relative to sum w|y| (reference
    paper/accuracy.py:72-81): lambda_i = -2 sum_{j<=i} w_j (fit_j - y_j) >= 0, lambda_{n-1} = 0,
    lambda_i = 0 where the fit steps up."""
    lam = -2 * np.cumsum(w * (fit - y))
    scale = 2 * float(np.sum(w * np.abs(y))) + 1e-300
    dual = float(np.max(np.clip(-lam, 0, None)))
    end = abs(float(lam[-1]))
    steps = fit[1:] > fit[:-1]
    slack = float(np.max(np.abs(lam[:-1][steps]))) if steps.any() else 0.0
    return max(dual, end, slack) / scale


def test_kkt_certificate() -> None:
    rng = np.random.default_rng(4)
    for n in (1, 2, 17, 500, 5000):
        y = np.linspace(0, 3, n) + rng.standard_normal(n)
        w = rng.random(n) + 0.1
        fit, _ = oracle.pava(y, w)
        assert kkt_violation(y, w, fit) < 1e-12
        assert np.all(np.diff(fit) >= 0)


def test_closed_forms() -> None:
    rng = np.random.default_rng(5)
    i = np.arange(50, dtype=np.float64)
    w = rng.random(50) + 0.1
    fit, starts = oracle.pava(i)  # increasing data is its own fit, every element a block
    np.testing.assert_array_equal(fit, i)
    assert starts.all()
    fit, starts = oracle.pava(i, w)  # weighted: each mean is w*y/w, y up to one rounding
    np.testing.assert_allclose(fit, i, rtol=2**-52)
    assert starts.all()
    fit, starts = oracle.pava(-i, w)  # decreasing data is one block at the weighted mean
    np.testing.assert_allclose(fit, np.full(50, np.average(-i, weights=w)), rtol=1e-14)
    assert starts[0] == 1 and not starts[1:].any()
    fit, starts = oracle.pava(np.full(50, 2.5))  # equal means pool: one block
    assert np.all(fit == 2.5) and starts.sum() == 1
    # the reference's known answers (tests/test_isotonic.py:127-140)
    np.testing.assert_array_equal(oracle.pava(np.array([3.0, 1.0, 2.0, 5.0]))[0], [2, 2, 2, 5])
    np.testing.assert_array_equal(oracle.pava(np.array([3.0, 1.0, 2.0]))[0], [2, 2, 2])
    # decreasing is minus the increasing fit of -y, same partition
    y = rng.standard_normal(40)
    a, sa = oracle.pava(y, w[:40], increasing=False)
    b, sb = oracle.pava(-y, w[:40])
    np.testing.assert_array_equal(a, -b)
    np.testing.assert_array_equal(sa, sb)


def test_nan_makes_only_its_row_nan() -> None:
    y = np.array([[3.0, np.nan, 2.0], [3.0, 1.0, 2.0]])
    fit, starts = oracle.pava(y)
    assert np.isnan(fit[0]).all()
    np.testing.assert_array_equal(starts[0], [1, 0, 0])
    np.testing.assert_array_equal(fit[1], [2, 2, 2])


def exact_pava(y: list[int], w: list[int]) -> list[int]:
    """PAVA in exact rational arithmetic; returns block starts."""
    stack: list[tuple[int, Fraction, Fraction]] = []
    for i, (yi, wi) in enumerate(zip(y, w)):
        stack.append((i, Fraction(wi), Fraction(wi * yi)))
        while len(stack) > 1 and stack[-2][2] / stack[-2][1] >= stack[-1][2] / stack[-1][1]:
            s, wb, tb = stack.pop()
            a, wa, ta = stack.pop()
            stack.append((a, wa + wb, ta + tb))
    return [s for s, _, _ in stack]


def test_long_double_mode_is_exact_on_integer_data() -> None:
    rng = np.random.default_rng(6)
    for _ in range(50):
        n = int(rng.integers(1, 300))
        y = (rng.random(n) < 1 / (1 + np.exp(-np.linspace(-3, 3, n)))).astype(int)
        w = rng.integers(1, 6, n)
        _, starts = oracle.pava(y.astype(float), w.astype(float), acc="f64x")
        assert list(np.flatnonzero(starts)) == exact_pava(list(y), list(w))


def test_backward_matches_finite_differences() -> None:
    rng = np.random.default_rng(8)
    for _ in range(20):
        n = int(rng.integers(2, 30))
        y = rng.standard_normal(n) * 3
        w = rng.random(n) + 0.1
        g = rng.standard_normal(n)
        fit, starts = oracle.pava(y, w)
        gy, gw = oracle.block_grad(starts, g, w, y, fit, want_w=True)
        eps = 1e-7
        for j in range(n):
            for arr, got in ((y, gy), (w, gw)):
                hi, lo = arr.copy(), arr.copy()
                hi[j] += eps
                lo[j] -= eps
                fy = oracle.pava(hi if arr is y else y, hi if arr is w else w)[0]
                fl = oracle.pava(lo if arr is y else y, lo if arr is w else w)[0]
                np.testing.assert_allclose(got[j], np.dot(g, fy - fl) / (2 * eps), rtol=1e-5, atol=1e-6)


def test_backward_block_average_kat() -> None:
    # reference tests/test_grad.py:32-37: [3, 1, 2] is one block; grad of sum(fit * c) is 3s.
    y = np.array([3.0, 1.0, 2.0])
    fit, starts = oracle.pava(y)
    gy, _ = oracle.block_grad(starts, np.array([1.0, 2.0, 6.0]))
    np.testing.assert_array_equal(gy, [3.0, 3.0, 3.0])


# --- planted mistakes: the checks above must catch them ------------------------------------


def python_pava(y: np.ndarray, w: np.ndarray, strict: bool = False, drop_weights: bool = False) -> np.ndarray:
    """A pure-Python PAVA used only to plant mistakes: ``strict`` pools only on a strictly
    larger previous mean (wrong on ties), ``drop_weights`` ignores w."""
    ww = np.ones_like(w) if drop_weights else w
    st: list[list[float]] = []
    for i in range(len(y)):
        st.append([i, ww[i], ww[i] * y[i]])
        while len(st) > 1:
            a, b = st[-2], st[-1]
            viol = a[2] * b[1] > b[2] * a[1] if strict else a[2] * b[1] >= b[2] * a[1]
            if not viol:
                break
            st.pop()
            a[1] += b[1]
            a[2] += b[2]
    out = np.empty(len(y))
    for k, (s, wt, tot) in enumerate(st):
        e = st[k + 1][0] if k + 1 < len(st) else len(y)
        out[int(s) : int(e)] = tot / wt
    return out


def planted_failures(mutation: dict[str, bool]) -> int:
    d = np.load(GOLDEN / "scipy_fits.npz", allow_pickle=False)
    off = d["offsets"]
    bad = 0
    for k in range(len(off) - 1):
        y = d["y"][off[k] : off[k + 1]]
        if len(y) == 0 or not d["increasing"][k]:
            continue
        w = d["w"][off[k] : off[k + 1]]
        got = python_pava(y, w, **mutation)
        if not np.allclose(got, d["x"][off[k] : off[k + 1]], rtol=1e-12, atol=1e-9):
            bad += 1
    return bad


def test_planted_mistakes_are_caught() -> None:
    assert planted_failures({}) == 0  # the unmutated restatement passes
    assert planted_failures({"drop_weights": True}) > 50  # a dropped term
    # Strict pooling (">" for ">=") leaves the fit unchanged on exact ties but splits their
    # blocks: the golden block lists catch it, while the correct rule matches them all.
    d = np.load(GOLDEN / "scipy_fits.npz", allow_pickle=False)
    off, boff = d["offsets"], d["block_offsets"]
    strict_bad = correct_bad = 0
    for k in range(len(off) - 1):
        y, w = d["y"][off[k] : off[k + 1]], d["w"][off[k] : off[k + 1]]
        if len(y) == 0 or not d["increasing"][k]:
            continue
        want = list(d["blocks"][boff[k] : boff[k + 1]])
        strict_bad += _blocks(y, w, strict=True) != want
        correct_bad += _blocks(y, w, strict=False) != want
    assert correct_bad == 0
    assert strict_bad > 0


def _blocks(y: np.ndarray, w: np.ndarray, strict: bool) -> list[int]:
    st: list[list[float]] = []
    for i in range(len(y)):
        st.append([i, w[i], w[i] * y[i]])
        while len(st) > 1 and (
            st[-2][2] * st[-1][1] > st[-1][2] * st[-2][1]
            if strict
            else st[-2][2] * st[-1][1] >= st[-1][2] * st[-2][1]
        ):
            b = st.pop()
            st[-1][1] += b[1]
            st[-1][2] += b[2]
    return [int(s[0]) for s in st] + [len(y)]
