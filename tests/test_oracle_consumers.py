"""The oracle of the consumers either side of the fit, pinned on the CPU (no GPU): soft ranks by
closed forms, limits, an invariant and finite differences; isotonic calibration by scikit-learn's
IsotonicRegression (committed golden vectors) and by np.interp; planted mistakes fail them."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def hard_ranks(x: np.ndarray) -> np.ndarray:
    return np.argsort(np.argsort(x, axis=-1, kind="stable"), axis=-1, kind="stable") + 1.0


# --- soft rank ------------------------------------------------------------------------------------


def test_soft_rank_two_elements_closed_form() -> None:
    # x = (a, b), a > b: while (a - b) / eps < 1 the dual pools both entries, so the ranks are
    # 1.5 +- (a - b) / (2 eps); beyond, the hard ranks (2, 1)
    for a, b, eps in ((0.3, 0.1, 1.0), (2.0, -1.0, 10.0), (0.5, 0.4, 0.05)):
        r, _ = oracle.soft_rank(np.array([[a, b]]), eps)
        d = (a - b) / eps
        want = [1.5 + d / 2, 1.5 - d / 2] if d < 1 else [2.0, 1.0]
        np.testing.assert_allclose(r[0], want, rtol=0, atol=1e-15)


def test_soft_rank_limits_and_sum() -> None:
    rng = np.random.default_rng(0)
    x = rng.standard_normal((20, 37))
    np.testing.assert_array_equal(oracle.soft_rank(x, 1e-9)[0], hard_ranks(x))
    np.testing.assert_allclose(oracle.soft_rank(x, 1e9)[0], 19.0, atol=1e-6)
    for eps in (0.1, 1.0, 5.0):
        r, _ = oracle.soft_rank(x, eps)
        np.testing.assert_allclose(r.sum(-1), 37 * 38 / 2, rtol=1e-13)  # the permutahedron's sum
        # order-preserving: a larger entry never gets a smaller soft rank
        o = np.argsort(x, axis=-1)
        assert (np.diff(np.take_along_axis(r, o, -1), axis=-1) >= -1e-12).all()


def test_soft_rank_vjp_matches_finite_differences() -> None:
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 9))
    g = rng.standard_normal((3, 9))
    for eps in (0.3, 2.0):
        vjp = oracle.soft_rank_vjp(x, eps, g)
        h = 1e-6
        num = np.zeros_like(x)
        for i in range(x.shape[1]):
            d = np.zeros_like(x)
            d[:, i] = h
            num[:, i] = ((oracle.soft_rank(x + d, eps)[0] - oracle.soft_rank(x - d, eps)[0]) * g).sum(-1) / (2 * h)
        np.testing.assert_allclose(vjp, num, rtol=1e-6, atol=1e-7)


def test_soft_rank_catches_a_planted_mistake() -> None:
    # the weights in increasing order instead of (n, ..., 1) breaks the hard-rank limit
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 6))
    perm = np.argsort(-x / 1e-9, axis=-1, kind="stable")
    s = np.take_along_axis(x / 1e-9, perm, -1)
    wrong, _ = oracle.pava(s - np.arange(1, 7, dtype=np.float64), increasing=False, acc="f64")
    r = np.empty_like(s)
    np.put_along_axis(r, perm, s - wrong, -1)
    assert not np.allclose(r, hard_ranks(x))


# --- calibration ----------------------------------------------------------------------------------


def golden_calib():
    d = np.load(GOLDEN / "sklearn_calib.npz", allow_pickle=False)
    off, qoff = d["offsets"], d["q_offsets"]
    for k in range(len(off) - 1):
        sl, ql = slice(off[k], off[k + 1]), slice(qoff[k], qoff[k + 1])
        w = d["w"][sl] if d["weighted"][k] else None
        yield d["x"][sl], d["y"][sl], w, bool(d["increasing"][k]), d["q"][ql], d["pred"][ql]


def test_calibration_matches_sklearn_golden() -> None:
    seen = 0
    for x, y, w, inc, q, pred in golden_calib():
        xp, fp = oracle.calibration_fit(x, y, w, increasing=inc)
        np.testing.assert_allclose(oracle.interp(q, xp, fp), pred, rtol=1e-12, atol=1e-12)
        seen += 1
    assert seen >= 100


def test_calibration_catches_a_planted_mistake() -> None:
    # pooling ties without their weights (plain means of the unique keys' values) changes the
    # fit wherever a weighted tie exists
    for x, y, w, inc, q, pred in golden_calib():
        if w is None or len(np.unique(x)) == len(x):
            continue
        xp, first = np.unique(np.sort(x), return_index=True)
        order = np.argsort(x, kind="stable")
        means = np.add.reduceat(y[order], first) / np.diff(np.append(first, len(x)))
        fit, _ = oracle.pava(means[None], np.diff(np.append(first, len(x)))[None].astype(float), increasing=inc)
        if not np.allclose(oracle.interp(q, xp, fit[0]), pred, rtol=1e-12, atol=1e-12):
            return
    pytest.fail("no golden problem caught unweighted pooling")


def test_interp_matches_numpy() -> None:
    rng = np.random.default_rng(3)
    xp = np.sort(rng.standard_normal(50))
    fp = np.cumsum(rng.random(50))
    x = np.concatenate([rng.standard_normal(1000) * 2, xp, [np.nan]])
    got = oracle.interp(x, xp, fp)
    np.testing.assert_allclose(got[:-1], np.interp(x[:-1], xp, fp), rtol=1e-14, atol=1e-14)
    assert np.isnan(got[-1])
    # one knot: constant
    np.testing.assert_array_equal(oracle.interp(np.array([-1.0, 0.0, 5.0]), np.array([0.5]), np.array([2.0])), 2.0)


def test_calibration_offsets_keep_segments_apart() -> None:
    # two segments fitted in one call (reference calibrate.py:171-187): the offsets keep them
    # from pooling across, so each equals its own fit
    rng = np.random.default_rng(4)
    x1, x2 = rng.random(40), rng.random(40) + 5.0
    y1, y2 = rng.random(40) * 3.0, rng.random(40) - 2.0
    xp, fp = oracle.calibration_fit(np.r_[x1, x2], np.r_[y1, y2], offset=np.r_[np.zeros(40), np.full(40, 1e6)])
    xa, fa = oracle.calibration_fit(x1, y1)
    xb, fb = oracle.calibration_fit(x2, y2)
    np.testing.assert_allclose(fp, np.r_[fa, fb], rtol=0, atol=1e-9)
    np.testing.assert_array_equal(xp, np.r_[xa, xb])


# --- ragged rows ----------------------------------------------------------------------------------


def test_pava_ragged_is_each_row_on_its_own() -> None:
    # grouping rows by length is the per-row fit; rows never pool across (each starts a block)
    rng = np.random.default_rng(7)
    ln = np.r_[rng.integers(0, 12, 300), [0, 1, 50]]
    off = np.r_[0, np.cumsum(ln)]
    y = rng.standard_normal(off[-1])
    w = rng.random(off[-1]) + 0.1
    for ww in (None, w):
        fit, starts = oracle.pava_ragged(y, off, ww, increasing=False)
        for r in range(len(ln)):
            sl = slice(off[r], off[r + 1])
            if ln[r] == 0:
                continue
            f, s = oracle.pava(y[sl][None], None if ww is None else ww[sl][None], increasing=False, acc="f64")
            np.testing.assert_array_equal(fit[sl], f[0])
            np.testing.assert_array_equal(starts[sl], s[0])
            assert starts[off[r]] == 1
    # one fit of the packed values as a single row pools across row ends
    whole, _ = oracle.pava(y[None], increasing=False, acc="f64")
    assert not np.allclose(whole[0], oracle.pava_ragged(y, off, increasing=False)[0])
