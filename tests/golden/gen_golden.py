"""Writes the golden vectors under tests/golden/ from scipy and scikit-learn, the third-party
solvers the reference's own tests check against (reference tests/test_isotonic.py:14-15,
30-37, 66-72).

    python tests/golden/gen_golden.py

Inputs mimic the reference's hypothesis strategies (tests/test_isotonic.py:19-27): rows of
0..60 values drawn from U(-1e3, 1e3) mixed with exact 0, 1 and -1 (so that ties occur),
unweighted or with weights in U(1e-3, 1e3), both directions. Ragged rows are stored
concatenated with an offsets array. Everything is float64 and loads with
``numpy.load(allow_pickle=False)``.

- scipy_fits.npz: ``scipy.optimize.isotonic_regression`` fit ``x`` and its ``blocks``
  (block start indices, ending with n) for every problem.
- sklearn_clip.npz: ``sklearn.isotonic.isotonic_regression`` with ``y_min``/``y_max`` (a NaN
  bound means "not given").
- scipy_long.npz: long structured rows of the reference's tests/test_isotonic.py:103-117
  patterns (at n = 20000), inputs ``y`` and their scipy fits ``x``.
- sklearn_calib.npz: ``sklearn.isotonic.IsotonicRegression`` fit on keys with ties (pooled
  into their weighted mean, as the reference's calibration example does,
  examples/ctr_calibration/calibrate.py:171-187) and its predictions (``out_of_bounds="clip"``,
  piecewise linear) at new points.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
from scipy.optimize import isotonic_regression as scipy_isotonic
from sklearn.isotonic import isotonic_regression as sklearn_isotonic

HERE = Path(__file__).resolve().parent


def draw_problem(rng: np.random.Generator, max_len: int = 60) -> tuple[np.ndarray, np.ndarray | None]:
    n = int(rng.integers(0, max_len + 1))
    y = rng.uniform(-1e3, 1e3, n)
    special = rng.random(n) < 0.3
    y[special] = rng.choice([0.0, 1.0, -1.0], int(special.sum()))
    if rng.random() < 0.1:  # a few rows of integers, where ties are exact
        y = rng.integers(-3, 4, n).astype(np.float64)
    w = None if rng.random() < 0.5 else rng.uniform(1e-3, 1e3, n)
    return y, w


def pack(rows: list[np.ndarray]) -> tuple[np.ndarray, np.ndarray]:
    offsets = np.zeros(len(rows) + 1, dtype=np.int64)
    offsets[1:] = np.cumsum([len(r) for r in rows])
    data = np.concatenate(rows) if rows else np.zeros(0)
    return data.astype(np.float64), offsets


def scipy_fits(count: int = 600, seed: int = 1) -> None:
    rng = np.random.default_rng(seed)
    ys, ws, xs, blocks, inc, weighted = [], [], [], [], [], []
    for k in range(count):
        y, w = draw_problem(rng)
        increasing = bool(k % 2 == 0)
        res = scipy_isotonic(y, weights=w, increasing=increasing)
        ys.append(y)
        ws.append(np.ones_like(y) if w is None else w)
        weighted.append(w is not None)
        xs.append(np.array(res.x, dtype=np.float64).copy())
        blocks.append(np.asarray(res.blocks, dtype=np.float64))  # in the row's own order
        inc.append(increasing)
    y, off = pack(ys)
    w, _ = pack(ws)
    x, _ = pack(xs)
    b, boff = pack(blocks)
    np.savez_compressed(
        HERE / "scipy_fits.npz",
        y=y, w=w, x=x, offsets=off, blocks=b.astype(np.int64), block_offsets=boff,
        increasing=np.array(inc), weighted=np.array(weighted),
    )


def sklearn_clip(count: int = 300, seed: int = 2) -> None:
    rng = np.random.default_rng(seed)
    ys, ws, xs, lo, hi, inc, weighted = [], [], [], [], [], [], []
    while len(ys) < count:
        y, w = draw_problem(rng)
        if len(y) == 0:
            continue  # sklearn rejects empty input (reference tests/test_isotonic.py:65)
        y_min = None if rng.random() < 0.3 else float(rng.uniform(-1e3, 1e3))
        y_max = None if rng.random() < 0.3 else float(rng.uniform(-1e3, 1e3))
        increasing = bool(rng.random() < 0.5)
        x = sklearn_isotonic(y, sample_weight=w, y_min=y_min, y_max=y_max, increasing=increasing)
        ys.append(y)
        ws.append(np.ones_like(y) if w is None else w)
        weighted.append(w is not None)
        xs.append(np.array(x, dtype=np.float64).copy())
        lo.append(np.nan if y_min is None else y_min)
        hi.append(np.nan if y_max is None else y_max)
        inc.append(increasing)
    y, off = pack(ys)
    w, _ = pack(ws)
    x, _ = pack(xs)
    np.savez_compressed(
        HERE / "sklearn_clip.npz",
        y=y, w=w, x=x, offsets=off, y_min=np.array(lo), y_max=np.array(hi),
        increasing=np.array(inc), weighted=np.array(weighted),
    )


def sklearn_calib(count: int = 120, seed: int = 3) -> None:
    """Isotonic calibration (sklearn's IsotonicRegression fit, then predict with
    out_of_bounds="clip"): keys with ties (rounded), labels 0/1 or real values, optional
    weights, both directions; predictions at points inside, at and beyond the knots."""
    from sklearn.isotonic import IsotonicRegression

    rng = np.random.default_rng(seed)
    keys, ys, ws, qs, ps, inc, weighted = [], [], [], [], [], [], []
    for k in range(count):
        n = int(rng.integers(1, 200))
        x = np.round(rng.normal(0.0, 1.0, n), int(rng.integers(1, 4)))
        if k % 3 == 0:
            y = (rng.random(n) < 1 / (1 + np.exp(-2 * x))).astype(np.float64)
        else:
            y = np.round(x + rng.normal(0.0, 0.7, n), 3)
        w = None if k % 2 == 0 else rng.uniform(0.1, 5.0, n)
        increasing = bool(k % 4 != 1)
        model = IsotonicRegression(increasing=increasing, out_of_bounds="clip").fit(x, y, sample_weight=w)
        q = np.concatenate([rng.normal(0.0, 1.5, 50), np.unique(x), [x.min() - 1, x.max() + 1]])
        keys.append(x)
        ys.append(y)
        ws.append(np.ones_like(y) if w is None else w)
        weighted.append(w is not None)
        qs.append(q)
        ps.append(np.asarray(model.predict(q), dtype=np.float64))
        inc.append(increasing)
    x, off = pack(keys)
    y, _ = pack(ys)
    w, _ = pack(ws)
    q, qoff = pack(qs)
    pr, _ = pack(ps)
    np.savez_compressed(
        HERE / "sklearn_calib.npz",
        x=x, y=y, w=w, offsets=off, q=q, pred=pr, q_offsets=qoff,
        increasing=np.array(inc), weighted=np.array(weighted),
    )


def long_patterns(n: int = 20000) -> np.ndarray:
    i = np.arange(n, dtype=np.float64)
    return np.stack([i, -i, (-1.0) ** i * i, np.full(n, 2.5), i % 97 - i / 1000])


def scipy_long() -> None:
    ys = long_patterns()
    xs = np.stack([scipy_isotonic(y).x for y in ys])
    np.savez_compressed(
        HERE / "scipy_long.npz",
        names=np.array(["increasing", "decreasing", "alternating", "constant", "sawtooth"]),
        y=ys,
        x=xs,
    )


if __name__ == "__main__":
    scipy_fits()
    sklearn_clip()
    scipy_long()
    sklearn_calib()
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)
