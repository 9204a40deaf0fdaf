"""TEST INFRASTRUCTURE ONLY: the CPU oracle for the isotonic path, and the reference's own
CPU solver where it was built.

Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg may import this
package, and only as the checker (or the timed CPU baseline) - never as the thing measured on
the GPU. The product package ``torchisotonic_amd`` never imports it.

- ``libti_oracle.so`` (built from ``ti_oracle.c``): a plain-C restatement of the reference CPU
  path (reference ``src/torchisotonic/csrc/pava.h:16-69``, ``ops.cpp:17-41``,
  ``_api.py:92-134``), accumulating in float32, float64 or long double.
- ``_ref/libti_ref.so`` (built from ``ref_driver.cpp`` + the reference's ``pava.h``, in place):
  the reference's own solver, present only where ``/root/reference`` was available at build
  time; its absence skips the tests that use it.

Both are built by ``make -C oracle`` (``__graft_entry__.build()`` runs it).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
_LIB = HERE / "libti_oracle.so"
_REF = HERE / "_ref" / "libti_ref.so"

_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p


def _bind(lib: ctypes.CDLL, name: str, nargs: int) -> ctypes._CFuncPtr:  # type: ignore[name-defined]
    fn = getattr(lib, name)
    fn.restype = _int
    fn.argtypes = [_vp] * 4 + [_i64, _i64, _int, _int] if nargs == 8 else None
    return fn


_lib: ctypes.CDLL | None = None
_ref: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB.exists():
            raise RuntimeError(f"oracle library missing: {_LIB} (run `make -C oracle`)")
        _lib = ctypes.CDLL(str(_LIB))
        for name in ("ti_oracle_pava_f32", "ti_oracle_pava_f64", "ti_oracle_pava_f64x"):
            _bind(_lib, name, 8)
        for name in ("ti_oracle_grad_f32", "ti_oracle_grad_f64"):
            fn = getattr(_lib, name)
            fn.restype = _int
            fn.argtypes = [_vp] * 7 + [_i64, _i64, _int]
    return _lib


def ref_lib() -> ctypes.CDLL | None:
    """The reference's own pava.h behind a C driver, or None if it was not built here."""
    global _ref
    if _ref is None and _REF.exists():
        _ref = ctypes.CDLL(str(_REF))
        for name in ("ti_ref_pava_f32", "ti_ref_pava_f64"):
            _bind(_ref, name, 8)
    return _ref


def default_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def _ptr(a: np.ndarray | None) -> int | None:
    return None if a is None else a.ctypes.data


def _as2d(y: np.ndarray) -> np.ndarray:
    return y.reshape(1, -1) if y.ndim == 1 else y


def pava(
    y: np.ndarray,
    w: np.ndarray | None = None,
    increasing: bool = True,
    acc: str = "same",
    with_starts: bool = True,
    threads: int | None = None,
    impl: str = "oracle",
) -> tuple[np.ndarray, np.ndarray | None]:
    """Isotonic fit of every row of ``y`` ([batch, n] or [n]) and its block starts (uint8).

    ``acc``: "same" accumulates in y's dtype as the reference CPU path does (float32 or
    float64); "f64" casts the data to float64 first (the float64 CPU fit of the cast data);
    "f64x" uses long double sums (exact on integer-valued data). ``impl="reference"`` runs the
    reference's own pava.h instead (``acc`` must be "same" or "f64").
    """
    shape = y.shape
    y2 = _as2d(np.asarray(y))
    if acc in ("f64", "f64x"):
        y2 = y2.astype(np.float64)
    y2 = np.ascontiguousarray(y2)
    dt = y2.dtype
    if dt not in (np.float32, np.float64):
        raise TypeError(f"oracle takes float32/float64, got {dt}")
    w2 = None
    if w is not None:
        w2 = np.ascontiguousarray(np.broadcast_to(np.asarray(w, dtype=dt), shape).reshape(y2.shape))
    out = np.empty_like(y2)
    starts = np.empty(y2.shape, dtype=np.uint8) if with_starts else None
    b, n = y2.shape
    t = threads if threads is not None else default_threads()
    if impl == "reference":
        rl = ref_lib()
        if rl is None:
            raise RuntimeError("reference CPU solver not built (oracle/_ref/libti_ref.so)")
        if acc == "f64x":
            raise ValueError("the reference solver has no long double mode")
        fn = rl.ti_ref_pava_f32 if dt == np.float32 else rl.ti_ref_pava_f64
    else:
        name = {"f64x": "ti_oracle_pava_f64x"}.get(
            acc, "ti_oracle_pava_f32" if dt == np.float32 else "ti_oracle_pava_f64"
        )
        fn = getattr(lib(), name)
    rc = fn(_ptr(y2), _ptr(w2), _ptr(out), _ptr(starts), b, n, int(increasing), t)
    if rc != 0:
        raise RuntimeError(f"oracle failed ({rc})")
    return out.reshape(shape), None if starts is None else starts.reshape(shape)


def block_grad(
    starts: np.ndarray,
    g: np.ndarray,
    w: np.ndarray | None = None,
    y: np.ndarray | None = None,
    fit: np.ndarray | None = None,
    want_w: bool = False,
    threads: int | None = None,
) -> tuple[np.ndarray, np.ndarray | None]:
    """Gradients of a fit whose blocks start where ``starts`` is set (reference
    ``_api.py:92-115``): ``gy = w G / W`` and, if ``want_w``, ``gw = (y - fit) G / W``. Sums
    run in g's dtype."""
    shape = g.shape
    g2 = np.ascontiguousarray(_as2d(g))
    dt = g2.dtype
    s2 = np.ascontiguousarray(_as2d(starts).astype(np.uint8))
    w2 = None if w is None else np.ascontiguousarray(_as2d(np.asarray(w, dtype=dt)))
    y2 = None if y is None else np.ascontiguousarray(_as2d(np.asarray(y, dtype=dt)))
    f2 = None if fit is None else np.ascontiguousarray(_as2d(np.asarray(fit, dtype=dt)))
    gy = np.empty_like(g2)
    gw = np.empty_like(g2) if want_w else None
    b, n = g2.shape
    fn = lib().ti_oracle_grad_f32 if dt == np.float32 else lib().ti_oracle_grad_f64
    rc = fn(
        _ptr(s2), _ptr(g2), _ptr(w2), _ptr(y2), _ptr(f2), _ptr(gy), _ptr(gw), b, n,
        threads if threads is not None else default_threads(),
    )
    if rc != 0:
        raise RuntimeError(f"oracle grad failed ({rc})")
    return gy.reshape(shape), None if gw is None else gw.reshape(shape)


# --- consumers either side of the fit ------------------------------------------------------------


def soft_rank(x: np.ndarray, eps: float, dtype: type = np.float64) -> tuple[np.ndarray, np.ndarray]:
    """L2 soft ranks of every row of ``x`` ([batch, n]) with regularisation ``eps``, as the
    reference wires torchsort's SoftRank to the isotonic solver (reference
    paper/soft_rank.py:31-55; Blondel et al. 2020): w = (n, ..., 1), s = sort(x * (1 / eps))
    descending, dual = the decreasing isotonic fit of z = s - w (float64 PAVA of z), ranks =
    s - dual in x's order. The tensor steps round in ``dtype`` as the GPU pipeline does (for
    float32: the scaled keys, z, the dual once from float64, the ranks). Returns the ranks and
    the dual's block starts (in sorted order)."""
    x = np.asarray(x).astype(dtype)
    n = x.shape[-1]
    theta = (x * dtype(1.0 / eps)).astype(dtype)
    perm = np.argsort(-theta, axis=-1, kind="stable")
    s = np.take_along_axis(theta, perm, -1)
    z = (s - np.arange(n, 0, -1).astype(dtype)).astype(dtype)
    dual, starts = pava(z.astype(np.float64), increasing=False, acc="f64")
    ranks = np.empty_like(s)
    np.put_along_axis(ranks, perm, (s - dual.astype(dtype)).astype(dtype), -1)
    return ranks, starts


def soft_rank_vjp(x: np.ndarray, eps: float, g: np.ndarray, dtype: type = np.float64) -> np.ndarray:
    """The vector-Jacobian product of ``soft_rank`` for the upstream gradient ``g`` (float64):
    with A the block-averaging map of the dual's partition (in sorted order),
    dx = (g - P^T A P g) / eps (reference paper/soft_rank.py:47-54)."""
    x = np.asarray(x).astype(dtype)
    g = np.asarray(g, dtype=np.float64)
    theta = (x * dtype(1.0 / eps)).astype(dtype)
    perm = np.argsort(-theta, axis=-1, kind="stable")
    _, starts = soft_rank(x, eps, dtype)
    gs = np.take_along_axis(g, perm, -1)
    avg, _ = block_grad(starts, gs)
    back = np.empty_like(avg)
    np.put_along_axis(back, perm, avg, -1)
    return (g - back) * (1.0 / eps)


def calibration_fit(
    keys: np.ndarray,
    y: np.ndarray,
    weight: np.ndarray | None = None,
    offset: np.ndarray | None = None,
    increasing: bool = True,
) -> tuple[np.ndarray, np.ndarray]:
    """The knots (xp, fp) of an isotonic calibration (reference examples/ctr_calibration/
    calibrate.py:171-187): sort the keys, pool equal keys into their (weighted) mean with their
    count (total weight) as weight, fit float64 PAVA over the unique keys; ``offset`` (per
    element) is added to the pooled means before the fit and subtracted after."""
    keys = np.asarray(keys, dtype=np.float64)
    y = np.asarray(y, dtype=np.float64)
    order = np.argsort(keys, kind="stable")
    ks, ys = keys[order], y[order]
    w = np.ones_like(ys) if weight is None else np.asarray(weight, dtype=np.float64)[order]
    xp, first, inverse = np.unique(ks, return_index=True, return_inverse=True)
    sums = np.add.reduceat(w * ys, first)
    weights = np.add.reduceat(w, first)
    means = sums / weights
    shift = np.zeros_like(means)
    if offset is not None:
        shift[inverse] = np.asarray(offset, dtype=np.float64)[order]
    fit, _ = pava((means + shift)[None], weights[None], increasing=increasing, acc="f64")
    return xp, fit[0] - shift


def interp(x: np.ndarray, xp: np.ndarray, fp: np.ndarray) -> np.ndarray:
    """Piecewise-linear interpolation through (xp, fp), constant beyond the ends, restating the
    reference's tensor formula operation for operation (reference examples/ctr_calibration/
    calibrate.py:163-168): j = searchsorted(xp, x) clamped to [1, m - 1],
    t = clamp((x - xp[j-1]) / max(xp[j] - xp[j-1], 1e-300), 0, 1), fp[j-1] + t (fp[j] - fp[j-1])."""
    x = np.asarray(x)
    xp = np.asarray(xp, dtype=x.dtype)
    fp = np.asarray(fp, dtype=x.dtype)
    m = len(xp)
    if m == 1:
        return np.where(np.isnan(x), x, fp[0]).astype(x.dtype)
    j = np.clip(np.searchsorted(xp, x, side="left"), 1, m - 1)
    x0, x1, f0, f1 = xp[j - 1], xp[j], fp[j - 1], fp[j]
    with np.errstate(divide="ignore", invalid="ignore"):
        t = (x - x0) / np.maximum(x1 - x0, x.dtype.type(1e-300))
    t = np.where(t < 0, x.dtype.type(0), np.where(t > 1, x.dtype.type(1), t))
    return (f0 + t * (f1 - f0)).astype(x.dtype)


def pava_ragged(
    values: np.ndarray,
    offsets: np.ndarray,
    w: np.ndarray | None = None,
    increasing: bool = True,
    acc: str = "f64",
) -> tuple[np.ndarray, np.ndarray]:
    """The isotonic fit of every row of a ragged set (row r is values[offsets[r]:offsets[r+1]])
    and the flat block starts (uint8, packed like values): ``pava`` of each row on its own, the
    rows grouped by length so that each length is one batched call."""
    values = np.asarray(values)
    offsets = np.asarray(offsets, dtype=np.int64)
    lengths = np.diff(offsets)
    fit = np.empty(values.shape, dtype=np.float64 if acc in ("f64", "f64x") else values.dtype)
    starts = np.zeros(values.shape, dtype=np.uint8)
    for n in np.unique(lengths):
        if n == 0:
            continue
        rows = np.flatnonzero(lengths == n)
        idx = offsets[rows][:, None] + np.arange(n)[None, :]
        f, s = pava(values[idx], None if w is None else np.asarray(w)[idx], increasing=increasing, acc=acc)
        fit[idx] = f
        starts[idx] = s
    return fit, starts
