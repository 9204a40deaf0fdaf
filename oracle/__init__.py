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
