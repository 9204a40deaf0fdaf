"""Helpers for the GPU parity tests: run the HIP path, run the oracle on the same inputs, and
compare within the tolerances of the parity contract:

- float64: |fit - oracle| <= 1e-12 * max|y| (oracle: float64 PAVA);
- float32: |fit - oracle| <= 4 ulp(1) * max|y| against the float64 PAVA of the float32 data
  (the reference's own accuracy method, paper/accuracy.py:16-19), and within the reference
  suite's 1e-4 of the float32-accumulating CPU path (reference tests/test_cuda.py:26-28);
- block starts identical to the oracle's on inputs without rounding-level ties.
"""

from __future__ import annotations

import numpy as np
import torch

import oracle
from torchisotonic_amd import _ext

F32_ULPS = 4 * 2.0**-23
F64_TOL = 1e-12


def gpu_fit(
    y: np.ndarray,
    w: np.ndarray | None = None,
    increasing: bool = True,
    y_min: float | None = None,
    y_max: float | None = None,
    with_starts: bool = True,
) -> tuple[np.ndarray, np.ndarray | None]:
    """The HIP fit of [batch, n] rows (through the tensor boundary), and its starts as uint8."""
    yt = torch.from_numpy(np.ascontiguousarray(y)).cuda()
    wt = None if w is None else torch.from_numpy(np.ascontiguousarray(w)).cuda()
    out, starts, bad, _ = _ext.fit(yt, wt, increasing, True, with_starts, y_min, y_max)
    if bad is not None:
        assert bad is False
    s = None
    if with_starts:
        s = _ext.starts_to_bool(starts, *y.shape).cpu().numpy().astype(np.uint8)
    return out.cpu().numpy(), s


def tolerance(y: np.ndarray) -> float:
    scale = float(np.nanmax(np.abs(y))) if y.size else 0.0
    scale = max(scale, 1e-300)
    return (F64_TOL if y.dtype == np.float64 else F32_ULPS) * scale


def check_fit(
    y: np.ndarray,
    w: np.ndarray | None = None,
    increasing: bool = True,
    check_starts: bool = True,
    y_min: float | None = None,
    y_max: float | None = None,
) -> tuple[np.ndarray, np.ndarray]:
    got, starts = gpu_fit(y, w, increasing, y_min, y_max)
    want, want_starts = oracle.pava(y, w, increasing=increasing, acc="f64")
    want_c = want.copy()
    if y_min is not None:
        want_c = np.where(want_c < y_min, y_min, want_c)
    if y_max is not None:
        want_c = np.where(want_c > y_max, y_max, want_c)
    assert got.dtype == y.dtype
    nan_rows = np.isnan(y).any(axis=-1)
    assert np.isnan(got[nan_rows]).all()
    ok = ~nan_rows
    diff = np.abs(got[ok].astype(np.float64) - want_c[ok])
    tol = tolerance(y[ok]) if ok.any() else 0.0
    assert diff.size == 0 or float(diff.max()) <= tol, (float(diff.max()), tol)
    if y.dtype == np.float32 and y_min is None and y_max is None:
        ref32, _ = oracle.pava(y, w, increasing=increasing)
        np.testing.assert_allclose(got[ok], ref32[ok], rtol=1e-4, atol=1e-4)
    if check_starts:
        assert starts is not None
        np.testing.assert_array_equal(starts[ok], want_starts[ok])
        assert (starts[nan_rows][:, :1] == 1).all() and (starts[nan_rows][:, 1:] == 0).all()
    return got, starts
