"""Isotonic calibration: the steps on either side of the isotonic fit in its flagship use,
turning scores into calibrated probabilities (sklearn's ``IsotonicRegression`` fit and predict,
on the GPU).

Follows the reference's calibration example (reference examples/ctr_calibration/
calibrate.py:163-187, README.md:42-57):

- ``calibration_fit(keys, y)``: sort the keys; pool equal keys into one point at their
  weighted mean with their total weight as its weight (sklearn pools duplicate X the same way);
  fit isotonic regression over the unique keys (this package's HIP kernels). Returns the knots
  ``(xp, fp)``. An optional per-element ``offset`` is added to the pooled means before the fit
  and subtracted after: segments placed far enough apart never pool across, so one fit serves
  many segments (the reference's per-segment calibration, calibrate.py:171-187).
- ``calibration_predict(x, xp, fp)``: piecewise-linear interpolation through the knots,
  constant beyond the ends (np.interp's semantics), in one HIP kernel (``ti_interp_indexed``)
  through a knot index that narrows each query's search to about four knots.

``IsotonicCalibrator`` wraps both, with sklearn's ``y_min`` / ``y_max`` clip and direction; it
builds the knot index once, after the fit, for all later predictions.
Sums run in float64 whatever the input dtype (the reference casts its scores to float64).
"""

from __future__ import annotations

import torch
from torch import Tensor

from torchisotonic_amd import _ext
from torchisotonic_amd._api import isotonic


def _pool_sorted(keys: Tensor, y: Tensor, w: Tensor | None) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Unique sorted keys, their weighted means, total weights, and each element's key index.
    Runs of one key are contiguous (the keys are sorted), so their sums are segment sums in a
    fixed order (no atomics)."""
    xp, inverse, counts = torch.unique_consecutive(keys, return_inverse=True, return_counts=True)
    if w is None:
        sums = torch.segment_reduce(y, "sum", lengths=counts)
        weights = counts.to(torch.float64)
    else:
        sums = torch.segment_reduce(w * y, "sum", lengths=counts)
        weights = torch.segment_reduce(w, "sum", lengths=counts)
    return xp, sums / weights, weights, inverse


def calibration_fit(
    keys: Tensor,
    y: Tensor,
    weight: Tensor | None = None,
    offset: Tensor | None = None,
    *,
    increasing: bool = True,
    y_min: float | None = None,
    y_max: float | None = None,
) -> tuple[Tensor, Tensor]:
    """The isotonic fit of ``y`` over the sorted unique ``keys`` (1-D tensors of one length, on
    the GPU): knots ``(xp, fp)``, float64. Equal keys are pooled into their (weighted) mean with
    their count (or total weight) as weight; ``offset`` (per element) is added to the pooled
    means before the fit and subtracted after (reference calibrate.py:171-187)."""
    for name, t in (("keys", keys), ("y", y)):
        if not isinstance(t, Tensor) or t.ndim != 1:
            raise ValueError(f"{name} must be a 1-D tensor")
    if y.shape != keys.shape:
        raise ValueError("keys and y must have one length")
    if keys.numel() == 0:
        raise ValueError("calibration needs at least one point")
    _ext._on_gpu(keys, "keys")
    keys64 = keys.to(torch.float64)
    sk, order = torch.sort(keys64, stable=True)
    ys = y.to(device=keys.device, dtype=torch.float64)[order]
    ws = None
    if weight is not None:
        ws = weight.to(device=keys.device, dtype=torch.float64)[order]
        if not bool((ws > 0).all()):
            raise ValueError("weight must be strictly positive")
    xp, means, weights, inverse = _pool_sorted(sk, ys, ws)
    shift = None
    if offset is not None:
        shift = torch.zeros_like(means)
        shift[inverse] = offset.to(device=keys.device, dtype=torch.float64)[order]
        means = means + shift
    fit = isotonic(means[None], weights[None], increasing=increasing)[0]
    if shift is not None:
        fit = fit - shift
    if y_min is not None or y_max is not None:
        fit = fit.clamp(min=y_min, max=y_max)
    return xp, fit


def calibration_predict(x: Tensor, xp: Tensor, fp: Tensor, index: Tensor | None = None) -> Tensor:
    """Calibrated values at ``x``: the piecewise-linear interpolation through ``(xp, fp)``,
    constant beyond the ends (reference calibrate.py:163-168, np.interp's semantics), computed
    in float64 and returned as float64. ``index``: the knot index of the float64 ``xp``
    (``torchisotonic_amd._ext.interp_index``), built here when not given."""
    return _ext.interp(x.to(torch.float64), xp.to(torch.float64), fp.to(torch.float64), index)


class IsotonicCalibrator:
    """Fit on (scores, labels), then map new scores to calibrated values: sklearn's
    ``IsotonicRegression(out_of_bounds="clip")`` on the GPU."""

    def __init__(self, *, increasing: bool = True, y_min: float | None = None, y_max: float | None = None) -> None:
        self.increasing = increasing
        self.y_min = y_min
        self.y_max = y_max
        self.xp: Tensor | None = None
        self.fp: Tensor | None = None
        self.index: Tensor | None = None

    def fit(self, scores: Tensor, labels: Tensor, weight: Tensor | None = None) -> "IsotonicCalibrator":
        self.xp, self.fp = calibration_fit(
            scores, labels, weight, increasing=self.increasing, y_min=self.y_min, y_max=self.y_max
        )
        self.index = _ext.interp_index(self.xp)
        return self

    def predict(self, scores: Tensor) -> Tensor:
        if self.xp is None or self.fp is None:
            raise RuntimeError("IsotonicCalibrator: call fit first")
        return calibration_predict(scores, self.xp, self.fp, self.index)

    __call__ = predict
