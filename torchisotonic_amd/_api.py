"""Batched isotonic regression with the semantics of ``sklearn.isotonic.isotonic_regression``,
on the GPU through hand-written HIP kernels for MI355X.

A drop-in for ``torchisotonic.isotonic`` (reference src/torchisotonic/_api.py:13-70): the same
signature, argument checks and messages, dtype policy, ``dim`` handling, weight broadcasting
and autograd behaviour. What differs inside: the clamp to ``[y_min, y_max]`` and its backward
are fused into the kernels, the weights' positivity is checked by the forward kernel as it
reads them (one read of ``w`` instead of two), the autograd node is C++ (no Python, and no
interpreter lock, in the backward), and the backward does not read the fit: rows of up to 32
elements recompute their block means from ``y`` and ``w``, longer rows take them from the final
hulls the forward left in its workspace (kept on the autograd context). There is no CPU
solver: tensors must be on a ROCm device (arguments are still validated first, so the
reference's error messages hold everywhere).
"""

from __future__ import annotations


import torch
from torch import Tensor

from torchisotonic_amd import _ext


def isotonic(
    y: Tensor,
    weight: Tensor | None = None,
    *,
    increasing: bool = True,
    y_min: float | None = None,
    y_max: float | None = None,
    dim: int = -1,
    exact: bool = True,
) -> Tensor:
    """Fit a monotone sequence to each 1-D slice of ``y`` taken along ``dim``.

    Every slice is replaced by its weighted least-squares projection onto the monotone
    sequences: non-decreasing by default, non-increasing when ``increasing=False`` (the
    result sklearn's ``isotonic_regression`` gives). ``weight``, if given, holds positive
    weights of y's shape or a shape that broadcasts to it. ``y_min`` / ``y_max`` clamp the
    result. Slices with a NaN return all NaN. The result has y's float dtype (float16 and
    bfloat16 are fitted in float32); integer input gives torch's default float dtype.

    Gradients flow to ``y`` and ``weight``. The fit is piecewise constant: each run of equal
    values (a block) is the weighted mean of ``y`` over the run, so an element's gradient is
    its weight times the block's summed upstream gradient over the block's total weight.

    ``exact`` exists so calls written for torchisotonic work unchanged. These kernels always
    accumulate and compare in float64 and round a float32 fit once, whatever it is set to.
    """
    # The common call, a [batch, n] float32/float64 tensor on the GPU fitted along its last axis
    # without weights, straight to the operator (the checks below all pass for it; a call's host
    # time matters where the GPU work is tens of microseconds).
    if (
        weight is None
        and type(y) is Tensor
        and y.ndim == 2
        and (dim == -1 or dim == 1)
        and y.is_cuda
        and (y.dtype is torch.float32 or y.dtype is torch.float64)
        and y.numel() > 0
    ):
        return _ext.ops().isotonic_fit(
            y, None, increasing, None if y_min is None else float(y_min), None if y_max is None else float(y_max)
        )
    # Argument checks and messages: reference _api.py:43-61.
    if not isinstance(y, Tensor):
        raise TypeError(f"y must be a torch.Tensor, got {type(y).__name__}")
    if y.is_complex():
        raise TypeError("complex tensors are not supported")
    if y.ndim == 0:
        raise ValueError("y must have at least one dimension")
    out_dtype = y.dtype if y.is_floating_point() else torch.get_default_dtype()
    acc = torch.float64 if out_dtype == torch.float64 else torch.float32
    last = dim == -1 or dim == y.ndim - 1
    rows = y if last else y.movedim(dim, -1)
    w: Tensor | None = None
    if weight is not None:
        if not isinstance(weight, Tensor):
            raise TypeError(f"weight must be a torch.Tensor, got {type(weight).__name__}")
        try:
            w = weight.to(device=y.device, dtype=acc)
            if w.shape != y.shape:
                w = w.broadcast_to(y.shape)
            w = w if last else w.movedim(dim, -1)
        except RuntimeError as e:
            raise ValueError(f"weight of shape {tuple(weight.shape)} does not fit y") from e
        if y.device.type != "cuda" and not bool((w > 0).all()):
            # On the GPU the forward kernel makes this check as it reads w.
            raise ValueError("weight must be strictly positive")
    shape = rows.shape
    if rows.numel() == 0:
        return y.to(out_dtype, copy=True)
    # (no view where the rows already are [batch, n]: every view is one more node for the
    # autograd engine to run in the backward, a few microseconds of host time each)
    two_d = rows.ndim == 2
    flat_y = (rows if two_d else rows.reshape(-1, shape[-1])).to(acc)
    flat_w = None if w is None else (w if two_d else w.reshape(-1, shape[-1]))
    lo = None if y_min is None else float(y_min)
    hi = None if y_max is None else float(y_max)
    _ext._on_gpu(flat_y, "y")
    # the clamped fit with its autograd node in C++ (csrc/ti_torch.cpp; the reference's Python
    # autograd.Function, _api.py:73-97, plus torch.clamp's backward)
    out: Tensor = _ext.ops().isotonic_fit(flat_y, flat_w, increasing, lo, hi)
    if not two_d:
        out = out.reshape(shape)
    return (out if last else out.movedim(-1, dim)).to(out_dtype)
