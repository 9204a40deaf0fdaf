"""Isotonic regression of ragged rows: rows of different lengths packed end to end, with their
offsets, fitted without a padding pass.

The reference fits equal-length rows only; its users pad ragged rows (tail values that never
pool into the data: above the row's maximum for an increasing fit, below its minimum for a
decreasing one) or lay them end to end with offsets
(reference README.md:100-103, examples/ctr_calibration/README.md:25-27). Here the packed values
and the row offsets (CSR layout) go to the GPU as they are:

- rows of 1 to 32 elements, the short-row regime, are fitted together in one HIP launch
  (``ti_fwd_ragged``: one thread per row, a workgroup's rows staged through LDS), after one
  kernel has checked the offsets and sized the rows and its four words have reached the host
  (the call's one wait); with ``max_len``, a bound on the row lengths, that launch goes before
  the wait and runs during it;
- longer rows are fitted a length bucket at a time (lengths in (2^(b-1), 2^b], a small bucket
  joined to the next): the plan's kernel gives each row its bucket key and each bucket its size,
  a stable sort of the keys on the device orders the rows (``ti_ragged_rows``), and each
  bucket's rows are gathered into one dense [k, L] block, each padded beyond its own extreme
  with the reference's rule for padding (a tail above the row's maximum for an increasing fit,
  below its minimum for a decreasing one, which pools with nothing of the row; for float32 the
  largest finite value, which needs no extreme), one ``ti_fwd`` over the block, and the fits
  scattered back (``ti_ragged_extreme``, ``ti_ragged_pack``, ``ti_ragged_unpack``);
- the backward of the rows of 1 to 32 elements is one HIP launch too (``ti_bwd_ragged``: one
  thread per row, the blocks read from the forward's flat start bits); each bucket of longer
  rows takes its gradients from its own forward (``ti_bwd`` over the block of g, scattered
  back).

The clamp to [y_min, y_max] is torch.clamp after the fit, as in the reference (_api.py:68-69).
These steps, and the backward, run in one C++ operator with its autograd node
(``torch.ops.torchisotonic_amd.isotonic_ragged_fit``, csrc/ti_torch.cpp): a call costs a few
microseconds of host time, where the same steps in Python and a Python autograd node cost more
than the kernels. The functions below compose the same C ABI calls step by step; the tests use
them to read the start bits.
"""

from __future__ import annotations

import threading

import torch
from torch import Tensor

from torchisotonic_amd import _ext

_local = threading.local()


def _host_words(device: torch.device) -> tuple[Tensor, torch.cuda.Event]:
    """Per thread and device: the pinned host words the plan is copied into, and the event
    recorded once they are there."""
    cache = getattr(_local, "plan", None)
    if cache is None:
        cache = _local.plan = {}
    if device.index not in cache:
        cache[device.index] = (torch.empty(_ext.RAGGED_PLAN_WORDS, dtype=torch.int64, pin_memory=True),
                               torch.cuda.Event())
    return cache[device.index]


_PLAN_I32 = 2 * _ext.RAGGED_PLAN_WORDS  # the plan's int32 words in the zeroed buffer


def _plan(offsets, lengths, values: Tensor, weighted: bool):
    """The row offsets as a device int64 tensor; zeroed device words for the fit (the flat
    start bits and the weight flag); and the plan of the offsets under way: one kernel
    (ti_ragged_plan) checks them, sizes the rows and their length buckets and writes each
    row's bucket key, and the plan's words are on their way to the host (the offsets
    themselves are never copied; ``_plan_wait`` reads the words)."""
    off = _offsets_tensor(offsets, lengths, values.device)
    nrows, total = off.numel() - 1, values.numel()
    # one zeroed buffer: the plan, the weight flag, the flat start bits
    zeros = torch.zeros(_PLAN_I32 + 2 + (total + 31) // 32, dtype=torch.int32, device=values.device)
    plan, bad, bits = zeros[:_PLAN_I32].view(torch.int64), zeros[_PLAN_I32:_PLAN_I32 + 1], zeros[_PLAN_I32 + 2:]
    keys = torch.empty(nrows, dtype=torch.uint8, device=values.device)
    host, ready = _host_words(values.device)
    with _ext._on_device(values.device):
        stream = torch.cuda.current_stream(values.device)
        _ext._check(_ext.load().ti_ragged_plan(off.data_ptr(), nrows, total, plan.data_ptr(), keys.data_ptr(),
                                               stream.cuda_stream), "isotonic_ragged")
        host.copy_(plan, non_blocking=True)
        ready.record(stream)
    return off, bits, (bad if weighted else None), (host, ready, offsets is None, total, keys)


def _offsets_tensor(offsets, lengths, device: torch.device) -> Tensor:
    """The row offsets as a contiguous device int64 tensor (from ``lengths`` by a cumulative
    sum); type errors raised, the values checked by the plan."""
    if (offsets is None) == (lengths is None):
        raise ValueError("give exactly one of offsets and lengths")
    src = offsets if offsets is not None else lengths
    t = src if isinstance(src, Tensor) else torch.as_tensor(src)
    if t.ndim != 1 or t.is_floating_point() or t.is_complex() or t.dtype == torch.bool:
        raise ValueError("offsets / lengths must be a 1-D integer sequence")
    t = t.to(device=device, dtype=torch.int64)
    if offsets is None:
        off = torch.zeros(t.numel() + 1, dtype=torch.int64, device=device)
        torch.cumsum(t, 0, out=off[1:])
        return off
    if t.numel() < 1:
        raise ValueError("offsets must hold at least one value")
    return t.contiguous()


_BUCKET_MERGE = 1 << 22  # a bucket joins the next while that pads at most this many elements
_ROW_MAP_BYTES = 0x7FFF0000  # ti_fwd_rows' limit on the packed arrays


def _buckets(words: list[int], n_long: int) -> list[tuple[int, int, int]]:
    """The length buckets of the longer rows from the plan's counts and longest rows, a bucket
    joined to the next longer one while that pads at most _BUCKET_MERGE more elements (a
    bucket's launches cost about as much as fitting that many): (first row in bucket order,
    rows, block length) triples."""
    out, first, k, L = [], 0, 0, 0
    for b in range(6, 64):
        kb, lb = words[4 + b], words[68 + b]
        if kb <= 0:
            continue
        if k > 0 and k * (lb - L) > _BUCKET_MERGE:
            out.append((first, k, L))
            first, k = first + k, 0
        k, L = k + kb, lb
    if k > 0:
        out.append((first, k, L))
    assert first + k == n_long, (first + k, n_long)
    return out


def _plan_wait(off: Tensor, pending) -> tuple[int, tuple]:
    """The plan's words, once they are on the host (the stream's later work keeps running): the
    offsets' errors raised, the longest row of at most 32 elements (0 if none), and the longer
    rows' plan: their number, their buckets and the rows' bucket keys."""
    host, ready, from_lengths, total, keys = pending
    ready.synchronize()
    words = host.tolist()
    err, short_max, n_long = words[0], words[1], words[2]
    if err & 4:
        raise ValueError("lengths must be non-negative" if from_lengths else "offsets must not decrease")
    if err & 3:
        raise ValueError(f"offsets must run from 0 to values.numel() = {total}")
    return int(short_max), (int(n_long), _buckets(words, n_long) if n_long else [], keys)


def _offsets(offsets, lengths, values: Tensor, weighted: bool):
    """``_plan`` and ``_plan_wait`` in a row: the offsets, validated, the longest short row, the
    longer rows' plan, and the zeroed bits and weight flag."""
    off, bits, bad, pending = _plan(offsets, lengths, values, weighted)
    short_max, long_plan = _plan_wait(off, pending)
    return off, short_max, long_plan, bits, bad


def _fit_short(values: Tensor, w: Tensor | None, out: Tensor, off: Tensor, nmax: int, bits: Tensor,
               bad: Tensor | None, increasing: bool) -> None:
    """One launch (ti_fwd_ragged) over every row of at most nmax elements; longer rows are left
    alone. Every offset is clamped in the kernel, so this may run before the plan is read."""
    flags = (_ext.INCREASING if increasing else 0) | _ext.EXACT
    with _ext._on_device(values.device):
        rc = _ext.load().ti_fwd_ragged(
            values.data_ptr(), _ext._ptr(w), out.data_ptr(), bits.data_ptr(), _ext._ptr(bad),
            off.data_ptr(), off.numel() - 1, values.numel(), nmax, _ext._dtype_code(values), flags,
            0.0, 0.0, _ext._stream(values),
        )
    _ext._check(rc, "isotonic_ragged")


def _fit_long(values: Tensor, w: Tensor | None, out: Tensor, off: Tensor, long_plan: tuple,
              increasing: bool) -> list:
    """The longer rows, a bucket at a time: the rows in bucket order (a stable sort of the plan's
    keys, ti_ragged_rows), then per bucket either (float32 sets under 2 GB) one ti_fwd_rows, which
    reads and writes the rows in place as the rows of a block padded with the largest finite
    value, or the block of its rows, each padded beyond its extreme (float32: the largest finite
    value; float64: ti_ragged_extreme), ti_fwd over it, and the fits scattered back
    (ti_ragged_pack, ti_ragged_unpack). Per bucket: its rows' (first, length) on the host, the
    block length L, the block's packed starts, its forward workspace, the y and w blocks (None in
    place)."""
    n_long, buckets, keys = long_plan
    if n_long == 0:
        return []
    lib = _ext.load()
    code = _ext._dtype_code(values)
    nrows, total = off.numel() - 1, values.numel()
    s = _ext._stream(values)
    inc = 1 if increasing else 0
    f32 = values.dtype == torch.float32
    pad = (1.0 if increasing else -1.0) * float(torch.finfo(torch.float32).max) if f32 else 0.0
    order = torch.sort(keys, stable=True).indices[nrows - n_long:].contiguous()
    rows = torch.empty(n_long, 2, dtype=torch.int64, device=values.device)
    ext = None if f32 else torch.zeros(n_long, dtype=torch.int64, device=values.device)
    with _ext._on_device(values.device):
        _ext._check(lib.ti_ragged_rows(off.data_ptr(), nrows, order.data_ptr(), n_long, rows.data_ptr(), s),
                    "isotonic_ragged")
    done = []
    # float32 sets under 2 GB: each bucket fitted in place (ti_fwd_rows), else through a block
    rows_mode = f32 and total * 4 < _ROW_MAP_BYTES
    flags = (_ext.INCREASING if increasing else 0) | _ext.EXACT
    for f, k, L in buckets:
        desc = rows[f:f + k]
        if rows_mode:
            starts = torch.empty(_ext.starts_words(k, L), dtype=torch.int32, device=values.device)
            bad = None if w is None else torch.zeros(1, dtype=torch.int32, device=values.device)
            with _ext._on_device(values.device):
                ws = _ext._workspace("fwd", k, L, code, w is not None, values.device)
                _ext._check(lib.ti_fwd_rows(values.data_ptr(), _ext._ptr(w), out.data_ptr(), starts.data_ptr(),
                                            _ext._ptr(bad), desc.data_ptr(), k, L, total, pad, code, flags, 0.0, 0.0,
                                            _ext._ptr(ws), 0 if ws is None else ws.numel(), s), "isotonic_ragged")
            if bad is not None and bool(bad.item()):
                raise ValueError("weight must be strictly positive")
            done.append((desc.cpu().numpy(), L, starts, ws, None, None))
            continue
        kp = None if ext is None else ext[f:f + k].data_ptr()
        with _ext._on_device(values.device):
            if ext is not None:
                _ext._check(lib.ti_ragged_extreme(values.data_ptr(), total, desc.data_ptr(), k, L, code, inc, kp, s),
                            "isotonic_ragged")
            yb = torch.empty(k, L, dtype=values.dtype, device=values.device)
            wb = None if w is None else torch.empty_like(yb)
            _ext._check(lib.ti_ragged_pack(values.data_ptr(), _ext._ptr(w), total, desc.data_ptr(), kp, pad, k, L,
                                           code, inc, yb.data_ptr(), _ext._ptr(wb), s), "isotonic_ragged")
        ob, starts, bad_b, ws = _ext.fit(yb, wb, increasing, True, True)
        if bad_b:
            raise ValueError("weight must be strictly positive")
        with _ext._on_device(values.device):
            _ext._check(lib.ti_ragged_unpack(ob.data_ptr(), None, desc.data_ptr(), k, L, code, out.data_ptr(), None,
                                             total, None, None, s), "isotonic_ragged")
        done.append((desc.cpu().numpy(), L, starts, ws, yb, wb))
    return done


def _fit(values: Tensor, w: Tensor | None, off: Tensor, short_max: int, long_plan: tuple,
         bits: Tensor, bad: Tensor | None, increasing: bool) -> tuple[Tensor, list]:
    """The fits of every row (packed like values) with the flat start bits of the short rows
    in ``bits`` (a longer row has its first bit only), and per bucket of longer rows what
    ``_fit_long`` returns."""
    out = torch.empty_like(values)
    if short_max > 0:
        _fit_short(values, w, out, off, short_max, bits, bad, increasing)
    long_rows = _fit_long(values, w, out, off, long_plan, increasing)
    if bad is not None and short_max > 0 and bool(bad.item()):
        raise ValueError("weight must be strictly positive")
    return out, long_rows


def isotonic_ragged(
    values: Tensor,
    offsets: Tensor | None = None,
    *,
    lengths: Tensor | None = None,
    weight: Tensor | None = None,
    increasing: bool = True,
    y_min: float | None = None,
    y_max: float | None = None,
    max_len: int | None = None,
) -> Tensor:
    """Isotonic regression of every row of a ragged set: row r is ``values[offsets[r]:
    offsets[r + 1]]`` (or give ``lengths``, its row lengths). ``values`` (and ``weight``, shaped
    like it, positive) is 1-D on a ROCm device; offsets run from 0 to ``values.numel()``. Returns
    the fits packed like ``values``, clamped to [y_min, y_max] where given; differentiable in
    ``values`` and ``weight``. Dtype rules as ``isotonic``.

    ``max_len``: a bound on the rows' lengths, where the caller knows one (the length rows
    would be padded to). The fit then starts without waiting for the offsets' plan to reach the
    host; a wrong bound costs a second launch, never a wrong result."""
    if not isinstance(values, Tensor):
        raise TypeError(f"values must be a torch.Tensor, got {type(values).__name__}")
    if values.ndim != 1:
        raise ValueError("values must be 1-D (rows packed end to end)")
    out_dtype = values.dtype if values.is_floating_point() else torch.get_default_dtype()
    acc = torch.float64 if out_dtype == torch.float64 else torch.float32
    _ext._on_gpu(values, "values")
    v = values.to(acc).contiguous()
    w = None
    if weight is not None:
        if not isinstance(weight, Tensor) or weight.shape != values.shape:
            raise ValueError("weight must be a tensor shaped like values")
        w = weight.to(device=values.device, dtype=acc).contiguous()
    if max_len is not None and (isinstance(max_len, bool) or not isinstance(max_len, int) or max_len < 0):
        raise ValueError("max_len must be a non-negative int")
    off = _offsets_tensor(offsets, lengths, values.device)
    fit = _ext.ops().isotonic_ragged_fit(v, w, off, increasing, max_len or 0, offsets is None)
    if values.numel() == 0:
        return values.to(out_dtype, copy=True)
    if y_min is not None or y_max is not None:
        fit = fit.clamp(min=y_min, max=y_max)
    return fit.to(out_dtype)
