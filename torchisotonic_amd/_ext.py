"""The boundary to the HIP kernels: a ctypes binding of libtorchisotonic_amd.so (C ABI in
include/torchisotonic_amd.h), the torch operator library over it (libtorchisotonic_amd_ops.so:
the fit with its autograd node in C++, which ``isotonic`` calls), and the tensor-level calls
the tests and the reference-named operators make.

Takes the place of the reference's JIT-built operator library (reference
src/torchisotonic/_ext.py:18-68): ``isotonic_tiles`` and ``isotonic_grad`` keep the
reference's names and argument meaning; ``fit`` and ``grad`` are what ``_api`` calls, with the
partition as a packed bit array instead of a bool tensor. Torch allocates every output and
workspace and supplies the current stream; the library never allocates and never falls back
to anything: a missing library, a tensor off the GPU or a failed launch raises.
"""

from __future__ import annotations

import ctypes
import functools
import threading
from pathlib import Path

import torch
from torch import Tensor

LIB_PATH = Path(__file__).resolve().parent / "libtorchisotonic_amd.so"
OPS_LIB_PATH = Path(__file__).resolve().parent / "libtorchisotonic_amd_ops.so"
ABI_VERSION = 10
RAGGED_PLAN_WORDS = 132  # (ti_ragged_plan)

F32, F64 = 0, 1
INCREASING, EXACT, CLIP_MIN, CLIP_MAX = 1, 2, 4, 8
STREAM_OUT, REPAIR_CHAIN = 16, 32  # hints: the results are the same with or without them

_vp, _i64, _int, _uint, _dbl, _sz = (
    ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_uint, ctypes.c_double, ctypes.c_size_t,
)

SYMBOLS = (
    "ti_abi_version",
    "ti_last_error",
    "ti_starts_words",
    "ti_fwd_workspace",
    "ti_fwd_geometry",
    "ti_fwd",
    "ti_fwd_ev",
    "ti_fwd_noalloc",
    "ti_fwd_ragged",
    "ti_bwd_ragged",
    "ti_ragged_plan",
    "ti_ragged_extreme",
    "ti_ragged_pack",
    "ti_ragged_unpack",
    "ti_ragged_rows",
    "ti_fwd_rows",
    "ti_bwd_rows",
    "ti_bwd_workspace",
    "ti_bwd",
    "ti_fwd_ev_hulls",
    "ti_fwd_marked",
    "ti_keep_bytes",
    "ti_keep",
    "ti_bwd_kept_workspace",
    "ti_bwd_kept",
    "ti_grad_workspace",
    "ti_grad",
    "ti_interp",
    "ti_interp_index_bytes",
    "ti_interp_index",
    "ti_interp_indexed",
    "ti_starts_to_bool",
)


@functools.cache
def load() -> ctypes.CDLL:
    """The HIP library, bound. torch is imported first so that the process has one HIP runtime
    (torch's; the library's libamdhip64.so.7 dependency resolves to it)."""
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"torchisotonic_amd: the HIP library {LIB_PATH} is not built "
            "(run `python -m torchisotonic_amd.build`)"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    lib.ti_abi_version.restype = _int
    lib.ti_abi_version.argtypes = []
    lib.ti_last_error.restype = ctypes.c_char_p
    lib.ti_last_error.argtypes = []
    lib.ti_starts_words.restype = _i64
    lib.ti_starts_words.argtypes = [_i64, _i64]
    for name in ("ti_fwd_workspace", "ti_bwd_workspace"):
        fn = getattr(lib, name)
        fn.restype = _int
        fn.argtypes = [_i64, _i64, _int, _int, ctypes.POINTER(_sz)]
    lib.ti_fwd_geometry.restype = _int
    lib.ti_fwd_geometry.argtypes = [_i64, _i64, _int, ctypes.POINTER(_i64), ctypes.POINTER(_int), ctypes.POINTER(_int)]
    lib.ti_fwd.restype = _int
    lib.ti_fwd.argtypes = [_vp] * 5 + [_i64, _i64, _int, _uint, _dbl, _dbl, _vp, _sz, _vp]
    lib.ti_fwd_ev.restype = _int
    lib.ti_fwd_ev.argtypes = [_vp] * 5 + [_i64, _i64, _int, _uint, _dbl, _dbl, _vp, _sz, _vp, _vp]
    lib.ti_fwd_noalloc.restype = _int
    lib.ti_fwd_noalloc.argtypes = [_vp] * 5 + [_i64, _i64, _int, _uint, _dbl, _dbl, _vp]
    lib.ti_fwd_ragged.restype = _int
    lib.ti_fwd_ragged.argtypes = [_vp] * 6 + [_i64, _i64, _i64, _int, _uint, _dbl, _dbl, _vp]
    lib.ti_bwd_ragged.restype = _int
    lib.ti_bwd_ragged.argtypes = [_vp] * 7 + [_i64, _i64, _i64, _int, _uint, _dbl, _dbl, _vp]
    lib.ti_ragged_plan.restype = _int
    lib.ti_ragged_plan.argtypes = [_vp, _i64, _i64, _vp, _vp, _vp]
    lib.ti_ragged_extreme.restype = _int
    lib.ti_ragged_extreme.argtypes = [_vp, _i64, _vp, _i64, _i64, _int, _int, _vp, _vp]
    lib.ti_ragged_pack.restype = _int
    lib.ti_ragged_pack.argtypes = [_vp, _vp, _i64, _vp, _vp, _dbl, _i64, _i64, _int, _int, _vp, _vp, _vp]
    lib.ti_ragged_rows.restype = _int
    lib.ti_ragged_rows.argtypes = [_vp, _i64, _vp, _i64, _vp, _vp]
    lib.ti_fwd_rows.restype = _int
    lib.ti_fwd_rows.argtypes = [_vp] * 6 + [_i64, _i64, _i64, _dbl, _int, _uint, _dbl, _dbl, _vp, _sz, _vp]
    lib.ti_bwd_rows.restype = _int
    lib.ti_bwd_rows.argtypes = [_vp, _vp, _sz] + [_vp] * 6 + [_i64, _i64, _i64, _int, _uint, _dbl, _dbl, _vp, _sz, _vp]
    lib.ti_ragged_unpack.restype = _int
    lib.ti_ragged_unpack.argtypes = [_vp, _vp, _vp, _i64, _i64, _int, _vp, _vp, _i64, _vp, _vp, _vp]
    lib.ti_bwd.restype = _int
    lib.ti_bwd.argtypes = [_vp, _vp, _sz] + [_vp] * 5 + [_i64, _i64, _int, _uint, _dbl, _dbl, _vp, _sz, _vp]
    lib.ti_fwd_ev_hulls.restype = _int
    lib.ti_fwd_ev_hulls.argtypes = [_vp] * 5 + [_i64, _i64, _int, _uint, _dbl, _dbl, _vp, _sz, _vp, _vp, _vp, _vp]
    lib.ti_fwd_marked.restype = _int
    lib.ti_fwd_marked.argtypes = [_vp] * 5 + [_i64, _i64, _int, _uint, _dbl, _dbl, _vp, _sz, _vp, _vp, _uint, _vp]
    lib.ti_keep_bytes.restype = _int
    lib.ti_keep_bytes.argtypes = [_i64, _i64, _int, _int, _i64, ctypes.POINTER(_sz)]
    lib.ti_keep.restype = _int
    lib.ti_keep.argtypes = [_vp, _sz, _vp, _sz, _i64, _i64, _int, _int, _i64, _vp]
    lib.ti_bwd_kept_workspace.restype = _int
    lib.ti_bwd_kept_workspace.argtypes = [_i64, _i64, _int, _int, _i64, ctypes.POINTER(_sz)]
    lib.ti_bwd_kept.restype = _int
    lib.ti_bwd_kept.argtypes = [_vp, _vp, _sz, _i64] + [_vp] * 5 + [_i64, _i64, _int, _uint, _dbl, _dbl, _vp, _sz, _vp]
    lib.ti_grad_workspace.restype = _int
    lib.ti_grad_workspace.argtypes = [_i64, _i64, _int, ctypes.POINTER(_sz)]
    lib.ti_grad.restype = _int
    lib.ti_grad.argtypes = [_vp] * 7 + [_i64, _i64, _int, _vp, _sz, _vp]
    lib.ti_interp.restype = _int
    lib.ti_interp.argtypes = [_vp] * 4 + [_i64, _i64, _int, _vp]
    lib.ti_interp_index_bytes.restype = _int
    lib.ti_interp_index_bytes.argtypes = [_i64, _int, ctypes.POINTER(_sz)]
    lib.ti_interp_index.restype = _int
    lib.ti_interp_index.argtypes = [_vp, _i64, _int, _vp, _sz, _vp]
    lib.ti_interp_indexed.restype = _int
    lib.ti_interp_indexed.argtypes = [_vp] * 4 + [_sz, _vp, _i64, _i64, _int, _vp]
    lib.ti_starts_to_bool.restype = _int
    lib.ti_starts_to_bool.argtypes = [_vp, _vp, _i64, _i64, _vp]
    got = lib.ti_abi_version()
    if got != ABI_VERSION:
        raise RuntimeError(f"torchisotonic_amd: library ABI {got}, expected {ABI_VERSION}")
    return lib


@functools.cache
def ops():
    """``torch.ops.torchisotonic_amd``, loaded: ``isotonic_fit(y, w, increasing, y_min, y_max)``,
    the clamped fit of [batch, n] rows with its backward in C++ (csrc/ti_torch.cpp)."""
    load()  # the C ABI library first, its version checked
    if not OPS_LIB_PATH.exists():
        raise RuntimeError(
            f"torchisotonic_amd: the operator library {OPS_LIB_PATH} is not built "
            "(run `python -m torchisotonic_amd.build`)"
        )
    torch.ops.load_library(str(OPS_LIB_PATH))
    return torch.ops.torchisotonic_amd


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().ti_last_error().decode(errors="replace")
        raise RuntimeError(f"torchisotonic_amd.{what}: {msg} (status {rc})")


def _on_gpu(t: Tensor, name: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(
            f"torchisotonic_amd runs on the GPU (HIP); {name} is on {t.device}. "
            "Move the tensors to a ROCm device first."
        )


def _dtype_code(t: Tensor) -> int:
    if t.dtype == torch.float32:
        return F32
    if t.dtype == torch.float64:
        return F64
    raise RuntimeError(f"torchisotonic_amd: kernels take float32 or float64, got {t.dtype}")


def _ptr(t: Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: Tensor) -> int:
    """The current stream of t's device, as the hipStream_t value the C ABI takes."""
    if _raw_stream is not None:
        return int(_raw_stream(t.device.index))
    return torch.cuda.current_stream(t.device).cuda_stream


class _on_device:
    """Makes t's device the current HIP device for the ABI calls (a no-op when it already is,
    which is the common case and saves a device switch per call)."""

    def __init__(self, device: torch.device) -> None:
        self.index = device.index
        self.prev: int | None = None

    def __enter__(self) -> None:
        cur = torch.cuda.current_device()
        if cur != self.index:
            self.prev = cur
            torch.cuda.set_device(self.index)

    def __exit__(self, *exc: object) -> None:
        if self.prev is not None:
            torch.cuda.set_device(self.prev)


@functools.lru_cache(maxsize=1024)
def starts_words(batch: int, n: int) -> int:
    return int(load().ti_starts_words(batch, n))


@functools.lru_cache(maxsize=1024)
def _workspace_bytes(kind: str, batch: int, n: int, dtype: int, weighted: bool) -> int:
    size = _sz(0)
    fn = load().ti_fwd_workspace if kind == "fwd" else load().ti_bwd_workspace
    _check(fn(batch, n, dtype, int(weighted), ctypes.byref(size)), f"{kind}_workspace")
    return int(size.value)


def geometry(batch: int, n: int, weighted: bool) -> dict:
    """The long-row forward's kernel geometry for a problem set (a diagnostic): elements per
    span of its first kernel, merge launches after it, rows per wave of the first kernel."""
    span0, levels, rpw = _i64(0), _int(0), _int(0)
    _check(
        load().ti_fwd_geometry(batch, n, int(weighted), ctypes.byref(span0), ctypes.byref(levels), ctypes.byref(rpw)),
        "fwd_geometry",
    )
    return {"span0": int(span0.value), "levels": int(levels.value), "rows_per_wave": int(rpw.value)}


def _workspace(kind: str, batch: int, n: int, dtype: int, weighted: bool, device: torch.device) -> Tensor | None:
    size = _workspace_bytes(kind, batch, n, dtype, weighted)
    if size == 0:
        return None
    return torch.empty(size, dtype=torch.uint8, device=device)


def _flags(increasing: bool, exact: bool, y_min: float | None, y_max: float | None) -> int:
    f = (INCREASING if increasing else 0) | (EXACT if exact else 0)
    f |= CLIP_MIN if y_min is not None else 0
    f |= CLIP_MAX if y_max is not None else 0
    return f


_local = threading.local()


def _weight_check(device: torch.device) -> tuple[torch.cuda.Event, torch.cuda.Stream, Tensor]:
    """Per thread and device: the event a weighted fit records once it has read every weight,
    a side stream that copies the weight flag out after that event, and a pinned host word to
    copy it into. The caller learns whether the weights were valid while the rest of its fit
    still runs on the current stream."""
    cache = getattr(_local, "weight_check", None)
    if cache is None:
        cache = _local.weight_check = {}
    entry = cache.get(device.index)
    if entry is None:
        event = torch.cuda.Event()
        event.record(torch.cuda.current_stream(device))  # (torch creates the HIP event here)
        entry = (event, torch.cuda.Stream(device), torch.zeros(1, dtype=torch.int32, pin_memory=True))
        cache[device.index] = entry
    return entry


def fit(
    y: Tensor,
    w: Tensor | None,
    increasing: bool,
    exact: bool = True,
    with_starts: bool = False,
    y_min: float | None = None,
    y_max: float | None = None,
    out: Tensor | None = None,
    hints: int = 0,
) -> tuple[Tensor, Tensor, Tensor | None, Tensor | None]:
    """The fit of every row of ``y`` ([batch, n], float32/float64, on the GPU; into ``out`` when
    given, a contiguous tensor of y's shape and dtype), clamped to
    [y_min, y_max] where given; the packed partition (int32 words) if ``with_starts`` (else an
    empty tensor); for weighted fits, whether some weight was not positive (the caller raises;
    known once the kernels have read w, which for long rows is before the fit has finished),
    else None; and the workspace, which the backward of rows longer than 32 elements reads (None
    when the fit needed none). ``hints``: STREAM_OUT and REPAIR_CHAIN bits passed through."""
    _on_gpu(y, "y")
    dtype = _dtype_code(y)
    if y.dim() != 2:
        raise RuntimeError("torchisotonic_amd.fit: y must be [batch, n]")
    y = y.contiguous()
    batch, n = y.shape
    if w is not None:
        _on_gpu(w, "weight")
        if w.shape != y.shape or w.dtype != y.dtype or w.device != y.device:
            raise RuntimeError("torchisotonic_amd.fit: w must match y in shape, dtype and device")
        w = w.contiguous()
    if out is None:
        out = torch.empty_like(y)
    elif out.shape != y.shape or out.dtype != y.dtype or not out.is_contiguous():
        raise RuntimeError("torchisotonic_amd.fit: out must be contiguous and match y")
    starts = torch.empty(
        starts_words(batch, n) if with_starts else 0, dtype=torch.int32, device=y.device
    )
    bad = torch.zeros(1, dtype=torch.int32, device=y.device) if w is not None else None
    args = (
        batch, n, dtype, _flags(increasing, exact, y_min, y_max) | (hints & (STREAM_OUT | REPAIR_CHAIN)),
        float(y_min) if y_min is not None else 0.0,
        float(y_max) if y_max is not None else 0.0,
    )
    with _on_device(y.device):
        ws = _workspace("fwd", batch, n, dtype, w is not None, y.device)
        ws_args = (_ptr(ws), 0 if ws is None else ws.numel(), _stream(y))
        ptrs = (_ptr(y), _ptr(w), _ptr(out), _ptr(starts) if with_starts else None, _ptr(bad))
        if bad is None:
            _check(load().ti_fwd(*ptrs, *args, *ws_args), "fit")
            return out, starts, None, ws
        event, side, host = _weight_check(y.device)
        _check(load().ti_fwd_ev(*ptrs, *args, *ws_args, event.cuda_event), "fit")
        side.wait_event(event)
        with torch.cuda.stream(side):
            host.copy_(bad, non_blocking=True)
        side.synchronize()
    return out, starts, bool(host.item()), ws


def grad(
    starts: Tensor,
    fwd_ws: Tensor | None,
    g: Tensor,
    w: Tensor | None,
    y: Tensor | None,
    want_y: bool,
    want_w: bool,
    y_min: float | None = None,
    y_max: float | None = None,
    increasing: bool = True,
) -> tuple[Tensor | None, Tensor | None]:
    """Gradients w.r.t. y and w of a fit whose packed partition is ``starts``, for the upstream
    gradient ``g`` (the clamp's backward included where y_min / y_max are given); ``fwd_ws``
    and ``increasing`` are the forward's."""
    _on_gpu(g, "grad")
    dtype = _dtype_code(g)
    batch, n = g.shape
    g = g.contiguous()
    if w is not None:
        w = w.contiguous()
    if y is not None:
        y = y.contiguous()
    gy = torch.empty_like(g) if want_y else None
    gw = torch.empty_like(g) if want_w else None
    if gy is None and gw is None:
        return None, None
    with _on_device(g.device):
        ws = _workspace("bwd", batch, n, dtype, w is not None, g.device)
        rc = load().ti_bwd(
            _ptr(starts), _ptr(fwd_ws), 0 if fwd_ws is None else fwd_ws.numel(),
            _ptr(g), _ptr(w), _ptr(y), _ptr(gy), _ptr(gw), batch, n, dtype,
            _flags(increasing, True, y_min, y_max),
            float(y_min) if y_min is not None else 0.0,
            float(y_max) if y_max is not None else 0.0,
            _ptr(ws), 0 if ws is None else ws.numel(), _stream(g),
        )
    _check(rc, "grad")
    return gy, gw


def interp_index(xp: Tensor) -> Tensor:
    """The knot index of ``xp`` (1-D, ascending, on the GPU; ti_interp_index): a uint8 tensor
    that ``interp`` takes to narrow each query's search to about four knots. It depends on
    ``xp`` only (its values and dtype), so one built after a fit serves every later call."""
    _on_gpu(xp, "xp")
    if xp.dim() != 1 or xp.numel() == 0:
        raise RuntimeError("torchisotonic_amd.interp_index: xp must be 1-D and non-empty")
    dtype = _dtype_code(xp)
    xpc = xp.contiguous()
    nbytes = _sz()
    lib = load()
    _check(lib.ti_interp_index_bytes(xpc.numel(), dtype, ctypes.byref(nbytes)), "interp_index")
    index = torch.empty(nbytes.value, dtype=torch.uint8, device=xp.device)
    with _on_device(xp.device):
        rc = lib.ti_interp_index(_ptr(xpc), xpc.numel(), dtype, _ptr(index), index.numel(), _stream(xpc))
    _check(rc, "interp_index")
    return index


def interp(x: Tensor, xp: Tensor, fp: Tensor, index: Tensor | None = None) -> Tensor:
    """Piecewise-linear interpolation of the knots (xp, fp) at x: the reference calibration
    example's interp (reference examples/ctr_calibration/calibrate.py:163-168) bit for bit.
    x of any shape; xp, fp 1-D of one length, xp ascending. Runs through a knot index
    (``interp_index(xp)``, built here when not given; ti_interp_indexed), whose output is
    ti_interp's bit for bit. An index built from ``xp`` in another dtype than ``x``'s is not
    used: the knots are searched in x's dtype, so the index is built again from those."""
    _on_gpu(x, "x")
    if xp.dim() != 1 or fp.shape != xp.shape or xp.numel() == 0:
        raise RuntimeError("torchisotonic_amd.interp: xp and fp must be 1-D, non-empty and of one length")
    dtype = _dtype_code(x)
    xc = x.contiguous()
    xpc = xp.to(device=x.device, dtype=x.dtype).contiguous()
    fpc = fp.to(device=x.device, dtype=x.dtype).contiguous()
    if index is None or xp.dtype != x.dtype:
        index = interp_index(xpc)
    elif index.dtype != torch.uint8 or index.dim() != 1 or index.device != x.device:
        raise RuntimeError("torchisotonic_amd.interp: index must be interp_index's uint8 tensor on x's device")
    out = torch.empty_like(xc)
    with _on_device(x.device):
        rc = load().ti_interp_indexed(_ptr(xc), _ptr(xpc), _ptr(fpc), _ptr(index), index.numel(), _ptr(out),
                                      xc.numel(), xpc.numel(), dtype, _stream(xc))
    _check(rc, "interp")
    return out


def starts_to_bool(starts: Tensor, batch: int, n: int) -> Tensor:
    """The packed partition as the reference's bool [batch, n] tensor (a test hook)."""
    out = torch.empty(batch, n, dtype=torch.uint8, device=starts.device)
    with _on_device(starts.device):
        rc = load().ti_starts_to_bool(_ptr(starts), _ptr(out), batch, n, _stream(starts))
    _check(rc, "starts_to_bool")
    return out.bool()


def bool_to_starts(starts: Tensor) -> Tensor:
    """A bool [batch, n] partition packed into the kernels' layout (int32 words)."""
    batch, n = starts.shape
    words = (n + 31) // 32
    bits = torch.zeros(batch, words * 32, dtype=torch.int64, device=starts.device)
    bits[:, :n] = starts.to(torch.int64)
    bits[:, 0] = 1
    weights = torch.bitwise_left_shift(
        torch.ones(32, dtype=torch.int64, device=starts.device),
        torch.arange(32, dtype=torch.int64, device=starts.device),
    )
    packed = (bits.view(batch, words, 32) * weights).sum(-1)
    packed = torch.where(packed >= 2**31, packed - 2**32, packed)
    return packed.to(torch.int32).reshape(-1)


def isotonic_tiles(
    y: Tensor, w: Tensor | None, increasing: bool, exact: bool = True, with_starts: bool = False
) -> tuple[Tensor, Tensor]:
    """The reference's operator (reference _ext.py:25-31): the fit of every row of ``y``
    ([batch, n], on the GPU) in y's dtype, and if ``with_starts`` a bool tensor marking where
    its blocks start (else an empty one)."""
    out, starts, bad, _ = fit(y, w, increasing, exact, with_starts)
    if bad:
        raise ValueError("weight must be strictly positive")
    if not with_starts:
        return out, torch.empty(0, dtype=torch.bool, device=y.device)
    return out, starts_to_bool(starts, *y.shape)


def isotonic_grad(
    out: Tensor, starts: Tensor, g: Tensor, w: Tensor | None, y: Tensor | None
) -> list[Tensor | None]:
    """The reference's gradient operator (reference _ext.py:34-40, grad.cuh:386-413): the
    gradients w.r.t. y and, given ``y`` (with ``w``), w.r.t. the weights, of a fit ``out`` whose
    blocks start where ``starts`` is set (bool [batch, n], or the packed int32 words), for the
    upstream gradient ``g``; rows of any length. Returns ``[gy, gw]``, ``gw`` empty without
    ``y`` (as the reference)."""
    _on_gpu(g, "grad")
    dtype = _dtype_code(g)
    if g.dim() != 2 or out.shape != g.shape:
        raise RuntimeError("torchisotonic_amd.isotonic_grad: out and g must be [batch, n] alike")
    if y is not None and w is None:
        raise RuntimeError("torchisotonic_amd.isotonic_grad: y is only needed for the weights' gradient")
    batch, n = g.shape
    packed = bool_to_starts(starts) if starts.dtype == torch.bool else starts.contiguous()
    g = g.contiguous()
    out = out.to(g.dtype).contiguous()
    w = None if w is None else w.to(g.dtype).contiguous()
    y = None if y is None else y.to(g.dtype).contiguous()
    gy = torch.empty_like(g)
    gw = torch.empty_like(g) if y is not None else torch.empty(0, dtype=g.dtype, device=g.device)
    if g.numel() == 0:
        return [gy, gw]
    size = _sz(0)
    _check(load().ti_grad_workspace(batch, n, dtype, ctypes.byref(size)), "grad_workspace")
    ws = torch.empty(size.value, dtype=torch.uint8, device=g.device) if size.value else None
    with _on_device(g.device):
        rc = load().ti_grad(
            _ptr(out), _ptr(packed), _ptr(g), _ptr(w), _ptr(y), _ptr(gy),
            _ptr(gw) if y is not None else None, batch, n, dtype,
            _ptr(ws), 0 if ws is None else ws.numel(), _stream(g),
        )
    _check(rc, "isotonic_grad")
    return [gy, gw]
