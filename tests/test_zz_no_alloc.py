"""ti_fwd_noalloc (the forward whose workspace is the library's own device scratch array) against
ti_fwd with a torch-allocated workspace, through the C ABI: bit-identical fits and partitions on
calls in a row, each later one smaller than the one before (the scratch keeps the previous
call's contents). The refusal of a set whose workspace exceeds the scratch is checked without a
GPU, in tests/test_abi.py: it comes before any device call."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from torchisotonic_amd import _ext

pytestmark = pytest.mark.gpu

SCRATCH = 64 << 20


def workspace_bytes(batch: int, n: int, dtype: int, weighted: bool) -> int:
    size = ctypes.c_size_t(0)
    assert _ext.load().ti_fwd_workspace(batch, n, dtype, int(weighted), ctypes.byref(size)) == 0
    return size.value


def run_both(batch: int, n: int, dtype: type, weighted: bool, flags: int, rising: bool = False) -> None:
    lib = _ext.load()
    code = _ext.F32 if dtype == np.float32 else _ext.F64
    need = workspace_bytes(batch, n, code, weighted)
    assert 0 < need <= SCRATCH
    print(f"noalloc {batch} x {n} {np.dtype(dtype).name} weighted={weighted} flags={flags} ({need} B)", flush=True)
    rng = np.random.default_rng(batch * n)
    # (rising: a vertex at every element, so every parent of an out-of-place level defers)
    base = 1e-3 * np.arange(n) + rng.random((batch, 1)) if rising else np.linspace(0, 3, n) + rng.standard_normal((batch, n))
    y = torch.from_numpy(base.astype(dtype)).cuda()
    w = torch.from_numpy((rng.random((batch, n)) + 0.1).astype(dtype)).cuda() if weighted else None
    words = _ext.starts_words(batch, n)
    s = torch.cuda.current_stream().cuda_stream
    lo, hi = -0.5, 2.5
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    out_a = torch.empty_like(y)
    st_a = torch.zeros(words, dtype=torch.int32, device="cuda")
    out_b = torch.full_like(y, float("nan"))
    st_b = torch.full((words,), -1, dtype=torch.int32, device="cuda")
    wp = None if w is None else w.data_ptr()
    rc = lib.ti_fwd(y.data_ptr(), wp, out_a.data_ptr(), st_a.data_ptr(), None, batch, n, code, flags, lo, hi,
                    ws.data_ptr(), need, s)
    assert rc == 0, lib.ti_last_error()
    rc = lib.ti_fwd_noalloc(y.data_ptr(), wp, out_b.data_ptr(), st_b.data_ptr(), None, batch, n, code, flags,
                            lo, hi, s)
    assert rc == 0, lib.ti_last_error()
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b)
    # (bits past n in a row's last word are not part of the partition: compare the n bits)
    assert torch.equal(_ext.starts_to_bool(st_a, batch, n), _ext.starts_to_bool(st_b, batch, n))


def test_noalloc_matches_fwd_on_calls_in_a_row() -> None:
    # largest first: each later call must not see the earlier one's leftovers
    run_both(40, 9000, np.float32, True, _ext.INCREASING)
    run_both(7, 3000, np.float32, True, _ext.INCREASING | _ext.CLIP_MIN | _ext.CLIP_MAX)
    run_both(100, 1000, np.float64, False, 0)
    run_both(3, 40, np.float32, False, _ext.INCREASING)


def test_noalloc_with_out_of_place_levels() -> None:
    # one row of 300000 (spans of 32): its second and third merge levels write their hulls into
    # the scratch's second vertex store and back, every parent's survivors written by
    # survivors_kernel from its table in the scratch; then two noisy rows of 150000 float64, whose
    # second level is out of place too, with tables and stores left over from the first call
    run_both(1, 300_000, np.float32, True, _ext.INCREASING, rising=True)
    run_both(2, 150_000, np.float64, False, _ext.INCREASING)


def test_noalloc_short_rows_need_no_scratch() -> None:
    lib = _ext.load()
    assert workspace_bytes(1000, 16, _ext.F32, False) == 0
    rng = np.random.default_rng(1)
    y = torch.from_numpy(rng.standard_normal((1000, 16)).astype(np.float32)).cuda()
    a, b = torch.empty_like(y), torch.empty_like(y)
    s = torch.cuda.current_stream().cuda_stream
    assert lib.ti_fwd(y.data_ptr(), None, a.data_ptr(), None, None, 1000, 16, 0, 1, 0.0, 0.0, None, 0, s) == 0
    assert lib.ti_fwd_noalloc(y.data_ptr(), None, b.data_ptr(), None, None, 1000, 16, 0, 1, 0.0, 0.0, s) == 0
    torch.cuda.synchronize()
    assert torch.equal(a, b)
