"""The backward from a kept state (ti_keep) against the backward from the forward's workspace, on
the GPU.

- Through the C ABI: ti_fwd_ev_hulls reports a bound on the final hulls' vertex counts (checked
  against the partition: a row's final hull has one vertex per block, plus its end point),
  ti_keep copies the final hulls and tile records, and ti_bwd_kept must give gradients
  identical, bit for bit, to ti_bwd's from the workspace: rows of one tile (the packed
  backward) and of many, float32 and float64, weighted or not, clamped, with NaN rows.
- Through autograd at C4's size (one weighted row of 1e8): the node keeps a few megabytes
  instead of the 3.6 GB workspace, and its gradients equal the workspace path's.
- Monotone data, whose final hull has every element as a vertex: the node keeps the workspace
  itself (the kept state would be as large), and its gradients are the oracle's.

Each test prints its case before the GPU work starts.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
import torchisotonic_amd
from torchisotonic_amd import _ext

pytestmark = pytest.mark.gpu


def say(*a: object) -> None:
    print(*a, flush=True)


def _p(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _buf(nbytes: int) -> torch.Tensor | None:
    return torch.empty(nbytes, dtype=torch.uint8, device="cuda") if nbytes else None


def _size(fn, *args) -> int:
    s = ctypes.c_size_t(0)
    assert fn(*args, ctypes.byref(s)) == 0, _ext.load().ti_last_error()
    return s.value


CASES = [
    # (batch, n, dtype, weighted, flags beyond increasing, nan rows)
    (7, 100, np.float32, True, 0, False),  # rows of one tile: the packed backward
    (300, 600, np.float64, False, _ext.CLIP_MIN | _ext.CLIP_MAX, False),
    (3, 5000, np.float32, False, 0, True),
    (2, 70_000, np.float64, True, _ext.CLIP_MAX, False),
    (1, 3_000_000, np.float32, True, 0, False),
]


@pytest.mark.parametrize(("batch", "n", "dtype", "weighted", "clip", "nan"), CASES)
def test_kept_backward_matches_workspace_backward(batch: int, n: int, dtype: type, weighted: bool,
                                                  clip: int, nan: bool) -> None:
    say(f"kept vs workspace backward: {batch}x{n} {np.dtype(dtype).name} weighted={weighted} clip={clip} nan={nan}")
    lib = _ext.load()
    rng = np.random.default_rng(batch * 7 + n)
    y = (np.linspace(0, 2, n) + rng.standard_normal((batch, n))).astype(dtype)
    if nan:
        y[1, n // 3] = np.nan
    w = (rng.random((batch, n)) + 0.1).astype(dtype) if weighted else None
    g = rng.standard_normal((batch, n)).astype(dtype)
    code = _ext.F32 if dtype == np.float32 else _ext.F64
    flags = _ext.INCREASING | clip
    lo, hi = (0.2, 1.5)
    yt, gt = torch.from_numpy(y).cuda(), torch.from_numpy(g).cuda()
    wt = None if w is None else torch.from_numpy(w).cuda()
    out = torch.empty_like(yt)
    starts = torch.empty(_ext.starts_words(batch, n), dtype=torch.int32, device="cuda")
    ws = _buf(_size(lib.ti_fwd_workspace, batch, n, code, int(weighted)))
    maxv = torch.zeros(1, dtype=torch.int64, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.ti_fwd_ev_hulls(_p(yt), _p(wt), _p(out), _p(starts), None, batch, n, code, flags, lo, hi,
                             _p(ws), ws.numel(), stream, None, None, _p(maxv))
    assert rc == 0, lib.ti_last_error()
    torch.cuda.synchronize()
    mv = int(maxv.item())
    # a bound: at least one vertex per block start and the row's end point, at most n + 1
    blocks = _ext.starts_to_bool(starts, batch, n).sum(dim=1) + 1
    assert int(blocks.max().item()) <= mv <= n + 1
    say(f"final hulls: at most {int(blocks.max().item())} vertices a row, bound {mv}")
    kept = _buf(_size(lib.ti_keep_bytes, batch, n, code, int(weighted), mv))
    assert kept.numel() < ws.numel()
    rc = lib.ti_keep(_p(ws), ws.numel(), _p(kept), kept.numel(), batch, n, code, int(weighted), mv, stream)
    assert rc == 0, lib.ti_last_error()
    want_w = weighted

    def run(from_kept: bool) -> tuple[torch.Tensor, torch.Tensor | None]:
        gy = torch.full_like(gt, float("nan"))
        gw = torch.full_like(gt, float("nan")) if want_w else None
        if from_kept:
            bws = _buf(_size(lib.ti_bwd_kept_workspace, batch, n, code, int(weighted), mv))
            rc = lib.ti_bwd_kept(_p(starts), _p(kept), kept.numel(), mv, _p(gt), _p(wt), _p(yt), _p(gy), _p(gw),
                                 batch, n, code, flags, lo, hi, _p(bws), 0 if bws is None else bws.numel(), stream)
        else:
            bws = _buf(_size(lib.ti_bwd_workspace, batch, n, code, int(weighted)))
            rc = lib.ti_bwd(_p(starts), _p(ws), ws.numel(), _p(gt), _p(wt), _p(yt), _p(gy), _p(gw), batch, n,
                            code, flags, lo, hi, _p(bws), 0 if bws is None else bws.numel(), stream)
        assert rc == 0, lib.ti_last_error()
        return gy, gw

    ky, kw = run(True)
    wy, ww = run(False)
    torch.cuda.synchronize()
    assert torch.equal(ky.isnan(), wy.isnan())
    np.testing.assert_array_equal(ky.cpu().numpy(), wy.cpu().numpy())
    if want_w:
        np.testing.assert_array_equal(kw.cpu().numpy(), ww.cpu().numpy())


def test_kept_state_is_independent_of_the_workspace() -> None:
    # after ti_keep the workspace may be overwritten: the backward from the kept state is unchanged
    batch, n = 4, 50_000
    say(f"kept state after the workspace is overwritten: {batch}x{n} float32 weighted")
    lib = _ext.load()
    rng = np.random.default_rng(5)
    y = torch.from_numpy((np.linspace(0, 3, n) + rng.standard_normal((batch, n))).astype(np.float32)).cuda()
    w = torch.from_numpy((rng.random((batch, n)) + 0.1).astype(np.float32)).cuda()
    g = torch.from_numpy(rng.standard_normal((batch, n)).astype(np.float32)).cuda()
    out = torch.empty_like(y)
    starts = torch.empty(_ext.starts_words(batch, n), dtype=torch.int32, device="cuda")
    ws = _buf(_size(lib.ti_fwd_workspace, batch, n, _ext.F32, 1))
    maxv = torch.zeros(1, dtype=torch.int64, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    assert lib.ti_fwd_ev_hulls(_p(y), _p(w), _p(out), _p(starts), None, batch, n, _ext.F32, _ext.INCREASING, 0.0,
                               0.0, _p(ws), ws.numel(), s, None, None, _p(maxv)) == 0
    torch.cuda.synchronize()
    mv = int(maxv.item())
    kept = _buf(_size(lib.ti_keep_bytes, batch, n, _ext.F32, 1, mv))
    assert lib.ti_keep(_p(ws), ws.numel(), _p(kept), kept.numel(), batch, n, _ext.F32, 1, mv, s) == 0

    def grads() -> tuple[torch.Tensor, torch.Tensor]:
        gy, gw = torch.empty_like(g), torch.empty_like(g)
        bws = _buf(_size(lib.ti_bwd_kept_workspace, batch, n, _ext.F32, 1, mv))
        assert lib.ti_bwd_kept(_p(starts), _p(kept), kept.numel(), mv, _p(g), _p(w), _p(y), _p(gy), _p(gw), batch,
                               n, _ext.F32, _ext.INCREASING, 0.0, 0.0, _p(bws), bws.numel(), s) == 0
        return gy, gw

    ay, aw = grads()
    ws.fill_(0xFF)  # every double of the old workspace a NaN, every index -1
    by, bw = grads()
    torch.cuda.synchronize()
    assert torch.equal(ay, by) and torch.equal(aw, bw)
    ey, ew = oracle.block_grad(_ext.starts_to_bool(starts, batch, n).cpu().numpy().astype(np.uint8),
                               g.double().cpu().numpy(), w.double().cpu().numpy(), y.double().cpu().numpy(),
                               out.double().cpu().numpy(), want_w=True)
    np.testing.assert_allclose(ay.cpu().numpy(), ey, rtol=1e-5, atol=1e-5 * float(np.abs(ey).max()))
    np.testing.assert_allclose(aw.cpu().numpy(), ew, rtol=1e-5, atol=1e-5 * float(np.abs(ew).max()))


def _c4(n: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    # BASELINE C4 (bench.py c4_inputs)
    rng = np.random.default_rng(0)
    s = np.sort(rng.standard_normal(n) * 1.5)
    y = (rng.random(n) < 1.0 / (1.0 + np.exp(-s))).astype(np.float32)
    del s
    w = rng.integers(1, 6, n).astype(np.float32)
    g = np.random.default_rng(1).standard_normal(n).astype(np.float32)
    return torch.from_numpy(y).cuda(), torch.from_numpy(w).cuda(), torch.from_numpy(g).cuda()


def test_autograd_keeps_little_at_c4() -> None:
    n = 100_000_000
    say(f"autograd kept state at C4: one weighted row of {n}")
    y, w, g = _c4(n)
    yr, wr = y.view(1, n).requires_grad_(), w.view(1, n).requires_grad_()
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    fit = torchisotonic_amd.isotonic(yr, wr)
    torch.cuda.synchronize()
    held = torch.cuda.memory_allocated() - before - fit.numel() * fit.element_size()
    ws = _size(_ext.load().ti_fwd_workspace, 1, n, _ext.F32, 1)
    say(f"c4: held between forward and backward beyond the fit: {held / 1e6:.1f} MB (workspace {ws / 1e9:.2f} GB)")
    # the partition (12.5 MB) and the kept hulls and tile records (under 2 MB)
    assert held < 16e6
    gy, gw = torch.autograd.grad(fit, (yr, wr), g.view(1, n))
    # the same gradients from the forward's workspace
    out, starts, bad, fws = _ext.fit(y.view(1, n), w.view(1, n), True, True, True)
    assert bad is False
    assert torch.equal(out, fit.detach())
    ry, rw = _ext.grad(starts, fws, g.view(1, n), w.view(1, n), y.view(1, n), True, True)
    torch.cuda.synchronize()
    assert torch.equal(gy, ry) and torch.equal(gw, rw)


KEEP_256MB = str(256 << 20)  # (TI_KEEP_MIN_BYTES: the node keeps hulls from 256 MB of workspace)


def _monotone_autograd(batch: int, n: int) -> tuple[int, int]:
    # rows already increasing (every element a vertex, its own block): the fit under autograd,
    # the memory it holds beside the fit, the workspace size, and both gradients against the
    # oracle's
    rng = np.random.default_rng(3)
    y = torch.from_numpy(np.cumsum(rng.random((batch, n)) + 0.01, axis=1)).cuda()
    w = torch.from_numpy(rng.random((batch, n)) + 0.1).cuda()
    g = torch.from_numpy(rng.standard_normal((batch, n))).cuda()
    ws = _size(_ext.load().ti_fwd_workspace, batch, n, _ext.F64, 1)
    assert ws >= 256 << 20  # (the size at which the node keeps hulls instead)
    yr, wr = y.clone().requires_grad_(), w.clone().requires_grad_()
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    fit = torchisotonic_amd.isotonic(yr, wr)
    torch.cuda.synchronize()
    held = torch.cuda.memory_allocated() - before - fit.numel() * fit.element_size()
    gy, gw = torch.autograd.grad(fit, (yr, wr), g)
    f = fit.detach().cpu().numpy()
    assert float(np.abs(f - y.cpu().numpy()).max()) <= 1e-12 * float(y.abs().max())
    starts = np.ones((batch, n), dtype=np.uint8)
    ey, ew = oracle.block_grad(starts, g.cpu().numpy(), w.cpu().numpy(), y.cpu().numpy(), f, want_w=True)
    np.testing.assert_allclose(gy.cpu().numpy(), ey, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(gw.cpu().numpy(), ew, rtol=1e-9, atol=1e-12 * float(np.abs(ey).max()))
    return held, ws


def test_autograd_keeps_the_workspace_for_monotone_rows(monkeypatch: pytest.MonkeyPatch) -> None:
    # every element a vertex, in a batch whose merges fill the GPU (one vertex store): the kept
    # hulls would be as large as the workspace, which is kept
    monkeypatch.setenv("TI_KEEP_MIN_BYTES", KEEP_256MB)
    say("autograd on 256 monotone weighted rows of 40000")
    held, ws = _monotone_autograd(256, 40_000)
    assert held >= ws


def test_autograd_keeps_hulls_for_a_monotone_row(monkeypatch: pytest.MonkeyPatch) -> None:
    # one row: its upper merge levels write into a second vertex store, so the hulls, every
    # element a vertex, take half the workspace and are kept in its place
    monkeypatch.setenv("TI_KEEP_MIN_BYTES", KEEP_256MB)
    n = 10_000_000
    say(f"autograd on a monotone weighted row of {n}")
    held, ws = _monotone_autograd(1, n)
    kb = ctypes.c_size_t(0)
    assert _ext.load().ti_keep_bytes(1, n, _ext.F64, 1, n + 1, ctypes.byref(kb)) == 0
    assert kb.value <= held < ws


def test_autograd_holds_workspaces_under_a_share_of_the_device() -> None:
    # C5's shape (1.33 GB of workspace): under 1/128 of the device's memory the node holds the
    # workspace itself (no bound kernel, no copy); with TI_KEEP_MIN_BYTES at 256 MB it keeps the
    # final hulls instead. The same gradients either way.
    import os

    b, n = 1000, 65536
    say(f"autograd workspace held or hulls kept: {b} x {n} weighted")
    ws = _size(_ext.load().ti_fwd_workspace, b, n, _ext.F32, 1)
    total = torch.cuda.get_device_properties(0).total_memory
    assert (256 << 20) <= ws <= total // 128
    rng = np.random.default_rng(5)
    y = torch.from_numpy((np.linspace(0, 3, n) + rng.standard_normal((b, n))).astype(np.float32)).cuda()
    w = torch.from_numpy((rng.random((b, n)) + 0.1).astype(np.float32)).cuda()
    g = torch.from_numpy(rng.standard_normal((b, n)).astype(np.float32)).cuda()
    grads = []
    for keep in (None, KEEP_256MB):
        if keep is None:
            os.environ.pop("TI_KEEP_MIN_BYTES", None)
        else:
            os.environ["TI_KEEP_MIN_BYTES"] = keep
        try:
            yr, wr = y.clone().requires_grad_(), w.clone().requires_grad_()
            torch.cuda.synchronize()
            before = torch.cuda.memory_allocated()
            fit = torchisotonic_amd.isotonic(yr, wr)
            torch.cuda.synchronize()
            held = torch.cuda.memory_allocated() - before - fit.numel() * fit.element_size()
            if keep is None:
                assert held >= ws
            else:
                assert held < 64e6  # (the partition's 8 MB, the kept hulls and tile records)
            grads.append(torch.autograd.grad(fit, (yr, wr), g))
        finally:
            os.environ.pop("TI_KEEP_MIN_BYTES", None)
    torch.cuda.synchronize()
    assert torch.equal(grads[0][0], grads[1][0]) and torch.equal(grads[0][1], grads[1][1])
