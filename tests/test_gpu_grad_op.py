"""The reference's stateless gradient operator, ``isotonic_grad(out, starts, g, w, y)`` (reference
src/torchisotonic/_ext.py:34-40, csrc/grad.cuh:304-413), through ti_grad on the GPU against the
oracle's block gradient (reference _api.py:92-115): rows from 16 elements to 1e7, partitions
from fits and arbitrary ones whose blocks span many tiles and scan groups (2048 elements a tile,
256 tiles a group), NaN rows, the bool and the packed partition."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from torchisotonic_amd import _ext

pytestmark = pytest.mark.gpu


def say(*a: object) -> None:
    print(*a, flush=True)


def op(fit, starts, g, w, y):
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    gy, gw = _ext.isotonic_grad(t(fit), t(starts.astype(bool)), t(g), t(w), t(y))
    return gy.cpu().numpy(), gw.cpu().numpy()


def want(starts, g, w, y, fit):
    f64 = lambda a: None if a is None else a.astype(np.float64)  # noqa: E731
    return oracle.block_grad(starts, f64(g), f64(w), f64(y), f64(fit), want_w=y is not None)


def close(got: np.ndarray, exp: np.ndarray, dtype: type) -> None:
    tol = 1e-11 if dtype == np.float64 else 1e-5
    scale = max(float(np.nanmax(np.abs(exp))), 1e-300)
    np.testing.assert_allclose(got, exp, rtol=tol, atol=tol * scale)


@pytest.mark.parametrize(("batch", "n"), [(100_000, 16), (700, 33), (9, 4096), (3, 100_000), (1, 10_000_000)])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("weighted", [False, True])
def test_matches_block_gradient_on_fits(batch: int, n: int, dtype: type, weighted: bool) -> None:
    say(f"isotonic_grad on fits: {batch} x {n} {np.dtype(dtype).name} weighted={weighted}")
    rng = np.random.default_rng(n + batch)
    y = (np.linspace(0, 3, n) + rng.standard_normal((batch, n))).astype(dtype)
    w = (rng.random((batch, n)) + 0.1).astype(dtype) if weighted else None
    g = rng.standard_normal((batch, n)).astype(dtype)
    fit, starts = oracle.pava(y, w, acc="f64")
    fit = fit.astype(dtype)
    gy, gw = op(fit, starts, g, w, y if weighted else None)
    ey, ew = want(starts, g, w, y if weighted else None, fit)
    close(gy, ey, dtype)
    if weighted:
        close(gw, ew, dtype)
    else:
        assert gw.size == 0  # no y: no weight gradient (as the reference)


@pytest.mark.parametrize(("batch", "n", "p"), [
    (1, 10_000_000, 1e-6),     # blocks of about 1e6 elements: hundreds of tiles, several groups
    (1, 10_000_000, 0.0),      # one block: every tile and group carries
    (3, 700_000, 3e-5),        # rows of several groups
    (5000, 300, 0.01),         # rows packed across tiles, blocks crossing tile edges
    (2, 2049, 0.5),            # two tiles, dense starts
])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_arbitrary_partitions(batch: int, n: int, p: float, dtype: type) -> None:
    # the operator is defined for any partition, not only fits
    say(f"isotonic_grad on random partitions: {batch} x {n} p={p} {np.dtype(dtype).name}")
    rng = np.random.default_rng(int(n * (p + 1)))
    starts = (rng.random((batch, n)) < p).astype(np.uint8)
    starts[:, 0] = 1
    g = rng.standard_normal((batch, n)).astype(dtype)
    w = (rng.random((batch, n)) + 0.1).astype(dtype)
    y = rng.standard_normal((batch, n)).astype(dtype)
    fit = rng.standard_normal((batch, n)).astype(dtype)
    gy, gw = op(fit, starts, g, w, y)
    ey, ew = want(starts, g, w, y, fit)
    close(gy, ey, dtype)
    close(gw, ew, dtype)
    gy, _ = op(fit, starts, g, None, None)
    ey, _ = want(starts, g, None, None, fit)
    close(gy, ey, dtype)


def test_packed_and_bool_starts_agree() -> None:
    say("isotonic_grad: packed words and bool partition")
    rng = np.random.default_rng(3)
    y = rng.standard_normal((40, 3000))
    fit, starts = oracle.pava(y)
    g = rng.standard_normal(y.shape)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    sb = t(starts.astype(bool))
    a, _ = _ext.isotonic_grad(t(fit), sb, t(g), None, None)
    b, _ = _ext.isotonic_grad(t(fit), _ext.bool_to_starts(sb), t(g), None, None)
    assert torch.equal(a, b)


def test_nan_rows_are_one_block() -> None:
    # a NaN row's fit is NaN with starts [1, 0, ...] (reference pava.h:29-38): one block, so gy
    # is the row's mean gradient, gw NaN
    say("isotonic_grad: NaN rows")
    rng = np.random.default_rng(4)
    y = rng.standard_normal((3, 5000))
    y[1, 77] = np.nan
    w = rng.random((3, 5000)) + 0.1
    g = rng.standard_normal((3, 5000))
    fit, starts = oracle.pava(y, w)
    gy, gw = op(fit, starts, g, w, y)
    np.testing.assert_allclose(gy[1], w[1] * g[1].sum() / w[1].sum(), rtol=1e-10)
    assert np.isnan(gw[1]).all() and not np.isnan(gw[[0, 2]]).any()
    ey, ew = want(starts[[0, 2]], g[[0, 2]], w[[0, 2]], y[[0, 2]], fit[[0, 2]])
    close(gy[[0, 2]], ey, np.float64)
    close(gw[[0, 2]], ew, np.float64)


def test_matches_the_autograd_backward() -> None:
    # ti_grad with the forward's fit and partition gives what autograd's backward gives (ti_bwd,
    # from the forward's hulls), up to the last bit of the fit
    say("isotonic_grad against autograd")
    import torchisotonic_amd

    rng = np.random.default_rng(5)
    y = torch.from_numpy(np.linspace(0, 3, 50_000) + rng.standard_normal((4, 50_000))).cuda().requires_grad_()
    w = torch.from_numpy(rng.random((4, 50_000)) + 0.1).cuda().requires_grad_()
    g = torch.from_numpy(rng.standard_normal((4, 50_000))).cuda()
    fit = torchisotonic_amd.isotonic(y, w)
    ay, aw = torch.autograd.grad(fit, (y, w), g)
    out, starts, _, _ = _ext.fit(y.detach(), w.detach(), True, True, True)
    gy, gw = _ext.isotonic_grad(out, starts, g, w.detach(), y.detach())
    torch.testing.assert_close(gy, ay, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(gw, aw, rtol=1e-10, atol=1e-12)
