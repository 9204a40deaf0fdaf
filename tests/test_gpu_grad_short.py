"""Gradients on the GPU for short rows: against the oracle's block sums on the GPU's own
partition and on the oracle's, against finite differences (gradcheck in float64), and the
reference's known answers (reference tests/test_grad.py, test_cuda.py:137-210)."""

from __future__ import annotations

from typing import Any

import numpy as np
import pytest
import torch
from torch.autograd import gradcheck

import oracle
import torchisotonic_amd
from torchisotonic_amd import _ext

pytestmark = pytest.mark.gpu


def rows(batch: int, n: int, seed: int, dtype: torch.dtype = torch.float64):
    g = torch.Generator().manual_seed(seed)
    y = torch.linspace(0, 3, n, dtype=dtype) + torch.randn(batch, n, generator=g, dtype=dtype)
    w = torch.rand(batch, n, generator=g, dtype=dtype) + 0.1
    c = torch.randn(batch, n, generator=g, dtype=dtype)
    return y, w, c


@pytest.mark.parametrize("seed", range(3))
@pytest.mark.parametrize(
    "kwargs", [{}, {"increasing": False}, {"y_min": -0.3, "y_max": 0.5}, {"dim": 0}]
)
def test_matches_finite_differences(seed: int, kwargs: dict[str, Any]) -> None:
    # reference tests/test_grad.py:21-29
    g = torch.Generator().manual_seed(seed)
    y = torch.randn(4, 13, generator=g, dtype=torch.float64).cuda().requires_grad_()
    w = (torch.rand(4, 13, generator=g, dtype=torch.float64) + 0.1).cuda().requires_grad_()
    assert gradcheck(lambda y, w: torchisotonic_amd.isotonic(y, w, **kwargs), (y, w))
    assert gradcheck(lambda y: torchisotonic_amd.isotonic(y, **kwargs), (y,))


def test_block_average() -> None:
    # reference tests/test_grad.py:32-37
    y = torch.tensor([3.0, 1.0, 2.0], device="cuda", requires_grad=True)
    c = torch.tensor([1.0, 2.0, 6.0], device="cuda")
    (grad,) = torch.autograd.grad((torchisotonic_amd.isotonic(y) * c).sum(), (y,))
    torch.testing.assert_close(grad.cpu(), torch.full((3,), 3.0))


@pytest.mark.parametrize(("batch", "n"), [(70, 1), (70, 5), (9, 16), (300, 17), (7, 31), (5000, 32)])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_gradients_match_oracle(batch: int, n: int, dtype: torch.dtype) -> None:
    # reference tests/test_cuda.py:137-157 against the CPU; here against the oracle's closed form
    # on the oracle's partition (tie-free data: the GPU's partition is the same).
    print(f"grad batch={batch} n={n} dtype={dtype}", flush=True)
    y, w, c = rows(batch, n, n, dtype)
    for inc in (True, False):
        yy = y.cuda().requires_grad_()
        ww = w.cuda().requires_grad_()
        fit = torchisotonic_amd.isotonic(yy, ww, increasing=inc)
        gy, gw = torch.autograd.grad((fit * c.cuda()).sum(), (yy, ww))
        ref_fit, starts = oracle.pava(y.numpy(), w.numpy(), increasing=inc, acc="f64")
        ey, ew = oracle.block_grad(
            starts, c.double().numpy(), w.double().numpy(), y.double().numpy(), ref_fit, want_w=True
        )
        tol = 1e-12 if dtype == torch.float64 else 1e-5
        np.testing.assert_allclose(gy.double().cpu().numpy(), ey, rtol=tol, atol=tol)
        scale = tol * (1 + float(y.abs().max()))
        np.testing.assert_allclose(gw.double().cpu().numpy(), ew, rtol=tol, atol=scale)
        (gy1,) = torch.autograd.grad((torchisotonic_amd.isotonic(yy, increasing=inc) * c.cuda()).sum(), (yy,))
        _, s1 = oracle.pava(y.numpy(), None, increasing=inc, acc="f64")
        e1, _ = oracle.block_grad(s1, c.double().numpy())
        np.testing.assert_allclose(gy1.double().cpu().numpy(), e1, rtol=tol, atol=tol)


def test_gradient_is_block_average_on_the_gpus_partition() -> None:
    # reference tests/test_cuda.py:160-183: whatever the data (ties included), the gradient is
    # the block average over the blocks the GPU's fit reports.
    rng = np.random.default_rng(3)
    for y in (
        np.round(rng.standard_normal((500, 24)) * 2),  # many exact ties
        np.ones((50, 32)),
        np.broadcast_to(np.arange(19.0), (40, 19)).copy(),
    ):
        w = rng.random(y.shape) + 0.1
        c = rng.standard_normal(y.shape)
        yy = torch.from_numpy(y).cuda().requires_grad_()
        for weights in (w, None):
            ww = None if weights is None else torch.from_numpy(weights).cuda().requires_grad_()
            fit = torchisotonic_amd.isotonic(yy, ww)
            inputs = (yy,) if ww is None else (yy, ww)
            got = torch.autograd.grad((fit * torch.from_numpy(c).cuda()).sum(), inputs)
            _, starts = _ext.isotonic_tiles(yy.detach(), None if ww is None else ww.detach(), True, True, True)
            s = starts.cpu().numpy().astype(np.uint8)
            ey, ew = oracle.block_grad(s, c, weights, y, fit.detach().cpu().numpy(), want_w=weights is not None)
            np.testing.assert_allclose(got[0].cpu().numpy(), ey, rtol=1e-12, atol=1e-12)
            if ww is not None:
                np.testing.assert_allclose(got[1].cpu().numpy(), ew, rtol=1e-9, atol=1e-9)


def test_clamp_gradient_matches_torch_clamp() -> None:
    # The fused clamp's backward is torch.clamp's: a block passes the gradient where
    # y_min <= fit <= y_max (equality included), and gw uses the unclamped fit.
    rng = np.random.default_rng(5)
    y = np.round(rng.standard_normal((400, 12)) * 2) / 2  # fits land exactly on the bounds
    w = rng.random(y.shape) + 0.1
    c = rng.standard_normal(y.shape)
    for lo, hi in ((-0.5, 0.5), (0.0, None), (None, 1.0), (1.0, -1.0)):
        yy = torch.from_numpy(y).cuda().requires_grad_()
        ww = torch.from_numpy(w).cuda().requires_grad_()
        out = torchisotonic_amd.isotonic(yy, ww, y_min=lo, y_max=hi)
        gy, gw = torch.autograd.grad((out * torch.from_numpy(c).cuda()).sum(), (yy, ww))
        # the same through an unclamped fit and torch's own clamp
        yy2 = torch.from_numpy(y).cuda().requires_grad_()
        ww2 = torch.from_numpy(w).cuda().requires_grad_()
        out2 = torchisotonic_amd.isotonic(yy2, ww2).clamp(min=lo, max=hi)
        gy2, gw2 = torch.autograd.grad((out2 * torch.from_numpy(c).cuda()).sum(), (yy2, ww2))
        torch.testing.assert_close(out, out2, rtol=0, atol=0)
        torch.testing.assert_close(gy, gy2, rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(gw, gw2, rtol=1e-12, atol=1e-12)


def test_nan_row_gradients() -> None:
    # CPU semantics (reference _api.py:92-97, pava.h:29-38): a NaN row is one block, so gy is
    # the row's average gradient and gw is NaN; through a clamp the row passes nothing.
    y = torch.tensor([[3.0, float("nan"), 2.0], [3.0, 1.0, 2.0]], dtype=torch.float64, device="cuda")
    w = torch.tensor([[1.0, 2.0, 3.0], [1.0, 1.0, 1.0]], dtype=torch.float64, device="cuda")
    c = torch.tensor([[1.0, 2.0, 6.0], [1.0, 2.0, 6.0]], dtype=torch.float64, device="cuda")
    yy, ww = y.clone().requires_grad_(), w.clone().requires_grad_()
    gy, gw = torch.autograd.grad((torchisotonic_amd.isotonic(yy, ww) * c).sum(), (yy, ww))
    torch.testing.assert_close(gy[0].cpu(), torch.tensor([1.0, 2.0, 3.0], dtype=torch.float64) * 9 / 6)
    assert gw[0].isnan().all()
    yy, ww = y.clone().requires_grad_(), w.clone().requires_grad_()
    gy, gw = torch.autograd.grad((torchisotonic_amd.isotonic(yy, ww, y_min=0.0) * c).sum(), (yy, ww))
    assert (gy[0] == 0).all() and gw[0].isnan().all()


def test_dtype_and_no_grad() -> None:
    # reference tests/test_grad.py:65-69
    y = torch.randn(2, 20, device="cuda", requires_grad=True)
    (grad,) = torch.autograd.grad(torchisotonic_amd.isotonic(y).sum(), (y,))
    assert grad.dtype == torch.float32
    assert not torchisotonic_amd.isotonic(torch.randn(2, 5, device="cuda")).requires_grad


@pytest.mark.parametrize("n", [12, 700, 9000])
def test_partial_requires_grad_and_broadcast_weights(n: int) -> None:
    # the C++ autograd node: only w differentiable, only y differentiable (w given), a weight
    # broadcast from one row (its gradient summed over the rows by autograd), and two backward
    # passes through one graph, on short, single-tile and multi-tile rows
    print(f"partial grads n={n}", flush=True)
    rng = np.random.default_rng(n)
    y = rng.standard_normal((3, n))
    wrow = rng.random(n) + 0.1
    c = rng.standard_normal((3, n))
    fit, starts = oracle.pava(y, np.broadcast_to(wrow, (3, n)))
    ey, ew = oracle.block_grad(starts, c, np.broadcast_to(wrow, (3, n)), y, fit, want_w=True)
    yt, ct = torch.from_numpy(y).cuda(), torch.from_numpy(c).cuda()
    wt = torch.from_numpy(wrow).cuda().requires_grad_()
    (gw,) = torch.autograd.grad((torchisotonic_amd.isotonic(yt, wt) * ct).sum(), (wt,))
    np.testing.assert_allclose(gw.cpu().numpy(), ew.sum(0), rtol=1e-9, atol=1e-9)
    yy = yt.clone().requires_grad_()
    out = torchisotonic_amd.isotonic(yy, wt.detach())
    assert out.requires_grad
    loss = (out * ct).sum()
    (g1,) = torch.autograd.grad(loss, (yy,), retain_graph=True)
    (g2,) = torch.autograd.grad(loss, (yy,))
    np.testing.assert_allclose(g1.cpu().numpy(), ey, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(g1, g2, rtol=0, atol=0)
