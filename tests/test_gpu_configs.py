"""The workloads bench.py measures, at (or near) their full size on the GPU, against the
oracle: the fit, its partition and the gradients, on the data each workload names (the
reference measures the same kind of batch x n grid, bench/bench.py:31-42, 108-110)."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from gpu_util import check_fit

pytestmark = pytest.mark.gpu


def grads(y, w, c, **kw):
    import torch

    import torchisotonic_amd

    yy = torch.from_numpy(y).cuda().requires_grad_()
    ww = None if w is None else torch.from_numpy(w).cuda().requires_grad_()
    fit = torchisotonic_amd.isotonic(yy, ww, **kw)
    inputs = (yy,) if ww is None else (yy, ww)
    gs = torch.autograd.grad((fit * torch.from_numpy(c).cuda()).sum(), inputs)
    return [x.cpu().numpy() for x in gs], fit.detach().cpu().numpy()


def test_c1_plumbing() -> None:
    # [1000, 5000] float32, 0.001 i + N(0, 1), unweighted, increasing: one wave per row, its
    # lanes' spans merged in the span kernel
    print("config c1", flush=True)
    rng = np.random.default_rng(0)
    y = (0.001 * np.arange(5000) + rng.standard_normal((1000, 5000))).astype(np.float32)
    check_fit(y)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_c3_weighted_clipped(dtype: type) -> None:
    # [1000, 5000] sigmoid(linspace(-4, 4) + N(0, 0.5)), w = U(0, 1) + 0.1, decreasing, clamped
    # to [0, 1]; forward and both gradients
    print(f"config c3 {np.dtype(dtype).name}", flush=True)
    rng = np.random.default_rng(3)
    n = 5000
    y = (1 / (1 + np.exp(-(np.linspace(-4, 4, n) + 0.5 * rng.standard_normal((1000, n)))))).astype(dtype)
    w = (rng.random((1000, n)) + 0.1).astype(dtype)
    check_fit(y, w, increasing=False, y_min=0.0, y_max=1.0)
    c = rng.standard_normal((1000, n)).astype(dtype)
    (gy, gw), fit = grads(y, w, c, increasing=False, y_min=0.0, y_max=1.0)
    want, starts = oracle.pava(y.astype(np.float64), w.astype(np.float64), increasing=False)
    assert ((want > 0.0) & (want < 1.0)).all()  # the clamp holds no block here: mask 1
    ey, ew = oracle.block_grad(starts, c.astype(np.float64), w.astype(np.float64), y.astype(np.float64),
                               want, want_w=True)
    tol = 1e-10 if dtype == np.float64 else 2e-5
    np.testing.assert_allclose(gy, ey, rtol=tol, atol=tol)
    np.testing.assert_allclose(gw, ew, rtol=tol, atol=tol)


def test_c5_bootstrap_rows() -> None:
    # shared labels Bernoulli(sigmoid(linspace(-4, 4, 65536))), per-row weights Exponential(1)
    # floored at 1e-6, increasing; 64 of the configuration's 1000 rows, forward and gradients
    print("config c5", flush=True)
    rng = np.random.default_rng(5)
    n = 65536
    lab = (rng.random(n) < 1 / (1 + np.exp(-np.linspace(-4, 4, n)))).astype(np.float32)
    y = np.broadcast_to(lab, (64, n)).copy()
    w = np.maximum(rng.exponential(1.0, (64, n)), 1e-6).astype(np.float32)
    # labels tie everywhere: the partition is not unique, so the fit alone is compared
    check_fit(y, w, check_starts=False)
    c = rng.standard_normal((64, n)).astype(np.float32)
    (gy, gw), fit = grads(y, w, c)
    # the gradient is the block average over the GPU's own blocks (as the fit reports them)
    from gpu_util import gpu_fit

    _, starts = gpu_fit(y, w)
    ey, ew = oracle.block_grad(starts, c.astype(np.float64), w.astype(np.float64), y.astype(np.float64),
                               fit.astype(np.float64), want_w=True)
    np.testing.assert_allclose(gy, ey, rtol=2e-5, atol=2e-5)
    np.testing.assert_allclose(gw, ew, rtol=2e-5, atol=2e-5)


@pytest.mark.parametrize(("batch", "n"), [(1000, 5000), (100_000, 16), (3, 70_000)])
def test_exact_false_through_the_api(batch: int, n: int) -> None:
    # exact=False (C3's float32 leg in the reference) gives the exact path's results bit for
    # bit, fit and gradients, and so meets the reference's exact=False bar: within 1e-4 of the
    # float32-accumulating CPU path (reference tests/test_cuda.py:26-28)
    import torch

    import torchisotonic_amd

    print(f"exact=False {batch}x{n}", flush=True)
    rng = np.random.default_rng(n)
    y = (1 / (1 + np.exp(-(np.linspace(-4, 4, n) + 0.5 * rng.standard_normal((batch, n)))))).astype(np.float32)
    w = (rng.random((batch, n)) + 0.1).astype(np.float32)
    c = torch.from_numpy(rng.standard_normal((batch, n)).astype(np.float32)).cuda()
    out = {}
    for exact in (True, False):
        yy = torch.from_numpy(y).cuda().requires_grad_()
        ww = torch.from_numpy(w).cuda().requires_grad_()
        fit = torchisotonic_amd.isotonic(yy, ww, increasing=False, y_min=0.0, y_max=1.0, exact=exact)
        out[exact] = (fit.detach(), *torch.autograd.grad((fit * c).sum(), (yy, ww)))
    for a, b in zip(out[True], out[False]):
        assert torch.equal(a, b)
    ref32, _ = oracle.pava(y, w, increasing=False)
    np.testing.assert_allclose(out[False][0].cpu().numpy(), np.clip(ref32, 0.0, 1.0), rtol=1e-4, atol=1e-4)
