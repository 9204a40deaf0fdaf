"""The benchmarked C2 forward + backward at full size, and the reference suite's edge cases at
the sizes where they reach the merge levels, through the public API on the GPU:

- C2, [1e6, 16] float32 decreasing, forward + backward with g ~ N(0, 1) (seed 1), as bench.py
  times it; and a weighted, clamped variant of 700 000 rows, past the 524 288 rows that the
  short-row backward's resident grid covers in one pass;
- float32 monotonicity where neighbouring slopes are within an ulp (reference
  tests/test_cuda.py:224-240, at n = 1000 and 100 000, three weightings);
- close values: strictly increasing rows whose neighbours are a few ulp apart are their own fit
  and pass the gradient unchanged (reference tests/test_grad.py:40-56, tests/test_cuda.py:213-222,
  the row of linspace(0, 1, 1e6) included);
- blocks whose means all round to 1.0 in float32: the gradient takes its blocks from the hull,
  not from equal fitted values (reference tests/test_cuda.py:268-294, n = 500, 3000, 100 000);
- rows of a batch are independent: rows of magnitude 1e30 beside ordinary ones, in every way
  the kernels share a wave or a workgroup between rows (one row a lane, several rows a wave,
  one row a wave), leave the ordinary rows' fits and gradients as they are alone.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import torchisotonic_amd
from gpu_util import tolerance

pytestmark = pytest.mark.gpu


def c2_rows(b: int, dtype: type = np.float32) -> np.ndarray:
    rng = np.random.default_rng(0)
    return (-0.1 * np.arange(16) + rng.standard_normal((b, 16))).astype(dtype)


def test_c2_forward_backward_full_size() -> None:
    # bench.py's C2 step: isotonic + autograd.grad of y, g ~ N(0, 1) seed 1
    print("C2 fwd+bwd [1e6, 16] float32", flush=True)
    b, n = 1_000_000, 16
    y = c2_rows(b)
    g = np.random.default_rng(1).standard_normal((b, n)).astype(np.float32)
    yt = torch.from_numpy(y).cuda().requires_grad_()
    fit = torchisotonic_amd.isotonic(yt, increasing=False)
    (gy,) = torch.autograd.grad(fit, (yt,), torch.from_numpy(g).cuda())
    want, starts = oracle.pava(y, None, increasing=False, acc="f64")
    assert float(np.abs(fit.detach().cpu().numpy() - want).max()) <= tolerance(y)
    ey, _ = oracle.block_grad(starts, g.astype(np.float64))
    got = gy.cpu().numpy()
    # G / count in float64, rounded once to float32
    np.testing.assert_allclose(got, ey, rtol=2.0**-23, atol=1e-30)
    # a block of one element passes g through exactly
    single = (starts == 1) & (np.concatenate([starts[:, 1:], np.ones((b, 1), np.uint8)], axis=1) == 1)
    assert np.array_equal(got[single.astype(bool)], g[single.astype(bool)])


@pytest.mark.parametrize("increasing", [False, True])
def test_short_rows_weighted_clamped_past_one_pass(increasing: bool) -> None:
    # 700 000 weighted rows of 16: blocks of 256 rows beyond the first 2048 x 256 take the
    # backward kernel's second pass; the clamp bounds cut through many blocks.
    print(f"short weighted clamped fwd+bwd [700000, 16] increasing={increasing}", flush=True)
    b, n = 700_000, 16
    rng = np.random.default_rng(5)
    y = (-0.1 * np.arange(n) + rng.standard_normal((b, n))).astype(np.float32)
    w = (rng.random((b, n)) + 0.1).astype(np.float32)
    g = rng.standard_normal((b, n)).astype(np.float32)
    lo, hi = -0.8, 0.4
    yt = torch.from_numpy(y).cuda().requires_grad_()
    wt = torch.from_numpy(w).cuda().requires_grad_()
    fit = torchisotonic_amd.isotonic(yt, wt, increasing=increasing, y_min=lo, y_max=hi)
    gy, gw = torch.autograd.grad(fit, (yt, wt), torch.from_numpy(g).cuda())
    y64, w64 = y.astype(np.float64), w.astype(np.float64)
    want, starts = oracle.pava(y64, w64, increasing=increasing)
    clamped = np.clip(want, lo, hi)
    assert float(np.abs(fit.detach().cpu().numpy() - clamped).max()) <= tolerance(y)
    mask = (want >= lo) & (want <= hi)
    assert 0.2 < mask.mean() < 0.9  # the clamp matters here
    ey, ew = oracle.block_grad(starts, g.astype(np.float64) * mask, w64, y64, want, want_w=True)
    np.testing.assert_allclose(gy.cpu().numpy(), ey, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(gw.cpu().numpy(), ew, rtol=1e-5, atol=1e-5 * (1 + float(np.abs(y).max())))


def monotone_rows(name: str, n: int) -> tuple[torch.Tensor, torch.Tensor]:
    # reference tests/test_cuda.py:224-240: the same three rows from the same seeds
    g = torch.Generator().manual_seed(n)
    i = torch.arange(n, dtype=torch.float64)
    one = torch.tensor(1.0).view(torch.int32)
    y = {
        "collinear": 1e6 + 1e-3 * i + 1e-9 * torch.randn(n, generator=g, dtype=torch.float64),
        "offset": 1e6 + torch.randn(n, generator=g, dtype=torch.float64),
        "consecutive": (one + torch.arange(n, dtype=torch.int32)).view(torch.float32).double(),
    }[name].float()
    u = torch.rand(n, generator=g)
    return y, u


@pytest.mark.parametrize("name", ["collinear", "offset", "consecutive"])
@pytest.mark.parametrize("n", [1000, 100_000])
def test_float32_fit_is_monotone(name: str, n: int) -> None:
    print(f"float32 monotone {name} n={n}", flush=True)
    y, u = monotone_rows(name, n)
    for w in (None, u + 0.1, torch.exp(8 * u)):
        fit = torchisotonic_amd.isotonic(y.cuda(), None if w is None else w.cuda()).cpu()
        assert bool((fit[1:] >= fit[:-1]).all())
        want, _ = oracle.pava(y.numpy(), None if w is None else w.numpy(), acc="f64")
        assert float(np.abs(fit.numpy() - want).max()) <= tolerance(y.numpy())


def close_values() -> list[torch.Tensor]:
    # reference tests/test_grad.py:40-45
    one = torch.tensor(1.0).view(torch.int32)
    consecutive = (one + torch.arange(1000, dtype=torch.int32)).view(torch.float32)
    return [consecutive[None], torch.linspace(0, 1, 10**6)[None]]


@pytest.mark.parametrize("row", range(2))
@pytest.mark.parametrize("batch", [1, 3])
def test_close_values_are_separate_blocks(row: int, batch: int) -> None:
    print(f"close values row={row} batch={batch}", flush=True)
    y = close_values()[row].expand(batch, -1).contiguous().cuda().requires_grad_()
    c = torch.randn(y.shape, generator=torch.Generator().manual_seed(row)).cuda()
    out = torchisotonic_amd.isotonic(y)
    assert torch.equal(out, y)
    (grad,) = torch.autograd.grad((out * c).sum(), (y,))
    assert torch.equal(grad, c)
    # every element starts a block, and the stateless gradient over that partition passes c
    fit, starts = torchisotonic_amd._ext.isotonic_tiles(y.detach(), None, True, True, True)
    assert bool(starts.all())
    gy = torchisotonic_amd._ext.isotonic_grad(fit, starts, c, None, None)[0]
    assert torch.equal(gy, c)


def hull_blocks(n: int) -> tuple[np.ndarray, np.ndarray, int]:
    # reference tests/test_cuda.py:268-283: blocks (1 + u, 1, ..., 1) of s elements, s falling
    # from S to 3, then 2, 3, ... one block per element
    sizes: list[int] = []
    while sum(sizes) + len(sizes) + 3 <= n:
        sizes.append(len(sizes) + 3)
    sizes.reverse()
    u = np.finfo(np.float32).eps
    y = np.ones(n, np.float32)
    starts = np.ones(n, np.uint8)
    at = 0
    for size in sizes:
        y[at] = 1 + u
        starts[at + 1 : at + size] = 0
        at += size
    y[at:] = np.arange(2, 2 + n - at, dtype=np.float32)
    return y[None], starts[None], at


@pytest.mark.parametrize("n", [500, 3000, 100_000])
def test_gradient_blocks_from_the_hull(n: int) -> None:
    print(f"hull blocks n={n}", flush=True)
    y, starts, at = hull_blocks(n)
    # the constructed partition is the exact one (long double PAVA on these float32 values)
    _, want_starts = oracle.pava(y, acc="f64x")
    np.testing.assert_array_equal(want_starts, starts)
    c = torch.randn(1, n, generator=torch.Generator().manual_seed(n))
    yy = torch.from_numpy(y).cuda().requires_grad_()
    fit = torchisotonic_amd.isotonic(yy)
    assert bool((fit[:, :at] == 1).all())  # the case this test is about
    (grad,) = torch.autograd.grad((fit * c.cuda()).sum(), (yy,))
    ey, _ = oracle.block_grad(starts, c.double().numpy())
    np.testing.assert_allclose(grad.cpu().numpy(), ey, rtol=1e-5, atol=1e-6)
    got_starts = torchisotonic_amd._ext.isotonic_tiles(yy.detach(), None, True, True, True)[1]
    np.testing.assert_array_equal(got_starts.cpu().numpy().astype(np.uint8), starts)


# (batch, n): rows of 32 one a lane (short kernel); 64 one a lane in batches of 8192 ("packed");
# 128 in a batch of 2 (16 spans a row, 4 rows a wave), 300 in 64 (4 rows a wave), 2000 in 1000
# (2 rows a wave); 5000 one row a wave
INDEPENDENCE_SHAPES = [(1000, 32), (8192, 64), (2, 128), (64, 300), (1000, 2000), (4, 5000)]


@pytest.mark.parametrize("batch,n", INDEPENDENCE_SHAPES)
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("weighted", [False, True])
def test_rows_are_independent_of_their_neighbours_magnitude(batch: int, n: int, dtype: type,
                                                             weighted: bool) -> None:
    print(f"row independence [{batch}, {n}] {np.dtype(dtype).name} weighted={weighted}", flush=True)
    rng = np.random.default_rng(batch + n)
    y = (0.01 * np.arange(n) + rng.standard_normal((batch, n))).astype(dtype)
    huge = np.zeros(batch, dtype=bool)
    huge[::3] = True  # every third row, the first included: 1e30 times larger, in runs of 1e30
    y[huge] = (y[huge].astype(np.float64) * 1e30).astype(dtype)
    w = (rng.random((batch, n)) + 0.1).astype(dtype) if weighted else None
    g = rng.standard_normal((batch, n)).astype(dtype)
    yt = torch.from_numpy(y).cuda().requires_grad_()
    wt = None if w is None else torch.from_numpy(w).cuda().requires_grad_()
    fit = torchisotonic_amd.isotonic(yt, weight=wt)
    grads = torch.autograd.grad(fit, [yt] + ([] if wt is None else [wt]), torch.from_numpy(g).cuda())
    want, starts = oracle.pava(y, w, acc="f64")
    ey, ew = oracle.block_grad(starts, g.astype(np.float64), None if w is None else w.astype(np.float64),
                               None if w is None else y.astype(np.float64), want, want_w=w is not None)
    got = fit.detach().cpu().numpy().astype(np.float64)
    tol = 4 * 2.0**-23 if dtype == np.float32 else 1e-12
    # each row within its own tolerance (its own magnitude), the ordinary rows above all
    scale = np.abs(y.astype(np.float64)).max(axis=1, keepdims=True)
    assert (np.abs(got - want) <= tol * scale).all(), float((np.abs(got - want) / scale).max())
    gtol = 1e-5 if dtype == np.float32 else 1e-11
    for gt, e in zip(grads, (ey, ew)):
        gt = gt.cpu().numpy().astype(np.float64)
        rscale = np.abs(e).max(axis=1, keepdims=True)
        assert (np.abs(gt - e) <= gtol * (np.abs(e) + rscale)).all(), float((np.abs(gt - e) / rscale).max())
