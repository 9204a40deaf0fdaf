"""Short rows (n <= 32, one thread per row) on the GPU against the oracle, the golden vectors
and the reference's known answers (reference tests/test_cuda.py:31-134, test_isotonic.py,
test_grad.py restated for the HIP path)."""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
import torchisotonic_amd
from gpu_util import check_fit, gpu_fit, tolerance

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def data(batch: int, n: int, dtype: type, seed: int) -> tuple[np.ndarray, np.ndarray]:
    rng = np.random.default_rng(seed)
    y = (np.linspace(0, 3, n) + rng.standard_normal((batch, n))).astype(dtype)
    w = (rng.random((batch, n)) + 0.1).astype(dtype)
    return y, w


@pytest.mark.parametrize("batch", [1, 129, 5000])
@pytest.mark.parametrize("n", [1, 2, 3, 7, 16, 17, 31, 32])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_matches_oracle(batch: int, n: int, dtype: type) -> None:
    print(f"short fit batch={batch} n={n} dtype={np.dtype(dtype).name}", flush=True)
    y, w = data(batch, n, dtype, batch * 1000 + n)
    check_fit(y)
    check_fit(y, w)
    check_fit(y, w, increasing=False)
    check_fit(y, None, increasing=False, y_min=-0.5, y_max=2.0)


def _golden_groups(name: str):
    d = np.load(GOLDEN / name, allow_pickle=False)
    off = d["offsets"]
    for k in range(len(off) - 1):
        n = off[k + 1] - off[k]
        if 1 <= n <= 32:
            yield k, d, slice(off[k], off[k + 1])


def test_scipy_golden_vectors() -> None:
    for k, d, sl in _golden_groups("scipy_fits.npz"):
        y = d["y"][sl][None]
        w = d["w"][sl][None] if d["weighted"][k] else None
        got, starts = gpu_fit(y, w, bool(d["increasing"][k]))
        np.testing.assert_allclose(got[0], d["x"][sl], rtol=1e-12, atol=1e-9)
        blocks = np.concatenate([np.flatnonzero(starts[0]), [y.shape[1]]])
        bo = d["block_offsets"]
        np.testing.assert_array_equal(blocks, d["blocks"][bo[k] : bo[k + 1]])


def test_sklearn_golden_clip() -> None:
    for k, d, sl in _golden_groups("sklearn_clip.npz"):
        y = d["y"][sl][None]
        w = d["w"][sl][None] if d["weighted"][k] else None
        lo, hi = float(d["y_min"][k]), float(d["y_max"][k])
        got, _ = gpu_fit(
            y, w, bool(d["increasing"][k]),
            None if math.isnan(lo) else lo, None if math.isnan(hi) else hi,
        )
        np.testing.assert_allclose(got[0], d["x"][sl], rtol=1e-12, atol=1e-9)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32, torch.float64])
def test_keeps_float_dtype(dtype: torch.dtype) -> None:
    # reference tests/test_isotonic.py:127-134
    got = torchisotonic_amd.isotonic(torch.tensor([3.0, 1.0, 2.0, 5.0], dtype=dtype, device="cuda"))
    assert got.dtype == dtype and got.is_cuda
    torch.testing.assert_close(got.double().cpu(), torch.tensor([2.0, 2.0, 2.0, 5.0], dtype=torch.float64))


def test_integers_become_default_float() -> None:
    got = torchisotonic_amd.isotonic(torch.tensor([3, 1, 2], device="cuda"))
    assert got.dtype == torch.get_default_dtype()
    torch.testing.assert_close(got.cpu(), torch.tensor([2.0, 2.0, 2.0]))


def test_single_element_and_empty() -> None:
    got = torchisotonic_amd.isotonic(torch.tensor([4.0], device="cuda"))
    torch.testing.assert_close(got.cpu(), torch.tensor([4.0]))
    for shape in [(0,), (3, 0), (0, 5)]:
        assert torchisotonic_amd.isotonic(torch.empty(shape, device="cuda")).shape == shape


def test_nan_rows() -> None:
    rng = np.random.default_rng(11)
    y = rng.standard_normal((300, 20))
    y[7, 3] = np.nan
    y[299, 19] = np.nan
    check_fit(y)
    check_fit(y.astype(np.float32), rng.random((300, 20)).astype(np.float32) + 0.1, increasing=False)


@pytest.mark.parametrize("dim", [0, 1, 2, -1])
def test_batch_along_any_dim(dim: int) -> None:
    torch.manual_seed(0)
    y = torch.randn(3, 4, 20, dtype=torch.float64).movedim(-1, dim)
    w = torch.rand_like(y) + 0.1
    got = torchisotonic_amd.isotonic(y.cuda(), w.cuda(), dim=dim).cpu()
    ry, rw = (t.movedim(dim, -1).reshape(-1, 20).numpy() for t in (y, w))
    want, _ = oracle.pava(ry, rw)
    np.testing.assert_allclose(got.movedim(dim, -1).reshape(-1, 20).numpy(), want, rtol=0, atol=1e-12 * 5)


def test_weight_broadcasts_and_must_be_positive() -> None:
    y = torch.tensor([[3.0, 1.0, 2.0], [1.0, 3.0, 2.0]], dtype=torch.float64, device="cuda")
    w = torch.tensor([1.0, 2.0, 3.0], dtype=torch.float64, device="cuda")
    got = torchisotonic_amd.isotonic(y, w).cpu().numpy()
    want, _ = oracle.pava(y.cpu().numpy(), np.broadcast_to(w.cpu().numpy(), (2, 3)))
    np.testing.assert_allclose(got, want, rtol=1e-14)
    for bad in (0.0, -1.0, math.nan):
        with pytest.raises(ValueError, match="strictly positive"):
            torchisotonic_amd.isotonic(y, torch.tensor([1.0, bad, 1.0], device="cuda"))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_c2_full_size_and_padded_variant(dtype: type) -> None:
    # y[b, i] = -0.1 i + N(0, 1), [1e6, 16], decreasing, unweighted.
    rng = np.random.default_rng(0)
    b, n = 1_000_000, 16
    y = (-0.1 * np.arange(n) + rng.standard_normal((b, n))).astype(dtype)
    print(f"C2 full size dtype={np.dtype(dtype).name}", flush=True)
    got, starts = check_fit(y, increasing=False)
    # padded variant: true lengths U{4..16}, the tail padded with (row min - 1), which never
    # pools with the data of a decreasing fit; the first len values are the unpadded fit.
    lens = np.random.default_rng(2).integers(4, 17, b)
    pad = y.copy()
    mask = np.arange(n)[None, :] >= lens[:, None]
    mins = np.where(~mask, y, np.inf).min(axis=1)
    pad[mask] = np.broadcast_to((mins - 1)[:, None], (b, n))[mask]
    pgot, _ = gpu_fit(pad, None, increasing=False, with_starts=False)
    for length in (4, 9, 16):
        rows = np.flatnonzero(lens == length)[:2000]
        sub = np.ascontiguousarray(y[rows, :length])
        want, _ = oracle.pava(sub, increasing=False, acc="f64")
        assert np.abs(pgot[rows, :length] - want).max() <= tolerance(sub)


@pytest.mark.parametrize("name", ["collinear", "offset", "consecutive"])
def test_float32_fit_is_monotone(name: str) -> None:
    # reference tests/test_cuda.py:224-240, at short-row lengths
    rng = np.random.default_rng(1)
    b, n = 4096, 32
    i = np.arange(n, dtype=np.float64)
    one = np.float32(1.0).view(np.int32)
    y = {
        "collinear": 1e6 + 1e-3 * i + 1e-9 * rng.standard_normal((b, n)),
        "offset": 1e6 + rng.standard_normal((b, n)),
        "consecutive": np.broadcast_to((one + np.arange(n, dtype=np.int32)).view(np.float32).astype(np.float64), (b, n)),
    }[name].astype(np.float32)
    u = rng.random((b, n))
    for w in (None, (u + 0.1).astype(np.float32), np.exp(8 * u).astype(np.float32)):
        got, _ = gpu_fit(y, w, with_starts=False)
        assert (np.diff(got, axis=1) >= 0).all()


def test_close_values_are_separate_blocks() -> None:
    # reference tests/test_grad.py:40-56, at a short-row length: increasing data is its own
    # fit, every element its own block, and the gradient passes unchanged.
    one = torch.tensor(1.0).view(torch.int32)
    row = (one + torch.arange(32, dtype=torch.int32)).view(torch.float32)
    y = row.expand(64, -1).contiguous().cuda().requires_grad_()
    c = torch.randn(y.shape, generator=torch.Generator().manual_seed(0)).cuda()
    out = torchisotonic_amd.isotonic(y)
    assert torch.equal(out, y)
    (grad,) = torch.autograd.grad((out * c).sum(), (y,))
    assert torch.equal(grad, c)


@pytest.mark.parametrize("n", [3, 8, 16, 32])
def test_unaligned_and_offset_inputs(n: int) -> None:
    # Tensors that start off a 16-byte boundary (views with a storage offset) take the
    # per-element staging path and must give the same fit and gradients.
    rng = np.random.default_rng(n)
    b = 777
    flat = rng.standard_normal(b * n + 1).astype(np.float32)
    wflat = (rng.random(b * n + 1) + 0.1).astype(np.float32)
    yt = torch.from_numpy(flat).cuda()[1:].view(b, n)
    wt = torch.from_numpy(wflat).cuda()[1:].view(b, n)
    assert yt.data_ptr() % 16 != 0
    for w in (None, wt):
        got = torchisotonic_amd.isotonic(yt, w, increasing=False).cpu().numpy()
        want, _ = oracle.pava(
            flat[1:].reshape(b, n), None if w is None else wflat[1:].reshape(b, n),
            increasing=False, acc="f64",
        )
        assert np.abs(got - want).max() <= tolerance(flat)
    yr = yt.clone()[:, :]  # aligned copy for the reference gradient
    g = torch.from_numpy(rng.standard_normal((b, n)).astype(np.float32)).cuda()
    y1 = yt.detach().requires_grad_()
    (g1,) = torch.autograd.grad(torchisotonic_amd.isotonic(y1), (y1,), g)
    y2 = yr.detach().requires_grad_()
    (g2,) = torch.autograd.grad(torchisotonic_amd.isotonic(y2), (y2,), g)
    torch.testing.assert_close(g1, g2, rtol=0, atol=0)
