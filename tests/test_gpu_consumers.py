"""The consumers either side of the fit on the GPU against the oracle: soft ranks forward and
backward at the reference's shapes and strengths (reference paper/soft_rank.py:22-28), and
isotonic calibration (fit over pooled keys, then interpolation) against the oracle and
scikit-learn's IsotonicRegression (committed golden vectors)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from torchisotonic_amd import _ext
from torchisotonic_amd.calibration import IsotonicCalibrator, calibration_fit, calibration_predict
from torchisotonic_amd.soft_rank import soft_rank

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def say(*a: object) -> None:
    print(*a, flush=True)


# (batch, n): the reference's soft-rank shapes, and strengths 1 and 1/n
SHAPES = [(1024, 100), (256, 1000), (64, 10_000), (8, 100_000), (1, 1_000_000)]


@pytest.mark.parametrize(("batch", "n"), SHAPES)
@pytest.mark.parametrize("strength", ["1", "1/n"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_soft_rank_matches_oracle(batch: int, n: int, strength: str, dtype: torch.dtype) -> None:
    eps = 1.0 if strength == "1" else 1.0 / n
    say(f"soft rank {batch}x{n} eps={strength} {dtype}")
    gen = torch.Generator().manual_seed(batch + n)
    x = torch.randn(batch, n, generator=gen, dtype=torch.float64)
    g = torch.randn(batch, n, generator=gen, dtype=torch.float64)
    xr = x.to(dtype).cuda().requires_grad_()
    r = soft_rank(xr, eps)
    (dx,) = torch.autograd.grad(r, xr, g.to(dtype).cuda())
    # the oracle on the same inputs, its tensor steps rounded in the same dtype (so its dual
    # has the GPU's partition); sums and the fit in float64
    npdt = np.float32 if dtype == torch.float32 else np.float64
    xx = xr.detach().cpu().numpy()
    want, _ = oracle.soft_rank(xx, eps, npdt)
    want_dx = oracle.soft_rank_vjp(xx, eps, g.to(dtype).double().numpy(), npdt)
    scale = max(float(np.abs(xx).max()) / eps, float(n))  # the largest sort key or rank
    if dtype == torch.float64:
        tol_r, tol_g = 1e-12 * scale, 1e-10  # (the float64 fit bar: 1e-12 of the data scale)
    else:
        # float32: the dual is the float64 fit rounded once, the ranks one float32 difference
        tol_r, tol_g = 4 * 2.0**-23 * scale, 2e-5
    np.testing.assert_allclose(r.detach().double().cpu().numpy(), want.astype(np.float64), rtol=0, atol=tol_r)
    scale = float(np.abs(want_dx).max())
    np.testing.assert_allclose(dx.double().cpu().numpy(), want_dx, rtol=tol_g, atol=tol_g * scale)


# A single row of 2^18 .. 2^20 elements is sorted padded with -inf to 2^20 + 1 (the size from
# which the sort library's faster algorithm runs): rows at both ends of that range and one past
# it, with many ties (the padded sort keeps their order, as the oracle's stable sort does; tied
# entries pool into one block of the decreasing fit, so their ranks do not depend on it).
@pytest.mark.parametrize("n", [1 << 18, 1 << 20, (1 << 20) + 1])
def test_soft_rank_single_row_padded_sort(n: int) -> None:
    say(f"soft rank 1x{n} with ties")
    gen = torch.Generator().manual_seed(n)
    x = torch.round(torch.randn(1, n, generator=gen, dtype=torch.float64) * 64) / 64
    g = torch.randn(1, n, generator=gen, dtype=torch.float64)
    xr = x.cuda().requires_grad_()
    r = soft_rank(xr, 1.0)
    (dx,) = torch.autograd.grad(r, xr, g.cuda())
    want, _ = oracle.soft_rank(x.numpy(), 1.0, np.float64)
    want_dx = oracle.soft_rank_vjp(x.numpy(), 1.0, g.numpy(), np.float64)
    scale = max(float(np.abs(x.numpy()).max()), float(n))
    np.testing.assert_allclose(r.detach().cpu().numpy(), want, rtol=0, atol=1e-12 * scale)
    np.testing.assert_allclose(dx.cpu().numpy(), want_dx, rtol=1e-10, atol=1e-10 * float(np.abs(want_dx).max()))


def test_soft_rank_limits_and_gradcheck() -> None:
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(6, 50, generator=gen, dtype=torch.float64).cuda()
    hard = torch.argsort(torch.argsort(x, -1), -1).double() + 1
    # (s - (s - w) with s near 1e9 is w to within the float64 spacing there)
    torch.testing.assert_close(soft_rank(x, 1e-9), hard, rtol=0, atol=1e-6)
    torch.testing.assert_close(soft_rank(x, 1e9), torch.full_like(x, 25.5), rtol=0, atol=1e-6)
    torch.testing.assert_close(soft_rank(x, 0.3).sum(-1), torch.full((6,), 50 * 51 / 2, dtype=torch.float64, device="cuda"))
    xs = torch.randn(2, 12, generator=gen, dtype=torch.float64).cuda().requires_grad_()
    assert torch.autograd.gradcheck(lambda t: soft_rank(t, 0.7), (xs,))


def test_soft_rank_backward_twice() -> None:
    # the graph is kept (as in the reference), so a second backward works
    x = torch.randn(3, 40, dtype=torch.float64, device="cuda").requires_grad_()
    r = soft_rank(x, 0.5)
    g = torch.randn_like(r)
    (a,) = torch.autograd.grad(r, x, g, retain_graph=True)
    (b,) = torch.autograd.grad(r, x, g)
    torch.testing.assert_close(a, b, rtol=0, atol=0)


# --- calibration ----------------------------------------------------------------------------------


def golden_calib():
    d = np.load(GOLDEN / "sklearn_calib.npz", allow_pickle=False)
    off, qoff = d["offsets"], d["q_offsets"]
    for k in range(len(off) - 1):
        sl, ql = slice(off[k], off[k + 1]), slice(qoff[k], qoff[k + 1])
        w = d["w"][sl] if d["weighted"][k] else None
        yield d["x"][sl], d["y"][sl], w, bool(d["increasing"][k]), d["q"][ql], d["pred"][ql]


def test_calibration_matches_sklearn_golden() -> None:
    say("calibration: sklearn golden vectors")
    for x, y, w, inc, q, pred in golden_calib():
        cal = IsotonicCalibrator(increasing=inc).fit(
            torch.from_numpy(x).cuda(), torch.from_numpy(y).cuda(), None if w is None else torch.from_numpy(w).cuda()
        )
        got = cal.predict(torch.from_numpy(q).cuda()).cpu().numpy()
        np.testing.assert_allclose(got, pred, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("n", [1000, 200_000, 5_000_000])
def test_calibration_matches_oracle(n: int) -> None:
    # scores with heavy ties (rounded), 0/1 labels, optional weights: knots against the oracle,
    # predictions bit for bit against the oracle's restatement of the reference formula
    say(f"calibration n={n}")
    rng = np.random.default_rng(n)
    s = np.round(rng.normal(0.0, 1.5, n), 3)
    y = (rng.random(n) < 1 / (1 + np.exp(-s))).astype(np.float64)
    w = rng.uniform(0.5, 2.0, n)
    for ww in (None, w):
        xp, fp = calibration_fit(torch.from_numpy(s).cuda(), torch.from_numpy(y).cuda(),
                                 None if ww is None else torch.from_numpy(ww).cuda())
        wxp, wfp = oracle.calibration_fit(s, y, ww)
        np.testing.assert_array_equal(xp.cpu().numpy(), wxp)
        np.testing.assert_allclose(fp.cpu().numpy(), wfp, rtol=0, atol=1e-12)
        q = np.concatenate([rng.normal(0.0, 2.0, 100_000), wxp, [np.nan, -np.inf, np.inf]])
        got = calibration_predict(torch.from_numpy(q).cuda(), xp, fp).cpu().numpy()
        want = oracle.interp(q, xp.cpu().numpy(), fp.cpu().numpy())
        np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_interp_kernel_is_the_reference_formula(dtype: torch.dtype) -> None:
    # ti_interp against the reference's tensor formula (calibrate.py:163-168) run with torch
    # ops on the same inputs, bit for bit, and against the oracle
    say(f"interp kernel {dtype}")
    gen = torch.Generator().manual_seed(5)
    xp = torch.sort(torch.randn(777, generator=gen, dtype=torch.float64))[0].to(dtype)
    fp = torch.cumsum(torch.rand(777, generator=gen, dtype=torch.float64), 0).to(dtype)
    x = (torch.randn(300_000, generator=gen, dtype=torch.float64) * 2).to(dtype)
    xd, xpd, fpd = x.cuda(), xp.cuda(), fp.cuda()
    i = torch.searchsorted(xpd, xd).clamp(1, len(xpd) - 1)
    x0, x1, f0, f1 = xpd[i - 1], xpd[i], fpd[i - 1], fpd[i]
    t = ((xd - x0) / (x1 - x0).clamp_min(1e-300)).clamp(0, 1)
    ref = f0 + t * (f1 - f0)
    got = _ext.interp(xd, xpd, fpd)
    assert torch.equal(got, ref)
    np.testing.assert_array_equal(got.cpu().numpy(), oracle.interp(x.numpy(), xp.numpy(), fp.numpy()))
    # one knot, and NaN
    one = _ext.interp(torch.tensor([-1.0, 3.0, float("nan")], dtype=dtype, device="cuda"),
                      torch.tensor([0.5], dtype=dtype, device="cuda"), torch.tensor([2.0], dtype=dtype, device="cuda"))
    assert one[:2].tolist() == [2.0, 2.0] and torch.isnan(one[2])


def _plain_interp(x: torch.Tensor, xp: torch.Tensor, fp: torch.Tensor) -> torch.Tensor:
    # ti_interp: the full binary search over all knots, no index
    out = torch.empty_like(x)
    code = _ext.F32 if x.dtype == torch.float32 else _ext.F64
    rc = _ext.load().ti_interp(x.data_ptr(), xp.data_ptr(), fp.data_ptr(), out.data_ptr(), x.numel(), xp.numel(),
                               code, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    return out


def _knot_sets(rng: np.random.Generator) -> dict[str, np.ndarray]:
    logit = rng.normal(-1.2, 1.5, 400_000)
    scores = np.unique((1 / (1 + np.exp(-logit))).astype(np.float32)).astype(np.float64)
    return {
        # float32 scores of a CTR model: dense in the middle, sparse in the tails
        "scores": scores,
        # uniform, and one dense cluster beside a far point (most knots in one bucket: searched)
        "uniform": np.sort(rng.random(300_000)),
        "cluster": np.r_[np.sort(rng.random(200_000) * 1e-6), 1e3],
        # repeated knots (non-decreasing), a few knots, two knots
        "repeats": np.sort(np.round(rng.normal(0, 1, 50_000), 2)),
        "few": np.sort(rng.normal(0, 1, 37)),
        "two": np.array([-1.0, 2.0]),
        # ends that give the index no scale: infinite or NaN last knot, all knots equal
        "inf_end": np.r_[np.sort(rng.random(5000)), np.inf],
        "nan_end": np.r_[np.sort(rng.random(5000)), np.nan],
        "equal": np.full(1000, 0.25),
    }


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_interp_index_gives_the_full_search_bit_for_bit(dtype: torch.dtype) -> None:
    # ti_interp_indexed against ti_interp on knot sets that stress the buckets (dense, sparse,
    # clustered, repeated, degenerate ends), at queries on, between and beyond the knots
    rng = np.random.default_rng(17)
    for name, xp_np in _knot_sets(rng).items():
        say(f"interp index {name} {dtype}")
        m = xp_np.size
        fin = xp_np[np.isfinite(xp_np)]
        lo, hi = fin.min(), fin.max()
        q = np.concatenate([
            rng.uniform(lo - 0.1 * (hi - lo + 1), hi + 0.1 * (hi - lo + 1), 200_000),
            xp_np, np.nextafter(fin, np.inf), np.nextafter(fin, -np.inf),
            [np.nan, -np.inf, np.inf, 0.0, -0.0, lo, hi],
        ])
        xp = torch.from_numpy(xp_np).to(dtype).cuda()
        fp = torch.cumsum(torch.rand(m, dtype=torch.float64, generator=torch.Generator().manual_seed(m)), 0)
        fp = fp.to(dtype).cuda()
        x = torch.from_numpy(q).to(dtype).cuda()
        want = _plain_interp(x, xp, fp)
        index = _ext.interp_index(xp)
        got = _ext.interp(x, xp, fp, index)
        torch.cuda.synchronize()
        assert torch.equal(got.isnan(), want.isnan()), name
        ok = ~want.isnan()
        assert torch.equal(got[ok], want[ok]), name
    # one index serves every later call; a smaller second call through the same index
    xp = torch.from_numpy(np.sort(rng.random(100_000))).to(dtype).cuda()
    fp = torch.rand(100_000, dtype=torch.float64).to(dtype).cuda()
    index = _ext.interp_index(xp)
    for n in (300_000, 1000):
        x = torch.rand(n, dtype=torch.float64).to(dtype).cuda()
        assert torch.equal(_ext.interp(x, xp, fp, index), _plain_interp(x, xp, fp))


def test_interp_ignores_an_index_of_other_knots() -> None:
    # An index built from float64 knots, used with float32 queries and knots (the calibrator's
    # index with float32 scores), or built from more knots: the kernel must not narrow by it,
    # so the result is the full search's.
    say("interp index of another dtype or knot count")
    rng = np.random.default_rng(23)
    xp64 = torch.from_numpy(np.unique(rng.random(200_000).astype(np.float32)).astype(np.float64)).cuda()
    # knots that round onto each other in float32, so float64 buckets misplace float32 values
    xp64 = torch.sort(torch.cat([xp64, xp64 + 1e-9])).values
    m = xp64.numel()
    fp64 = torch.cumsum(torch.rand(m, dtype=torch.float64, device="cuda"), 0)
    x32 = torch.from_numpy(np.r_[rng.random(100_000), xp64[::7].cpu().numpy()]).float().cuda()
    xp32, fp32 = xp64.float(), fp64.float()
    want = _plain_interp(x32, xp32, fp32)
    lib = _ext.load()
    stream = torch.cuda.current_stream().cuda_stream
    # (an index of fewer knots is refused outright: its buffer is smaller than m knots need)
    with pytest.raises(RuntimeError):
        _ext.interp(x32, xp32, fp32, _ext.interp_index(xp32[: m // 2]))
    for idx in (_ext.interp_index(xp64), _ext.interp_index(torch.cat([xp32, xp32 + 2]))):
        out = torch.empty_like(x32)
        rc = lib.ti_interp_indexed(x32.data_ptr(), xp32.data_ptr(), fp32.data_ptr(), idx.data_ptr(), idx.numel(),
                                   out.data_ptr(), x32.numel(), m, _ext.F32, stream)
        assert rc == 0
        assert torch.equal(out, want)
    # through the wrapper, a float64 index with float32 queries is built again in float32
    assert torch.equal(_ext.interp(x32, xp64, fp64, _ext.interp_index(xp64)), want)


def test_calibrator_keeps_its_knot_index() -> None:
    say("calibrator knot index")
    rng = np.random.default_rng(21)
    s = rng.random(100_000)
    y = (rng.random(100_000) < s).astype(np.float64)
    cal = IsotonicCalibrator().fit(torch.from_numpy(s).cuda(), torch.from_numpy(y).cuda())
    assert cal.index is not None and cal.index.dtype == torch.uint8
    q = torch.from_numpy(rng.uniform(-0.5, 1.5, 50_000)).cuda()
    assert torch.equal(cal.predict(q), _plain_interp(q, cal.xp, cal.fp))


def test_calibration_offsets_fit_segments_at_once() -> None:
    # the reference's per-segment calibration: one fit, segments kept apart by offsets
    rng = np.random.default_rng(6)
    keys = np.r_[rng.random(500), rng.random(500) + 3.0]
    y = np.r_[(rng.random(500) < 0.3), (rng.random(500) < 0.7)].astype(np.float64)
    off = np.r_[np.zeros(500), np.full(500, 1e3)]
    xp, fp = calibration_fit(torch.from_numpy(keys).cuda(), torch.from_numpy(y).cuda(), offset=torch.from_numpy(off).cuda())
    wxp, wfp = oracle.calibration_fit(keys, y, offset=off)
    np.testing.assert_array_equal(xp.cpu().numpy(), wxp)
    np.testing.assert_allclose(fp.cpu().numpy(), wfp, rtol=0, atol=1e-12)
