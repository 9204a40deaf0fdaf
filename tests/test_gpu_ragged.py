"""Ragged rows (packed end to end with offsets) on the GPU against the oracle's per-row fits:
short rows in one launch and longer rows a length bucket at a time through the regular kernels
(each row padded beyond its extreme in the bucket's block), with block starts, the backward (one
launch for the short rows, from the forward's flat start bits; each bucket from its own
forward), rows whose pad joins their last block (NaN rows, the largest finite value), the
clamp, and C2's padded variant (lengths U{4..16}: a padded row's first len_b fitted values equal
the ragged row's fit; reference README.md:100-103)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from gpu_util import tolerance
from torchisotonic_amd import _ext, isotonic, isotonic_ragged
from torchisotonic_amd import ragged as rg

pytestmark = pytest.mark.gpu


def say(*a: object) -> None:
    print(*a, flush=True)


def ragged_set(lengths: np.ndarray, dtype: type, seed: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    rng = np.random.default_rng(seed)
    off = np.zeros(len(lengths) + 1, dtype=np.int64)
    np.cumsum(lengths, out=off[1:])
    pos = np.arange(off[-1]) - np.repeat(off[:-1], lengths)  # index within the row
    y = (0.1 * pos + rng.standard_normal(off[-1])).astype(dtype)
    w = (rng.random(off[-1]) + 0.1).astype(dtype)
    return y, w, off


def run(y: np.ndarray, w: np.ndarray | None, off: np.ndarray, increasing: bool):
    yt = torch.from_numpy(y).cuda()
    wt = None if w is None else torch.from_numpy(w).cuda()
    off_t, short_max, spans, bits, bad = rg._offsets(torch.from_numpy(off).cuda(), None, yt, wt is not None)
    out, long_rows = rg._fit(yt, wt, off_t, short_max, spans, bits, bad, increasing)
    starts = _ext.starts_to_bool(bits, 1, len(y))[0].cpu().numpy().astype(np.uint8)
    for rows, L, s, *_ in long_rows:  # each longer row's partition: its row of the bucket's block
        sb = _ext.starts_to_bool(s, len(rows), L).cpu().numpy()
        first, ln = np.array(rows, dtype=np.int64).T
        keep = np.arange(L)[None, :] < ln[:, None]
        starts[(first[:, None] + np.arange(L)[None, :])[keep]] = sb[keep]
    return out.cpu().numpy(), starts


def check(y, w, off, increasing):
    got, starts = run(y, w, off, increasing)
    want, want_starts = oracle.pava_ragged(y, off, w, increasing=increasing, acc="f64")
    assert got.dtype == y.dtype
    diff = np.abs(got.astype(np.float64) - want)
    assert diff.size == 0 or float(diff.max()) <= tolerance(y), (float(diff.max()), tolerance(y))
    np.testing.assert_array_equal(starts, want_starts)


LENGTH_SETS = {
    "1..32": lambda rng: rng.integers(1, 33, 20_000),
    "0..40": lambda rng: rng.integers(0, 41, 5_000),     # empty rows, and rows past 32
    "ones": lambda rng: np.ones(3_000, dtype=np.int64),
    "mixed": lambda rng: np.r_[rng.integers(1, 9, 3000), [33, 1000, 70_000], rng.integers(1, 33, 3000), [0, 0]],
    "long": lambda rng: np.array([40, 5000, 33]),        # no short row
}


@pytest.mark.parametrize("lengths", list(LENGTH_SETS))
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("increasing", [True, False])
def test_matches_oracle(lengths: str, dtype: type, weighted: bool, increasing: bool) -> None:
    say(f"ragged {lengths} {np.dtype(dtype).name} weighted={weighted} increasing={increasing}")
    rng = np.random.default_rng(len(lengths) * 7 + weighted)
    ln = LENGTH_SETS[lengths](rng).astype(np.int64)
    y, w, off = ragged_set(ln, dtype, int(ln.sum()))
    check(y, w if weighted else None, off, increasing)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_unaligned_base(dtype: type) -> None:
    # values starting one element past a 16-byte boundary: the kernel stages element by element
    rng = np.random.default_rng(9)
    ln = rng.integers(0, 20, 4000)
    y, w, off = ragged_set(ln, dtype, 9)
    big = torch.from_numpy(np.r_[np.zeros(1, dtype=dtype), y]).cuda()
    wb = torch.from_numpy(np.r_[np.ones(1, dtype=dtype), w]).cuda()
    assert big[1:].data_ptr() % 16 != 0
    for ww, wt in ((None, None), (w, wb[1:])):
        got = isotonic_ragged(big[1:], torch.from_numpy(off).cuda(), weight=wt).cpu().numpy()
        want, _ = oracle.pava_ragged(y, off, ww, acc="f64")
        assert float(np.abs(got.astype(np.float64) - want).max()) <= tolerance(y)


def test_nan_rows_and_ties() -> None:
    # a NaN row is all NaN with its first start only; its neighbours are untouched; ties pool
    y, _, off = ragged_set(np.array([5, 7, 3, 40, 6]), np.float64, 3)
    y[off[1] + 2] = np.nan
    y[off[3] + 10] = np.nan
    y[off[4]:off[5]] = 1.0
    got, starts = run(y, None, off, True)
    for r in (1, 3):
        assert np.isnan(got[off[r]:off[r + 1]]).all()
        assert starts[off[r]] == 1 and not starts[off[r] + 1:off[r + 1]].any()
    for r in (0, 2):
        want, ws = oracle.pava(y[off[r]:off[r + 1]][None], acc="f64")
        np.testing.assert_allclose(got[off[r]:off[r + 1]], want[0], rtol=0, atol=1e-12)
        np.testing.assert_array_equal(starts[off[r]:off[r + 1]], ws[0])
    assert (got[off[4]:] == 1.0).all() and starts[off[4]:].tolist() == [1, 0, 0, 0, 0, 0]


def test_c2_padded_variant() -> None:
    # C2 [1e6, 16] f32 decreasing, rows of len_b ~ U{4..16} (seed 2) padded with min - 1: the
    # padded fit's first len_b values equal the ragged fit of the unpadded rows
    say("C2 padded variant")
    batch, n = 1_000_000, 16
    rng = np.random.default_rng(0)
    y = (-0.1 * np.arange(n, dtype=np.float32)[None, :] + rng.standard_normal((batch, n), dtype=np.float32)).astype(np.float32)
    lens = np.random.default_rng(2).integers(4, 17, batch)
    keep = np.arange(n)[None, :] < lens[:, None]
    pad = np.where(keep, y, np.inf).min(axis=1) - 1
    yp = np.where(keep, y, pad[:, None]).astype(np.float32)
    padded = isotonic(torch.from_numpy(yp).cuda(), increasing=False).cpu().numpy()
    packed = y[keep]
    off = np.zeros(batch + 1, dtype=np.int64)
    np.cumsum(lens, out=off[1:])
    got = isotonic_ragged(torch.from_numpy(packed).cuda(), torch.from_numpy(off), increasing=False).cpu().numpy()
    np.testing.assert_array_equal(got, padded[keep])
    want, _ = oracle.pava_ragged(packed, off, increasing=False, acc="f64")
    assert float(np.abs(got - want).max()) <= tolerance(packed)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("weighted", [False, True])
def test_backward_matches_block_gradient(dtype: type, weighted: bool) -> None:
    say(f"ragged backward {np.dtype(dtype).name} weighted={weighted}")
    rng = np.random.default_rng(11)
    ln = np.r_[rng.integers(0, 33, 20_000), [100, 5000], rng.integers(1, 33, 100)].astype(np.int64)
    y, w, off = ragged_set(ln, dtype, 12)
    g = rng.standard_normal(len(y)).astype(dtype)
    yt = torch.from_numpy(y).cuda().requires_grad_()
    wt = torch.from_numpy(w).cuda().requires_grad_() if weighted else None
    out = isotonic_ragged(yt, torch.from_numpy(off).cuda(), weight=wt)
    grads = torch.autograd.grad(out, [yt] + ([wt] if weighted else []), torch.from_numpy(g).cuda())
    fit, starts = oracle.pava_ragged(y, off, w if weighted else None, acc="f64")
    ey, ew = oracle.block_grad(starts, g.astype(np.float64), w.astype(np.float64) if weighted else None,
                               y.astype(np.float64) if weighted else None, fit, want_w=weighted)
    tol = 1e-11 if dtype == np.float64 else 1e-5
    for got, exp in zip(grads, (ey, ew)):
        scale = max(float(np.abs(exp).max()), 1e-300)
        np.testing.assert_allclose(got.double().cpu().numpy(), exp, rtol=tol, atol=tol * scale)


def _grads(y: np.ndarray, w: np.ndarray | None, off: np.ndarray, g: np.ndarray, increasing: bool = True):
    yt = torch.from_numpy(y).cuda().requires_grad_()
    wt = None if w is None else torch.from_numpy(w).cuda().requires_grad_()
    out = isotonic_ragged(yt, torch.from_numpy(off).cuda(), weight=wt, increasing=increasing)
    grads = torch.autograd.grad(out, [yt] + ([] if wt is None else [wt]), torch.from_numpy(g).cuda())
    return out.detach().cpu().numpy(), [t.cpu().numpy() for t in grads]


def _block_grads(fit, starts, y, w, g):
    ey, ew = oracle.block_grad(starts, g.astype(np.float64), None if w is None else w.astype(np.float64),
                               None if w is None else y.astype(np.float64), fit, want_w=w is not None)
    return [e for e in (ey, ew) if e is not None]


def test_long_rows_of_uniform_lengths() -> None:
    # 1e5 rows of lengths U{1..2000} (about 1e8 elements; eleven length buckets and the short
    # rows), weighted float32: fit, partition and both gradients against the oracle's rows
    say("ragged 1e5 rows, lengths U{1..2000}, float32 weighted")
    rng = np.random.default_rng(31)
    ln = rng.integers(1, 2001, 100_000).astype(np.int64)
    y, w, off = ragged_set(ln, np.float32, 32)
    got, starts = run(y, w, off, True)
    fit, want_starts = oracle.pava_ragged(y, off, w, acc="f64")
    assert float(np.abs(got.astype(np.float64) - fit).max()) <= tolerance(y)
    np.testing.assert_array_equal(starts, want_starts)
    del got, starts
    g = rng.standard_normal(len(y)).astype(np.float32)
    out, grads = _grads(y, w, off, g)
    assert float(np.abs(out.astype(np.float64) - fit).max()) <= tolerance(y)
    for gt, e in zip(grads, _block_grads(fit, want_starts, y, w, g)):
        np.testing.assert_allclose(gt.astype(np.float64), e, rtol=1e-5, atol=1e-5 * float(np.abs(e).max()))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("increasing", [True, False])
@pytest.mark.parametrize("weighted", [False, True])
def test_rows_whose_pad_joins_their_last_block(dtype: type, increasing: bool, weighted: bool) -> None:
    # rows past 32 elements whose pad cannot lie beyond their extreme: NaN rows (one block over
    # the row and its pad) and, in float32, rows ending in the largest finite value (a last block
    # that pools with the pad); their fits and gradients are the row's own, the pad's weight taken
    # out (float32 buckets in place, float64 ones through a block and ti_ragged_unpack)
    say(f"ragged pad joins the last block: {np.dtype(dtype).name} increasing={increasing} weighted={weighted}")
    rng = np.random.default_rng(41)
    # buckets: (32, 64] rows 0, 2, 3, 7 (L = 64); (64, 128] rows 5, 10; (256, 512] rows 1, 8;
    # (512, 1024] rows 4, 9; row 6 short
    ln = np.array([40, 300, 33, 40, 1000, 70, 5, 64, 500, 1020, 128], dtype=np.int64)
    y, w, off = ragged_set(ln, dtype, 42)
    y[off[1] + 7] = np.nan       # a NaN row, 300 elements padded to 500
    y[off[3] + 1] = np.nan       # a NaN row, 40 elements padded to 64
    if dtype == np.float32:      # (float64 sums of the largest float64 overflow in any fit)
        top = np.float32((1 if increasing else -1) * np.finfo(np.float32).max)
        y[off[3] - 1] = top          # ends at the extreme: a last block of its own, padded to 64
        y[off[5] - 3:off[5]] = top   # three of them, padded to 1020
        y[off[6] - 10] = top         # the extreme before smaller values: no pooling with the pad
        y[off[8] - 1] = top          # a row as long as its block: no pad
    g = rng.standard_normal(len(y)).astype(dtype)
    ww = w if weighted else None
    out, grads = _grads(y, ww, off, g, increasing)
    fit, starts = oracle.pava_ragged(y, off, ww, increasing=increasing, acc="f64")
    np.testing.assert_array_equal(np.isnan(out), np.isnan(fit))
    for r in range(len(ln)):  # each row within the tolerance of its own magnitude
        a, b = off[r], off[r + 1]
        if not np.isnan(fit[a:b]).any():
            assert float(np.abs(out[a:b].astype(np.float64) - fit[a:b]).max()) <= tolerance(y[a:b]), r
    gtol = 1e-5 if dtype == np.float32 else 1e-11
    for gt, e in zip(grads, _block_grads(fit, starts, y, ww, g)):
        scale = float(np.abs(e[np.isfinite(e)]).max())
        np.testing.assert_allclose(gt.astype(np.float64), e, rtol=gtol, atol=gtol * scale)


def _ragged_abi(y: np.ndarray, w: np.ndarray | None, off: np.ndarray, g: np.ndarray, flags: int, lo: float,
                hi: float, want_w: bool, shift: int = 0):
    # ti_fwd_ragged then ti_bwd_ragged through the C ABI; `shift` puts every array one element
    # past a 16-byte boundary (the element-by-element staging)
    lib = _ext.load()
    n, nrows = len(y), len(off) - 1
    dt = torch.float32 if y.dtype == np.float32 else torch.float64
    code = _ext.F32 if y.dtype == np.float32 else _ext.F64

    def dev(a: np.ndarray) -> torch.Tensor:
        t = torch.zeros(n + shift, dtype=dt, device="cuda")
        t[shift:] = torch.from_numpy(a).cuda()
        return t[shift:]

    yt, gt = dev(y), dev(g)
    wt = None if w is None else dev(w)
    out, gy = dev(np.zeros_like(y)), dev(np.zeros_like(y))
    gw = dev(np.zeros_like(y)) if want_w else None
    offt = torch.from_numpy(off).cuda()
    bits = torch.zeros((n + 31) // 32 + 1, dtype=torch.int32, device="cuda")
    max_len = int(max(1, min(32, (off[1:] - off[:-1]).max())))
    s = torch.cuda.current_stream().cuda_stream
    assert lib.ti_fwd_ragged(yt.data_ptr(), _ext._ptr(wt), out.data_ptr(), bits.data_ptr(), None, offt.data_ptr(),
                             nrows, n, max_len, code, flags, lo, hi, s) == 0
    assert lib.ti_bwd_ragged(bits.data_ptr(), gt.data_ptr(), _ext._ptr(wt), yt.data_ptr(), gy.data_ptr(),
                             _ext._ptr(gw), offt.data_ptr(), nrows, n, max_len, code, flags, lo, hi, s) == 0
    torch.cuda.synchronize()
    return out.cpu().numpy(), gy.cpu().numpy(), None if gw is None else gw.cpu().numpy()


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("shift", [0, 1])
def test_backward_abi_with_the_forward_clamp(dtype: type, weighted: bool, shift: int) -> None:
    # ti_bwd_ragged after a clamped ti_fwd_ragged: the block gradient, zero in blocks whose fit
    # the clamp moved (torch.clamp's mask on the block mean), rows of 0 to 32 elements
    say(f"ragged backward, C ABI, clamp: {np.dtype(dtype).name} weighted={weighted} shift={shift}")
    rng = np.random.default_rng(21 + shift)
    ln = rng.integers(0, 33, 30_000).astype(np.int64)
    y, w, off = ragged_set(ln, dtype, 22)
    g = rng.standard_normal(len(y)).astype(dtype)
    lo, hi = -0.3, 1.2
    flags = _ext.INCREASING | _ext.EXACT | _ext.CLIP_MIN | _ext.CLIP_MAX
    out, gy, gw = _ragged_abi(y, w if weighted else None, off, g, flags, lo, hi, weighted, shift)
    fit, starts = oracle.pava_ragged(y, off, w if weighted else None, acc="f64")
    np.testing.assert_allclose(out.astype(np.float64), np.clip(fit, lo, hi), rtol=0, atol=tolerance(y))
    ey, ew = oracle.block_grad(starts, g.astype(np.float64), w.astype(np.float64) if weighted else None,
                               y.astype(np.float64) if weighted else None, fit, want_w=weighted)
    mask = (fit >= lo) & (fit <= hi)
    # (a block mean within rounding of a bound may fall either side of it in the kernel's dtype:
    # those elements are left out, the rest compared)
    clear = (np.abs(fit - lo) > 1e-5) & (np.abs(fit - hi) > 1e-5)
    assert clear.mean() > 0.99 and (~mask & clear).any() and (mask & clear).any()
    tol = 1e-11 if dtype == np.float64 else 1e-5
    for got, exp in ((gy, ey), (gw, ew)):
        if exp is None:
            continue
        exp = exp * mask
        scale = max(float(np.abs(exp).max()), 1e-300)
        np.testing.assert_allclose(got.astype(np.float64)[clear], exp[clear], rtol=tol, atol=tol * scale)


def test_backward_c2_rows_at_full_size() -> None:
    # C2's rows at their own lengths (1e6 rows, len ~ U{4..16}, seed 2), decreasing, float32:
    # the one-launch backward against the oracle's block gradient
    say("ragged backward, C2 rows at full size")
    b, n = 1_000_000, 16
    rng = np.random.default_rng(0)
    y2 = (-0.1 * np.arange(n) + rng.standard_normal((b, n))).astype(np.float32)
    lens = np.random.default_rng(2).integers(4, n + 1, b)
    packed = y2[np.arange(n)[None, :] < lens[:, None]]
    off = np.r_[0, np.cumsum(lens)].astype(np.int64)
    g = np.random.default_rng(3).standard_normal(len(packed)).astype(np.float32)
    yt = torch.from_numpy(packed).cuda().requires_grad_()
    out = isotonic_ragged(yt, torch.from_numpy(off).cuda(), increasing=False)
    (gy,) = torch.autograd.grad(out, [yt], torch.from_numpy(g).cuda())
    fit, starts = oracle.pava_ragged(packed, off, increasing=False, acc="f64")
    ey, _ = oracle.block_grad(starts, g.astype(np.float64))
    np.testing.assert_allclose(gy.double().cpu().numpy(), ey, rtol=1e-5, atol=1e-5 * float(np.abs(ey).max()))


def test_lengths_clamp_and_gradcheck() -> None:
    gen = torch.Generator().manual_seed(4)
    ln = torch.tensor([3, 0, 7, 1, 40, 12])
    y = torch.randn(int(ln.sum()), generator=gen, dtype=torch.float64).cuda()
    a = isotonic_ragged(y, lengths=ln, y_min=-0.2, y_max=0.5)
    off = np.r_[0, np.cumsum(ln.numpy())]
    want, _ = oracle.pava_ragged(y.cpu().numpy(), off, acc="f64")
    np.testing.assert_allclose(a.cpu().numpy(), np.clip(want, -0.2, 0.5), rtol=0, atol=1e-12)
    yy = y.clone().requires_grad_()
    ww = (torch.rand(len(y), generator=gen, dtype=torch.float64) + 0.5).cuda().requires_grad_()
    assert torch.autograd.gradcheck(lambda t, u: isotonic_ragged(t, lengths=ln, weight=u, increasing=False), (yy, ww))


@pytest.mark.parametrize("max_len", [0, 4, 16, 32, 1000])
def test_max_len_bound(max_len: int) -> None:
    # a bound on the row lengths lets the short rows' launch start before the plan is read: the
    # same fits, starts and gradients whether the bound is right (16), too small (4: a second
    # launch), loose (32, 1000) or absent (0), with rows past 32 and empty rows present
    say(f"ragged max_len={max_len}")
    rng = np.random.default_rng(31)
    ln = np.r_[rng.integers(0, 17, 20_000), [40, 0, 300], rng.integers(1, 17, 500)].astype(np.int64)
    y, w, off = ragged_set(ln, np.float32, 32)
    g = rng.standard_normal(len(y)).astype(np.float32)
    yt = torch.from_numpy(y).cuda().requires_grad_()
    wt = torch.from_numpy(w).cuda().requires_grad_()
    out = isotonic_ragged(yt, torch.from_numpy(off).cuda(), weight=wt, increasing=False, max_len=max_len)
    gy, gw = torch.autograd.grad(out, [yt, wt], torch.from_numpy(g).cuda())
    fit, starts = oracle.pava_ragged(y, off, w, increasing=False, acc="f64")
    assert float(np.abs(out.detach().double().cpu().numpy() - fit).max()) <= tolerance(y)
    ey, ew = oracle.block_grad(starts, g.astype(np.float64), w.astype(np.float64), y.astype(np.float64), fit,
                               want_w=True)
    for got, exp in ((gy, ey), (gw, ew)):
        np.testing.assert_allclose(got.double().cpu().numpy(), exp, rtol=1e-5, atol=1e-5 * float(np.abs(exp).max()))


def test_max_len_with_bad_offsets_raises() -> None:
    # with a bound, the short rows' kernel runs on offsets not yet checked (it clamps every one
    # into the packed array and each row into its workgroup's range); the plan then raises
    y = torch.randn(100, device="cuda")
    for off, msg in (([0, 40, 20, 100], "decrease"), ([0, 50, 150], "offsets must run"), ([5, 50, 100], "offsets must run")):
        with pytest.raises(ValueError, match=msg):
            isotonic_ragged(y, torch.tensor(off), max_len=16)
    good = isotonic_ragged(y, torch.tensor([0, 40, 60, 100]), max_len=16)
    want, _ = oracle.pava_ragged(y.cpu().numpy(), np.array([0, 40, 60, 100]), acc="f64")
    assert float(np.abs(good.cpu().numpy() - want).max()) <= tolerance(y.cpu().numpy())
    with pytest.raises(ValueError, match="max_len"):
        isotonic_ragged(y, torch.tensor([0, 100]), max_len=-1)


def test_argument_errors() -> None:
    y = torch.randn(10, device="cuda")
    with pytest.raises(ValueError, match="offsets"):
        isotonic_ragged(y, torch.tensor([0, 4, 9]))
    with pytest.raises(ValueError, match="decrease"):
        isotonic_ragged(y, torch.tensor([0, 6, 4, 10]))
    with pytest.raises(ValueError, match="non-negative"):
        isotonic_ragged(y, lengths=[6, -1, 5])
    with pytest.raises(ValueError, match="integer"):
        isotonic_ragged(y, torch.tensor([0.0, 10.0]))
    with pytest.raises(ValueError, match="exactly one"):
        isotonic_ragged(y)
    with pytest.raises(ValueError, match="positive"):
        isotonic_ragged(y, lengths=torch.tensor([4, 6]), weight=torch.zeros(10, device="cuda"))
    with pytest.raises(ValueError, match="positive"):
        isotonic_ragged(torch.randn(50, device="cuda"), lengths=torch.tensor([10, 40]),
                        weight=torch.cat([torch.ones(10), -torch.ones(40)]).cuda())
    with pytest.raises(RuntimeError, match="GPU"):
        isotonic_ragged(torch.randn(10), lengths=torch.tensor([10]))
    assert isotonic_ragged(torch.empty(0, device="cuda"), lengths=torch.tensor([0, 0])).numel() == 0
