"""The C ABI without a GPU: the library loads, exports every function include/*.h declares,
reports its version, sizes its buffers, and turns bad arguments into status codes and
messages before touching the device (the reference's preconditions, tiles.cuh:1926-1934 and
grad.cuh:389-394, as TI_E* codes)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from torchisotonic_amd import _ext

HEADERS = sorted((Path(__file__).resolve().parents[1] / "include").glob("*.h"))


def declared_functions() -> list[str]:
    names = []
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(ti_\w+)\s*\(", text, flags=re.M)
    return names


def test_headers_declare_the_bound_symbols() -> None:
    names = declared_functions()
    assert len(names) >= 8
    assert set(names) == set(_ext.SYMBOLS)


def test_library_exports_every_declared_function() -> None:
    lib = _ext.load()
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_abi_version() -> None:
    assert _ext.load().ti_abi_version() == _ext.ABI_VERSION


def test_starts_words() -> None:
    lib = _ext.load()
    assert lib.ti_starts_words(1_000_000, 16) == 1_000_000
    assert lib.ti_starts_words(3, 33) == 6
    assert lib.ti_starts_words(1, 100_000_000) == 3_125_000
    assert lib.ti_starts_words(0, 5) == 0


def test_workspace_queries() -> None:
    lib = _ext.load()
    size = ctypes.c_size_t(123)
    assert lib.ti_fwd_workspace(1000, 16, _ext.F32, 0, ctypes.byref(size)) == 0
    assert size.value == 0
    assert lib.ti_fwd_workspace(1000, 32, _ext.F32, 0, ctypes.byref(size)) == 0
    assert size.value == 0  # short rows: no workspace
    assert lib.ti_fwd_workspace(1000, 33, _ext.F32, 0, ctypes.byref(size)) == 0
    assert size.value > 0  # longer rows: span hulls, merges and tile records
    # one vertex store shared by every merge level: span0 + 1 slots per span of span0 elements;
    # float32 data: 20 bytes a slot weighted (index, sums and weights rounded to float64), 12
    # unweighted; float64 data: 36 and 20 (double-double sums); per-level counts and totals and
    # the tile records are small beside it. Batches too small to spread their upper merge levels
    # over the GPU (fewer than 256 parents a level) hold a second store, into which those levels
    # write their hulls out of place.
    n = 100_000_000
    slots = -(-n // 256) * 257  # C4's spans of 256
    for dtype, weighted, per_slot in ((_ext.F32, 1, 20), (_ext.F32, 0, 12), (_ext.F64, 1, 36), (_ext.F64, 0, 20)):
        assert lib.ti_fwd_workspace(1, n, dtype, weighted, ctypes.byref(size)) == 0
        assert 2 * per_slot * slots < size.value < 2 * per_slot * slots * 1.03, (dtype, weighted, size.value)
    # C4 (one weighted float32 row of 1e8) within 4.2 GB
    assert lib.ti_fwd_workspace(1, n, _ext.F32, 1, ctypes.byref(size)) == 0
    assert size.value < 4.2e9
    # 256 rows of 1e6: one store (spans of 256: 3907 a row, 20 bytes a weighted float32 slot)
    assert lib.ti_fwd_workspace(256, 1_000_000, _ext.F32, 1, ctypes.byref(size)) == 0
    slots = 256 * 3907 * 257
    assert 20 * slots < size.value < 20 * slots * 1.03
    assert lib.ti_bwd_workspace(1000, 16, _ext.F64, 1, ctypes.byref(size)) == 0
    assert size.value == 0
    assert lib.ti_bwd_workspace(1000, 65536, _ext.F32, 1, ctypes.byref(size)) == 0
    assert size.value > 0
    assert lib.ti_fwd_workspace(10, 16, 7, 0, ctypes.byref(size)) == 2  # TI_EDTYPE
    assert lib.ti_fwd_workspace(10, 16, 0, 0, None) == 1  # TI_EINVAL


def test_kept_state_sizes() -> None:
    # what a backward keeps in place of the forward's workspace: each row's final hull in
    # max_vertices slots (float32: 20 bytes weighted, 12 unweighted; float64: 36, 20), its count,
    # NaN flag and totals (40 bytes) and 32 bytes a tile (2048 elements weighted, 4096
    # unweighted), against the workspace's slot for every element
    lib = _ext.load()
    size, ws = ctypes.c_size_t(0), ctypes.c_size_t(0)
    n = 100_000_000
    assert lib.ti_keep_bytes(1, n, _ext.F32, 1, 1083, ctypes.byref(size)) == 0
    tiles = -(-n // 2048)
    assert 20 * 1083 + 32 * tiles + 40 <= size.value < 20 * 1083 + 32 * tiles + 40 + 8 * 256
    assert size.value < 2e6
    assert lib.ti_fwd_workspace(1, n, _ext.F32, 1, ctypes.byref(ws)) == 0
    assert size.value * 1000 < ws.value
    assert lib.ti_keep_bytes(1000, 65536, _ext.F32, 0, 300, ctypes.byref(size)) == 0
    assert 1000 * (12 * 300 + 32 * 16 + 40) <= size.value < 1000 * (12 * 300 + 32 * 16 + 40) + 8 * 256
    assert lib.ti_keep_bytes(1000, 65536, _ext.F64, 1, 300, ctypes.byref(size)) == 0
    assert 1000 * (36 * 300 + 32 * 32 + 40) <= size.value < 1000 * (36 * 300 + 32 * 32 + 40) + 8 * 256
    # the backward's workspace from a kept state: per-tile scans and 16 bytes a kept slot,
    # against 16 bytes an element from the workspace
    kb, wb = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert lib.ti_bwd_kept_workspace(1, n, _ext.F32, 1, 1083, ctypes.byref(kb)) == 0
    assert lib.ti_bwd_workspace(1, n, _ext.F32, 1, ctypes.byref(wb)) == 0
    assert kb.value < 4e6 and wb.value > 16 * n
    # short rows keep nothing; max_vertices must be a hull's vertex count of such rows
    assert lib.ti_keep_bytes(1000, 32, _ext.F32, 1, 0, ctypes.byref(size)) == 0
    assert size.value == 0
    assert lib.ti_keep_bytes(10, 100, _ext.F32, 1, 0, ctypes.byref(size)) == 1
    assert lib.ti_keep_bytes(10, 100, _ext.F32, 1, 102, ctypes.byref(size)) == 1
    assert lib.ti_bwd_kept_workspace(10, 100, _ext.F32, 1, 0, ctypes.byref(size)) == 1
    assert b"max_vertices" in lib.ti_last_error()


def call_fwd(y: int | None, out: int | None, batch: int, n: int, dtype: int = 0) -> int:
    return _ext.load().ti_fwd(y, None, out, None, None, batch, n, dtype, 1, 0.0, 0.0, None, 0, None)


@pytest.mark.parametrize(
    ("args", "code", "words"),
    [
        ((1, 2, 4, 16, 5), 2, "dtype"),
        ((1, 2, -1, 16), 1, "batch >= 0"),
        ((1, 2, 4, 0), 1, "n >= 1"),
        ((1, 2, 1, 2**31), 3, "2^31"),
        ((None, 2, 4, 16), 1, "null"),
        ((1, None, 4, 16), 1, "null"),
        ((8, 8, 4, 16), 1, "alias"),
    ],
)
def test_fwd_argument_errors(args: tuple, code: int, words: str) -> None:
    assert call_fwd(*args) == code
    assert words in _ext.load().ti_last_error().decode()


def test_empty_batch_is_a_no_op() -> None:
    assert call_fwd(None, None, 0, 16) == 0
    assert _ext.load().ti_last_error() == b""


def test_noalloc_refuses_sets_beyond_its_scratch() -> None:
    # ti_fwd_noalloc refuses on the sizes alone, before any device call: here, with no GPU and
    # null buffers, a missing check would end in a device error instead of TI_EWORKSPACE.
    lib = _ext.load()
    size = ctypes.c_size_t(0)
    batch, n = 1000, 65536
    assert lib.ti_fwd_workspace(batch, n, _ext.F32, 1, ctypes.byref(size)) == 0
    assert size.value > 64 << 20
    rc = lib.ti_fwd_noalloc(None, None, None, None, None, batch, n, _ext.F32, 1, 0.0, 0.0, None)
    assert rc == 4  # TI_EWORKSPACE
    assert b"scratch holds" in lib.ti_last_error()


def test_bwd_argument_errors() -> None:
    lib = _ext.load()
    def bwd(starts, g, w, y, gy, gw, batch, n, flags, fws=None, fwsb=0, ws=None, wsb=0):
        return lib.ti_bwd(starts, fws, fwsb, g, w, y, gy, gw, batch, n, 0, flags, 0.0, 0.0, ws, wsb, None)

    # gw wanted without y
    assert bwd(1, 2, None, None, None, 3, 4, 16, 1) == 1
    assert b"y is needed" in lib.ti_last_error()
    # clamp mask without y
    assert bwd(1, 2, None, None, 3, None, 4, 16, 1 | 4) == 1
    # starts missing
    assert bwd(None, 2, None, None, 3, None, 4, 16, 1) == 1
    # nothing wanted: fine, no launch
    assert bwd(1, 2, None, None, None, None, 4, 16, 1) == 0
    # a row over 32 elements without the forward's workspace
    for n in (33, 100_000):
        assert bwd(1, 2, None, None, 3, None, 2, n, 1) == 4
        assert b"forward's workspace" in lib.ti_last_error()


def test_kept_state_argument_errors() -> None:
    # ti_keep and ti_bwd_kept refuse what they cannot use before any launch
    lib = _ext.load()
    n = 100_000
    ws = ctypes.c_size_t(0)
    assert lib.ti_fwd_workspace(2, n, _ext.F32, 1, ctypes.byref(ws)) == 0
    kb = ctypes.c_size_t(0)
    assert lib.ti_keep_bytes(2, n, _ext.F32, 1, 500, ctypes.byref(kb)) == 0

    def keep(fws, fwsb, kept, keptb, mv=500, batch=2, nn=n):
        return lib.ti_keep(fws, fwsb, kept, keptb, batch, nn, _ext.F32, 1, mv, None)

    # no forward workspace, or one too small
    assert keep(None, 0, 256, kb.value) == 4
    assert keep(256, ws.value - 1, 256, kb.value) == 4
    assert b"forward's workspace" in lib.ti_last_error()
    # a kept buffer too small
    assert keep(256, ws.value, 256, kb.value - 1) == 4
    # unaligned
    assert keep(256, ws.value, 264, kb.value) == 1
    # a bound no hull of these rows can have
    assert keep(256, ws.value, 256, kb.value, mv=0) == 1
    assert keep(256, ws.value, 256, kb.value, mv=n + 2) == 1
    assert b"max_vertices" in lib.ti_last_error()
    # rows of at most 32 elements keep nothing
    assert keep(None, 0, None, 0, mv=0, nn=32) == 0

    def bwd_kept(kept, keptb, mv, g=2, gy=3, batch=2, nn=n, ws_=None, wsb=0):
        # (weighted, as the kept state above: w given)
        return lib.ti_bwd_kept(1, kept, keptb, mv, g, 5, None, gy, None, batch, nn, _ext.F32,
                               _ext.INCREASING, 0.0, 0.0, ws_, wsb, None)

    bws = ctypes.c_size_t(0)
    assert lib.ti_bwd_kept_workspace(2, n, _ext.F32, 1, 500, ctypes.byref(bws)) == 0
    assert bws.value > 0
    assert bwd_kept(None, 0, 500, ws_=256, wsb=bws.value) == 4
    assert b"kept state" in lib.ti_last_error()
    assert bwd_kept(256, kb.value - 1, 500, ws_=256, wsb=bws.value) == 4
    assert b"kept state" in lib.ti_last_error()
    assert bwd_kept(256, kb.value, 0, ws_=256, wsb=bws.value) == 1
    assert b"max_vertices" in lib.ti_last_error()
    assert bwd_kept(256, kb.value, 500, ws_=None, wsb=0) == 4  # (no backward workspace)
    assert b"workspace of" in lib.ti_last_error()
    # rows of at most 32 elements: the short-row backward, no kept state needed
    assert bwd_kept(None, 0, 0, gy=None, nn=16) == 0


def test_grad_argument_errors() -> None:
    lib = _ext.load()

    def grad(out, starts, g, w, y, gy, gw, batch, n, ws=None, wsb=0):
        return lib.ti_grad(out, starts, g, w, y, gy, gw, batch, n, 0, ws, wsb, None)

    size = ctypes.c_size_t(7)
    assert lib.ti_grad_workspace(1000, 2, _ext.F32, ctypes.byref(size)) == 0 and size.value == 0
    assert lib.ti_grad_workspace(1, 2048, _ext.F32, ctypes.byref(size)) == 0 and size.value == 0
    assert lib.ti_grad_workspace(1, 2049, _ext.F64, ctypes.byref(size)) == 0 and size.value > 0
    assert lib.ti_grad_workspace(1, 100_000_000, _ext.F32, ctypes.byref(size)) == 0
    assert size.value < 100_000_000 // 8  # well under a byte an element
    # y without w (the reference's check, grad.cuh:393)
    assert grad(1, 2, 3, None, 5, 6, 7, 4, 16) == 1
    assert b"y is only needed" in lib.ti_last_error()
    # gw wanted without the fit
    assert grad(None, 2, 3, 4, 5, 6, 7, 4, 16) == 1
    # starts, g or gy missing
    assert grad(1, None, 3, None, None, 6, None, 4, 16) == 1
    assert grad(1, 2, None, None, None, 6, None, 4, 16) == 1
    assert grad(1, 2, 3, None, None, None, None, 4, 16) == 1
    # several tiles without a workspace
    assert grad(1, 2, 3, None, None, 6, None, 2, 100_000) == 4
    # empty batch: nothing to do
    assert grad(None, None, None, None, None, None, None, 0, 16) == 0


def test_ragged_backward_argument_errors() -> None:
    lib = _ext.load()

    def bwd(starts, g, w, y, gy, gw, nrows=10, max_len=16, dtype=_ext.F32, flags=0):
        return lib.ti_bwd_ragged(starts, g, w, y, gy, gw, 64, nrows, 100, max_len, dtype, flags, 0.0, 0.0, None)

    assert bwd(8, 16, None, None, 24, None, dtype=5) == 2
    assert bwd(8, 16, None, None, 24, None, nrows=-1) == 1
    assert bwd(8, 16, None, None, 24, None, max_len=0) == 3
    assert bwd(8, 16, None, None, 24, None, max_len=33) == 3
    # gw needs w and y; the clamp needs y
    assert bwd(8, 16, None, 40, 24, 32) == 1 and b"gw needs" in lib.ti_last_error()
    assert bwd(8, 16, 48, None, 24, 32) == 1
    assert bwd(8, 16, None, None, 24, None, flags=_ext.CLIP_MIN) == 1
    # missing inputs, no output, aliased outputs
    assert bwd(None, 16, None, None, 24, None) == 1
    assert bwd(8, None, None, None, 24, None) == 1
    assert bwd(8, 16, None, None, None, None) == 1
    assert bwd(8, 16, None, None, 16, None) == 1 and b"alias" in lib.ti_last_error()
    assert bwd(8, 16, 48, 40, 24, 24) == 1
    # no rows: nothing to do
    assert bwd(None, None, None, None, None, None, nrows=0) == 0


def test_interp_index_sizes_and_argument_errors() -> None:
    lib = _ext.load()
    size = ctypes.c_size_t(0)
    # a 256-byte header, then one 4-byte entry a bucket of four knots (and one more), rounded up
    assert lib.ti_interp_index_bytes(1, _ext.F64, ctypes.byref(size)) == 0 and size.value == 512
    assert lib.ti_interp_index_bytes(6_000_000, _ext.F64, ctypes.byref(size)) == 0
    assert 256 + 4 * 1_500_001 <= size.value < 256 + 4 * 1_500_001 + 256 and size.value % 256 == 0
    assert lib.ti_interp_index_bytes(6_000_000, _ext.F32, ctypes.byref(size)) == 0  # the same for float32
    assert lib.ti_interp_index_bytes(0, _ext.F64, ctypes.byref(size)) == 1
    assert lib.ti_interp_index_bytes(1 << 32, _ext.F64, ctypes.byref(size)) == 3
    assert lib.ti_interp_index_bytes(10, 7, ctypes.byref(size)) == 2
    assert lib.ti_interp_index_bytes(10, _ext.F64, None) == 1
    assert lib.ti_interp_index_bytes(1000, _ext.F64, ctypes.byref(size)) == 0
    need = size.value
    # build: missing xp or index, an index too small, a misaligned index
    assert lib.ti_interp_index(None, 1000, _ext.F64, 256, need, None) == 1
    assert lib.ti_interp_index(8, 1000, _ext.F64, None, need, None) == 1
    assert lib.ti_interp_index(8, 1000, _ext.F64, 256, need - 1, None) == 4
    assert b"need" in lib.ti_last_error()
    assert lib.ti_interp_index(8, 1000, _ext.F64, 264, need, None) == 1
    # interpolate: the same index checks, then the buffers; no queries is no work
    assert lib.ti_interp_indexed(8, 16, 24, 256, need - 1, 32, 10, 1000, _ext.F64, None) == 4
    assert lib.ti_interp_indexed(8, 16, 24, None, need, 32, 10, 1000, _ext.F64, None) == 1
    assert lib.ti_interp_indexed(8, 16, 24, 264, need, 32, 10, 1000, _ext.F64, None) == 1
    assert lib.ti_interp_indexed(None, 16, 24, 256, need, 32, 10, 1000, _ext.F64, None) == 1
    assert lib.ti_interp_indexed(8, 16, 24, 256, need, 32, -1, 1000, _ext.F64, None) == 1
    assert lib.ti_interp_indexed(None, None, None, 256, need, None, 0, 1000, _ext.F64, None) == 0


def test_errors_are_per_thread() -> None:
    import threading

    lib = _ext.load()
    assert call_fwd(1, 2, 4, 16, 9) == 2
    seen = []
    t = threading.Thread(target=lambda: seen.append(lib.ti_last_error()))
    t.start()
    t.join()
    assert seen == [b""]
    assert b"dtype" in lib.ti_last_error()


def test_operator_library_registers_the_fit() -> None:
    # the torch operator over the C ABI loads without a GPU and has the documented schema
    ops = _ext.ops()
    schema = str(ops.isotonic_fit.default._schema)
    assert schema.startswith("torchisotonic_amd::isotonic_fit(Tensor y, Tensor? w, bool increasing")
    assert "float? y_min" in schema and "float? y_max" in schema and schema.endswith("-> Tensor")


def test_rows_entry_points_refuse_before_any_launch() -> None:
    # ti_fwd_rows / ti_bwd_rows check dtype, block length and the packed arrays' size before any
    # device call (null buffers here: a missing check would end in a device error)
    lib = _ext.load()

    def fwd(k, L, total, dtype):
        return lib.ti_fwd_rows(None, None, None, None, None, None, k, L, total, 0.0, dtype, 1, 0.0, 0.0, None, 0, None)

    def bwd(k, L, total, dtype):
        return lib.ti_bwd_rows(None, None, 0, None, None, None, None, None, None, k, L, total, dtype, 1, 0.0, 0.0,
                               None, 0, None)

    for call in (fwd, bwd):
        assert call(4, 64, 1000, _ext.F64) == 2  # TI_EDTYPE: float32 only
        assert b"float32 only" in lib.ti_last_error()
        assert call(4, 32, 1000, _ext.F32) == 1  # TI_EINVAL: the short-row regime has no row map
        assert b"longer than 32" in lib.ti_last_error()
        assert call(4, 64, 1000, _ext.F32) == 1  # rows missing
        assert b"rows must not be null" in lib.ti_last_error()
        assert call(4, 64, 0x7FFF0000 // 4 + 1, _ext.F32) == 3  # TI_ESIZE: one buffer resource's reach
        assert b"2147418112 bytes" in lib.ti_last_error()
