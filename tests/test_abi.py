"""CPU checks of the C-ABI library: it loads, exports every symbol that
include/dotcache_hip.h declares, and its host-only entry points (blob sizes,
read-byte accounting, decode planner) give the right answers.  No GPU call."""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

from dotcache_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def _declared():
    text = (ROOT / "include" / "dotcache_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dc_[a-z_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = _declared()
    assert "dc_decode_paged" in names and "dc_encode_rows" in names
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.SIGNATURES), "ctypes table out of sync with the header"


def test_abi_version():
    assert _lib.lib().dc_abi_version() == 1


def test_blob_bytes_match_layout():
    g = _lib.geometry(128, 32, 64)
    # M0 sym 4-bit: codes 4*64*4*4 = 4096, scales 64*4*2 = 512 -> 4608 (a multiple of 256)
    assert _lib.page_blob_bytes(_lib.FMT_M0_SYMMETRIC, 4, g) == 4608
    assert _lib.page_blob_bytes(_lib.FMT_M0_AFFINE, 4, g) == 4096 + 512 + 512 + 0  # 5120, already aligned
    assert _lib.page_blob_bytes(_lib.FMT_M3_F16, 0, g) == 16384
    with pytest.raises(ValueError):
        _lib.page_blob_bytes(_lib.FMT_M0_AFFINE, 5, g)


def test_read_bytes_are_algorithmic_bytes():
    g = _lib.geometry(128, 32, 64)
    assert _lib.page_read_bytes(_lib.FMT_M3_F16, 0, 64, g) == 16384
    assert _lib.page_read_bytes(_lib.FMT_M0_SYMMETRIC, 4, 64, g) == 4608
    assert _lib.page_read_bytes(_lib.FMT_M0_AFFINE, 4, 10, g) == 10 * (64 + 16)
    g64 = _lib.geometry(128, 64, 64)
    assert _lib.page_read_bytes(_lib.FMT_M0_SYMMETRIC, 8, 64, g64) == 64 * (128 + 4)  # C4 V: 132 B/token


def _plan(seq_pages, heads, per):
    sp = np.asarray(seq_pages, dtype=np.int32)
    L = _lib.lib()
    ni, nm, npart = C.c_int32(), C.c_int32(), C.c_int32()
    items = (_lib.WorkItem * 256)()
    merges = (_lib.MergeItem * 256)()
    st = L.dc_plan_decode(sp.ctypes.data, sp.size, heads, per, C.addressof(items), 256, C.byref(ni),
                          C.addressof(merges), 256, C.byref(nm), C.byref(npart))
    _lib.check(st, "plan")
    its = [(i.seq, i.kv_head, i.page_begin, i.page_end, i.partial) for i in items[: ni.value]]
    ms = [(m.seq, m.kv_head, m.partial_begin, m.count) for m in merges[: nm.value]]
    return its, ms, npart.value


def test_planner_covers_every_page_once():
    its, ms, npart = _plan([5, 1, 9], 2, 4)
    for b, n in enumerate([5, 1, 9]):
        for h in range(2):
            covered = sorted(p for (s, hh, pb, pe, _) in its if s == b and hh == h for p in range(pb, pe))
            assert covered == list(range(n))
    # sequence 1 (one page) is not split: it writes the output directly
    assert all(part == -1 for (s, _, _, _, part) in its if s == 1)
    assert npart == 2 * (2 + 3)
    assert sorted(ms) == [(0, 0, 0, 2), (0, 1, 2, 2), (2, 0, 4, 3), (2, 1, 7, 3)]


def _plan_fill(seq_pages, heads, target, min_pages=2):
    sp = np.asarray(seq_pages, dtype=np.int32)
    L = _lib.lib()
    ni, nm, npart, big = C.c_int32(), C.c_int32(), C.c_int32(), C.c_int32()
    st = L.dc_plan_decode_fill(sp.ctypes.data, sp.size, heads, target, min_pages, None, 0, C.byref(ni), None, 0,
                               C.byref(nm), C.byref(npart), C.byref(big))
    if st != _lib.DC_ESPACE:
        _lib.check(st, "plan fill")
    items = (_lib.WorkItem * max(ni.value, 1))()
    merges = (_lib.MergeItem * max(nm.value, 1))()
    st = L.dc_plan_decode_fill(sp.ctypes.data, sp.size, heads, target, min_pages, C.addressof(items), ni.value,
                               C.byref(ni), C.addressof(merges), nm.value, C.byref(nm), C.byref(npart), C.byref(big))
    _lib.check(st, "plan fill")
    its = [(i.seq, i.kv_head, i.page_begin, i.page_end, i.partial) for i in items[: ni.value]]
    ms = [(m.seq, m.kv_head, m.partial_begin, m.count) for m in merges[: nm.value]]
    return its, ms, npart.value, big.value


def _check_plan_shape(its, ms, npart, seq_pages, heads):
    """Every (sequence, head) covers its pages once, in order, by near-equal
    items; split streams own consecutive partial slots named by their merge."""
    for b, n in enumerate(seq_pages):
        for h in range(heads):
            mine = [(pb, pe, part) for (s, hh, pb, pe, part) in its if s == b and hh == h]
            assert [p for (pb, pe, _) in mine for p in range(pb, pe)] == list(range(n))
            sizes = [pe - pb for (pb, pe, _) in mine]
            assert max(sizes) - min(sizes) <= 1
            if len(mine) == 1:
                assert mine[0][2] == -1
            else:
                (m,) = [m for m in ms if m[0] == b and m[1] == h]
                assert m[3] == len(mine) and [part for (_, _, part) in mine] == list(range(m[2], m[2] + m[3]))
    assert npart == sum(m[3] for m in ms)


def test_fill_planner_uses_the_whole_budget():
    """C5's shape (4 x 4 streams of 1025 pages, one item per SIMD): the
    page-count split leaves 976 items (17 pages); the fill planner spends the
    other 48 on three more splits per stream, 64 items of 16 or 17 pages."""
    its, ms, npart, big = _plan_fill([1025] * 4, 4, 1024)
    assert len(its) == 1024 and big == 17 and len(ms) == 16 and all(m[3] == 64 for m in ms)
    _check_plan_shape(its, ms, npart, [1025] * 4, 4)
    # C3's shape already fills the budget: the plan of dc_plan_decode with 8 pages per split
    its, ms, npart, big = _plan_fill([256] * 8, 4, 1024)
    assert len(its) == 1024 and big == 8 and all(pe - pb == 8 for (_, _, pb, pe, _) in its)


def test_fill_planner_ragged_and_limits():
    rng = np.random.default_rng(11)
    pages = rng.integers(1, 300, size=20).tolist()
    its, ms, npart, big = _plan_fill(pages, 2, 100)
    assert len(its) <= 100
    _check_plan_shape(its, ms, npart, pages, 2)
    # no split item below the minimum page count
    assert all(pe - pb >= 2 for (s, _, pb, pe, part) in its if part >= 0)
    # never a larger item than the smallest page-count split that fits
    from dotcache_amd.decode import choose_pages_per_split

    assert big <= choose_pages_per_split(np.asarray(pages), 2, target_items=100)
    # more streams than the budget: one item per stream, over the target
    its, ms, npart, big = _plan_fill([3] * 10, 2, 8)
    assert len(its) == 20 and not ms and big == 3
    with pytest.raises(ValueError):
        _plan_fill([3, 0], 1, 8)
    with pytest.raises(ValueError):  # no item budget
        _plan_fill([3], 1, 0)


def test_planner_rejects_empty_sequence():
    with pytest.raises(ValueError):
        _plan([3, 0], 1, 2)


def test_workspace_holds_the_partials():
    assert _lib.lib().dc_decode_workspace_bytes(10, 7, 128) == 10 * 7 * 130 * 4


def test_planner_reports_short_tables():
    sp = np.asarray([100], dtype=np.int32)
    ni, nm, npart = C.c_int32(), C.c_int32(), C.c_int32()
    items = (_lib.WorkItem * 2)()
    st = _lib.lib().dc_plan_decode(sp.ctypes.data, 1, 1, 10, C.addressof(items), 2, C.byref(ni), None, 0,
                                   C.byref(nm), C.byref(npart))
    assert st == _lib.DC_ESPACE and ni.value == 10 and nm.value == 1


def test_decode_path_switch():
    """Paths 0 (auto), 1 (generic) and 2 (MFMA only) are accepted; anything
    else is DC_EINVAL, and the Python wrapper maps names onto them."""
    from dotcache_amd.decode import set_decode_path

    lib = _lib.lib()
    try:
        for path in (0, 1, 2):
            assert lib.dc_set_decode_path(path) == _lib.DC_OK
        assert lib.dc_set_decode_path(3) == _lib.DC_EINVAL
        assert lib.dc_set_decode_path(-1) == _lib.DC_EINVAL
        for name in ("auto", "generic", "mfma"):
            set_decode_path(name)
        with pytest.raises(ValueError):
            set_decode_path("fast")
    finally:
        lib.dc_set_decode_path(0)


def test_mfma_head_block_switch():
    """Head blocks 0 (automatic), 4, 8 and 16 are accepted; anything else is
    DC_EINVAL from the library and ValueError from the wrapper."""
    from dotcache_amd.decode import set_mfma_head_block

    lib = _lib.lib()
    try:
        for nqb in (0, 4, 8, 16):
            assert lib.dc_set_mfma_head_block(nqb) == _lib.DC_OK
            set_mfma_head_block(nqb)
        for bad in (-1, 1, 2, 12, 32):
            assert lib.dc_set_mfma_head_block(bad) == _lib.DC_EINVAL
        with pytest.raises(ValueError):
            set_mfma_head_block(2)
    finally:
        lib.dc_set_mfma_head_block(0)
