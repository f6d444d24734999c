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
    assert _lib.lib().dc_abi_version() == 2


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


def _plan_fill(seq_pages, heads, target, cpp=1, cost=None, min_chunks=None, last_tokens=None):
    """dc_plan_decode_fill; items as (seq, head, first chunk, end chunk,
    partial) with chunk positions counted along the stream."""
    sp = np.asarray(seq_pages, dtype=np.int32)
    L = _lib.lib()
    min_chunks = 2 * cpp if min_chunks is None else min_chunks
    cp, stride = None, 0
    if cost is not None:
        cost = np.ascontiguousarray(cost, dtype=np.float32)
        cp, stride = cost.ctypes.data, cost.shape[2]
    ni, nm, npart, big = C.c_int32(), C.c_int32(), C.c_int32(), C.c_int32()
    lt = None if last_tokens is None else np.ascontiguousarray(last_tokens, dtype=np.int32)
    args = (sp.ctypes.data, None if lt is None else lt.ctypes.data, sp.size, heads, cpp, cp, stride, target, min_chunks)
    st = L.dc_plan_decode_fill(*args, None, 0, C.byref(ni), None, 0, C.byref(nm), C.byref(npart), C.byref(big))
    if st != _lib.DC_ESPACE:
        _lib.check(st, "plan fill")
    items = (_lib.WorkItem * max(ni.value, 1))()
    merges = (_lib.MergeItem * max(nm.value, 1))()
    st = L.dc_plan_decode_fill(*args, C.addressof(items), ni.value, C.byref(ni), C.addressof(merges), nm.value,
                               C.byref(nm), C.byref(npart), C.byref(big))
    _lib.check(st, "plan fill")
    its = []
    for i in items[: ni.value]:
        assert 0 <= i.chunk_begin < cpp and 0 <= i.chunk_end < cpp and i.reserved == 0
        u0 = i.page_begin * cpp + i.chunk_begin
        u1 = i.page_end * cpp if i.chunk_end == 0 else (i.page_end - 1) * cpp + i.chunk_end
        its.append((i.seq, i.kv_head, u0, u1, i.partial))
    ms = [(m.seq, m.kv_head, m.partial_begin, m.count) for m in merges[: nm.value]]
    return its, ms, npart.value, big.value


def _check_plan_shape(its, ms, npart, seq_pages, heads, cpp=1, equal=True, last_chunks=None):
    """Every (sequence, head) covers its chunks once, in order, by non-empty
    (without costs: near-equal) items; split streams own consecutive partial
    slots named by their merge.  ``last_chunks[b]``: the chunks of sequence
    b's last page that hold tokens (default: all)."""
    for b, n in enumerate(seq_pages):
        live = n * cpp if last_chunks is None else (n - 1) * cpp + last_chunks[b]
        for h in range(heads):
            mine = [(u0, u1, part) for (s, hh, u0, u1, part) in its if s == b and hh == h]
            assert [u for (u0, u1, _) in mine for u in range(u0, u1)] == list(range(live))
            sizes = [u1 - u0 for (u0, u1, _) in mine]
            assert min(sizes) >= 1
            if equal:
                assert max(sizes) - min(sizes) <= 1
            if len(mine) == 1:
                assert mine[0][2] == -1
            else:
                (m,) = [m for m in ms if m[0] == b and m[1] == h]
                assert m[3] == len(mine) and [part for (_, _, part) in mine] == list(range(m[2], m[2] + m[3]))
    assert npart == sum(m[3] for m in ms)


def test_fill_planner_uses_the_whole_budget():
    """C5's shape (4 x 4 streams of 1025 pages, one item per SIMD): whole
    pages give 64 items of 16 or 17 pages per stream; cut at 32-token chunks
    (4 per 128-token page) the largest item is 65 chunks (16.25 pages)."""
    its, ms, npart, big = _plan_fill([1025] * 4, 4, 1024)
    assert len(its) == 1024 and big == 17 and len(ms) == 16 and all(m[3] == 64 for m in ms)
    _check_plan_shape(its, ms, npart, [1025] * 4, 4)
    its, ms, npart, big = _plan_fill([1025] * 4, 4, 1024, cpp=4)
    assert len(its) == 1024 and big == 65 and all(m[3] == 64 for m in ms)
    _check_plan_shape(its, ms, npart, [1025] * 4, 4, cpp=4)
    # C3's shape already fills the budget: 8-page items, which chunk cuts keep on page boundaries
    for cpp in (1, 2):
        its, ms, npart, big = _plan_fill([256] * 8, 4, 1024, cpp=cpp)
        assert len(its) == 1024 and big == 8 * cpp and all(u1 - u0 == 8 * cpp for (_, _, u0, u1, _) in its)
        assert all(u0 % cpp == 0 for (_, _, u0, _, _) in its)


def test_fill_planner_page_costs():
    """Costed pages: each stream is cut at its cost quantiles, so no item
    costs more than its stream's mean item cost plus one chunk; the streams
    with dearer pages get more items."""
    rng = np.random.default_rng(5)
    pages = [1025] * 4
    cost = np.ones((4, 4, 1025), dtype=np.float32)
    cost[:, :, -2:] = 2.2  # the exact recent window of a long-context pool
    cost[:, 1, :] *= 1.5    # one KV head's keys held exact
    cpp = 4
    its, ms, npart, big = _plan_fill(pages, 4, 1024, cpp=cpp, cost=cost)
    assert len(its) <= 1024
    _check_plan_shape(its, ms, npart, pages, 4, cpp=cpp, equal=False)
    chunk = np.repeat(cost, cpp, axis=2) / cpp
    per_stream = {}
    for (b, h, u0, u1, _) in its:
        per_stream.setdefault((b, h), []).append(float(chunk[b, h, u0:u1].sum()))
    for (b, h), c in per_stream.items():
        assert max(c) <= chunk[b, h].sum() / len(c) + chunk[b, h].max() + 1e-6
    n_items = {k: len(v) for k, v in per_stream.items()}
    assert all(n_items[(b, 1)] > n_items[(b, 0)] for b in range(4))
    # the largest item cost is within one chunk of the best split of the budget
    worst = max(max(c) for c in per_stream.values())
    assert worst <= chunk.sum() / 1024 * 1.05 + chunk.max()
    # random costs on ragged streams: same guarantees
    pages = rng.integers(1, 200, size=12).tolist()
    cost = rng.uniform(0.5, 3.0, size=(12, 2, 200)).astype(np.float32)
    its, ms, npart, big = _plan_fill(pages, 2, 150, cpp=2, cost=cost)
    assert len(its) <= 150
    _check_plan_shape(its, ms, npart, pages, 2, cpp=2, equal=False)
    with pytest.raises(ValueError):  # a negative cost
        bad = cost.copy()
        bad[0, 0, 0] = -1.0
        _plan_fill(pages, 2, 150, cpp=2, cost=bad)
    with pytest.raises(ValueError):  # costs shorter than the longest sequence
        _plan_fill(pages, 2, 150, cpp=2, cost=cost[:, :, : max(pages) - 1])


def test_fill_planner_ragged_and_limits():
    rng = np.random.default_rng(11)
    pages = rng.integers(1, 300, size=20).tolist()
    for cpp in (1, 2, 4):
        its, ms, npart, big = _plan_fill(pages, 2, 100, cpp=cpp)
        assert len(its) <= 100
        _check_plan_shape(its, ms, npart, pages, 2, cpp=cpp)
        # no split item below the minimum (two pages' chunks)
        assert all(u1 - u0 >= 2 * cpp for (s, _, u0, u1, part) in its if part >= 0)
        # never a larger item than the smallest whole-page split that fits
        from dotcache_amd.decode import choose_pages_per_split

        assert big <= cpp * choose_pages_per_split(np.asarray(pages), 2, target_items=100)
    # more streams than the budget: one item per stream, over the target
    its, ms, npart, big = _plan_fill([3] * 10, 2, 8)
    assert len(its) == 20 and not ms and big == 3
    with pytest.raises(ValueError):
        _plan_fill([3, 0], 1, 8)
    with pytest.raises(ValueError):  # no item budget
        _plan_fill([3], 1, 0)
    with pytest.raises(ValueError):  # no chunks per page
        _plan_fill([3], 1, 8, cpp=0)


def test_fill_planner_cuts_only_chunks_that_hold_tokens():
    """A partial last page counts only the chunks that hold tokens: 128-token
    pages (4 chunks), last pages of 10, 33 and 128 tokens.  Without the
    counts, four items over two pages put the last item on the 10-token
    page's empty chunks 2 and 3."""
    its, ms, npart, _ = _plan_fill([2], 1, 4, cpp=4, min_chunks=1)
    assert (0, 0, 6, 8, 3) in its  # the empty tail, as an item of its own
    its, ms, npart, big = _plan_fill([2], 1, 4, cpp=4, min_chunks=1, last_tokens=[10])
    assert [(u0, u1) for (_, _, u0, u1, _) in its] == [(0, 1), (1, 2), (2, 3), (3, 5)] and big == 2
    _check_plan_shape(its, ms, npart, [2], 1, cpp=4, last_chunks=[1])
    # several sequences and heads, with and without page costs
    sp, last = [2, 3, 5], [10, 33, 128]
    lc = [(t + 31) // 32 for t in last]
    for cost in (None, np.random.default_rng(0).uniform(0.5, 2.0, size=(3, 2, 5)).astype(np.float32)):
        its, ms, npart, _ = _plan_fill(sp, 2, 24, cpp=4, cost=cost, min_chunks=1, last_tokens=last)
        _check_plan_shape(its, ms, npart, sp, 2, cpp=4, equal=cost is None, last_chunks=lc)
    with pytest.raises(ValueError):  # more tokens than a page holds
        _plan_fill([2], 1, 4, cpp=4, last_tokens=[129])
    with pytest.raises(ValueError):
        _plan_fill([2], 1, 4, cpp=4, last_tokens=[0])


def test_make_plan_chunk_fields_and_checks():
    """make_plan's fill plans carry the chunk cuts; DecodePlan.check rejects
    them for pools of another page size."""
    from dotcache_amd.decode import chunks_per_page, make_plan

    assert [chunks_per_page(c) for c in (16, 32, 48, 64, 128, 256)] == [1, 1, 2, 2, 4, 8]
    plan = make_plan([1025] * 4, 4, device="cpu", target_items=1024, chunks_per_page=4)
    assert plan.n_items == 1024 and plan.largest_chunks == 65 and plan.pages_per_split == 17
    cb, ce = plan.host_items[:, 5], plan.host_items[:, 6]
    assert np.any(cb != 0) and np.any(ce != 0)
    plan.check(np.full(4, 1025), 4, 1025, 4)
    with pytest.raises(ValueError):
        plan.check(np.full(4, 1025), 4, 1025, 2)
    cost = np.ones((4, 4, 1025), dtype=np.float32)
    with pytest.raises(ValueError):
        make_plan([1025] * 4, 4, device="cpu", target_items=1024, chunks_per_page=4, page_cost=cost[:, :2])
    costed = make_plan([1025] * 4, 4, device="cpu", target_items=1024, chunks_per_page=4, page_cost=cost)
    assert np.array_equal(costed.host_items, plan.host_items)


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


def test_page_costs_weigh_pages_within_a_stream():
    """page_costs: within a stream, pages cost their compressed bytes plus a
    fixed amount per 32-token chunk; each stream's costs sum to its page
    count; past a sequence's pages the cost is 0."""
    from dotcache_amd.decode import CHUNK_COST_BYTES, page_costs
    from dotcache_amd.page_pool import DevicePagePool, PoolGeometry

    geo = PoolGeometry(128, 32, 64)
    kp = DevicePagePool(geo, device="cpu", reserve_bytes=1 << 20, reserve_pages=32)
    vp = DevicePagePool(geo, device="cpu", reserve_bytes=1 << 20, reserve_pages=32)
    m0k = kp.allocate(_lib.FMT_M0_AFFINE, 4, 3, tokens=64)
    m3k = kp.allocate(_lib.FMT_M3_F16, 0, 2, tokens=64)
    kp.set_tokens(m3k[1:], 5)  # a partial newest page
    vids = vp.allocate(_lib.FMT_M0_SYMMETRIC, 4, 5, tokens=64)
    vp.set_tokens(vids[4:], 5)
    kt = np.zeros((2, 1, 4), np.int32)
    vt = np.zeros((2, 1, 4), np.int32)
    kt[0, 0] = [m0k[0], m0k[1], m0k[2], m3k[0]]  # stream 0: three M0 pages, then an exact page
    vt[0, 0] = vids[:4]
    kt[1, 0, :1] = [m3k[1]]                      # stream 1: one partial page
    vt[1, 0, :1] = [vids[4]]
    c = page_costs(kp, vp, kt, vt, np.array([4, 1]))
    g = geo.c()
    raw = np.array([_lib.page_read_bytes(_lib.FMT_M0_AFFINE, 4, 64, g)] * 3 + [_lib.page_read_bytes(_lib.FMT_M3_F16, 0, 64, g)],
                   np.float64)
    raw += _lib.page_read_bytes(_lib.FMT_M0_SYMMETRIC, 4, 64, g) + 2 * CHUNK_COST_BYTES
    np.testing.assert_allclose(c[0, 0], raw * 4 / raw.sum(), rtol=1e-6)
    assert c[0, 0, 3] > 1.3 * c[0, 0, 0]  # the exact page reads 16 KiB of keys instead of 5
    np.testing.assert_allclose(c[1, 0], [1.0, 0.0, 0.0, 0.0])


def test_page_record_calls_reject_bad_strides():
    """dc_gather_page_records and dc_decode_paged_records check rec_stride
    (1..64) before touching the device."""
    L = _lib.lib()
    geo = _lib.geometry(128, 32, 64)
    pool = _lib.Pool(None, 0, None, 0, geo, 0)
    assert C.sizeof(_lib.PageRecord) == 16
    for bad in (0, 65):
        assert L.dc_gather_page_records(pool, pool, None, None, 1, None, 1, 1, 1, None, bad, None) == _lib.DC_EINVAL
        assert L.dc_decode_paged_records(pool, pool, None, None, 1, None, 1, None, 0, None, _lib.DT_F32, 1.0, 1, 1,
                                         1, None, None, 0, C.c_void_p(16), bad, None) == _lib.DC_EINVAL


def test_waves_per_simd_follows_the_instance():
    """dc_decode_waves_per_simd walks the MFMA kernel's instance selection
    without launching: 2 for M0 keys at head_dim 128 with up to 8 heads per
    block (C4's pools), 1 for M3 keys (C3), head_dim 256 (C5), 16-head
    blocks, and the generic kernel."""
    from dotcache_amd.decode import set_decode_path, set_mfma_head_block

    L = _lib.lib()

    def pool(hd, gs, masks):
        m = 0
        for fmt, bits in masks:
            m |= _lib.format_bit(fmt, bits)
        return _lib.Pool(None, 0, None, 0, _lib.geometry(hd, gs, 64), m)

    m3, aff4, sym4, sym8 = (_lib.FMT_M3_F16, 0), (_lib.FMT_M0_AFFINE, 4), (_lib.FMT_M0_SYMMETRIC, 4), (
        _lib.FMT_M0_SYMMETRIC, 8)
    c4 = (pool(128, 32, [m3, aff4]), pool(128, 64, [sym8]))
    c3 = (pool(128, 32, [m3]), pool(128, 32, [sym4]))
    c5 = (pool(256, 32, [m3, aff4]), pool(256, 32, [m3, aff4]))
    try:
        assert L.dc_decode_waves_per_simd(*c4, 6) == 2
        assert L.dc_decode_waves_per_simd(*c4, 12) == 1  # a 16-head block
        assert L.dc_decode_waves_per_simd(*c3, 7) == 1
        assert L.dc_decode_waves_per_simd(*c5, 4) == 1
        set_mfma_head_block(16)
        assert L.dc_decode_waves_per_simd(*c4, 6) == 1
        set_mfma_head_block(0)
        set_decode_path("generic")
        assert L.dc_decode_waves_per_simd(*c4, 6) == 1
    finally:
        set_decode_path("auto")
        set_mfma_head_block(0)
