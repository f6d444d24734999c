"""Region plans (``make_region_plan``) on the host: the front pages of each
stream go to their own leading items, every token chunk of every stream is
covered exactly once, and each stream's partials are consecutive slots
named by one merge item."""
import numpy as np
import pytest

from dotcache_amd.decode import make_region_plan


def _chunks(items, cpp):
    """(seq, head, absolute chunk) triples the items cover."""
    out = []
    for seq, head, pb, pe, _, cb, ce, _ in items:
        first = pb * cpp + cb
        end = pe * cpp if ce == 0 else (pe - 1) * cpp + ce
        out += [(seq, head, c) for c in range(first, end)]
    return out


@pytest.mark.parametrize("front_items", [None, 3])
def test_region_plan_covers_each_chunk_once(front_items):
    sp = np.array([9, 4, 1, 12], dtype=np.int32)
    H, cpp = 3, 4
    last = np.array([128, 37, 5, 90], dtype=np.int32)
    front = np.array([[7, 8], [0, 4], [0, 1], [12, 12]])  # middle, whole stream, one-page stream, none
    plan = make_region_plan(sp, H, front, device="cpu", chunks_per_page=cpp, last_page_tokens=last,
                            target_items=40, front_items=front_items)
    it = plan.host_items
    nf = plan.n_front
    # front items only inside the front ranges, bulk items only outside
    for k, (seq, head, pb, pe, *_rest) in enumerate(it):
        inside = front[seq, 0] <= pb and pe <= front[seq, 1]
        assert inside == (k < nf), (k, it[k])
    want = []
    for b in range(len(sp)):
        n_chunks = (sp[b] - 1) * cpp + (last[b] + 31) // 32
        want += [(b, h, c) for h in range(H) for c in range(n_chunks)]
    got = _chunks(it, cpp)
    assert sorted(got) == sorted(want) and len(got) == len(want)
    if front_items is None:  # one front item per chunk
        fr_chunks = sum(len(_chunks(it[k:k + 1], cpp)) for k in range(nf))
        assert nf == fr_chunks
    # partial slots: consecutive per stream, one merge each
    part = it[:, 4]
    seen = set()
    for seq, head, first, count in plan.host_merges:
        rows = np.flatnonzero((it[:, 0] == seq) & (it[:, 1] == head))
        assert len(rows) == count > 1
        assert sorted(part[rows].tolist()) == list(range(first, first + count))
        seen.add((seq, head))
    for seq, head in {(int(s), int(h)) for s, h in it[:, :2]} - seen:
        rows = np.flatnonzero((it[:, 0] == seq) & (it[:, 1] == head))
        assert len(rows) == 1 and part[rows[0]] == -1
    assert plan.n_partials == int((part >= 0).sum())
    plan.check(sp, H, 16, cpp)


def test_region_plan_rejects_bad_ranges():
    sp = np.array([4, 4], dtype=np.int32)
    with pytest.raises(ValueError):
        make_region_plan(sp, 1, np.array([[0, 5], [0, 1]]), device="cpu", chunks_per_page=2)
    with pytest.raises(ValueError):
        make_region_plan(sp, 1, np.array([[3, 2], [0, 1]]), device="cpu", chunks_per_page=2)


@pytest.mark.parametrize("ratio", [1.0, 1.6, 3.0])
def test_lead_trail_split_layout(ratio):
    """lead_trail_split on a plain plan's shares: the first items are the
    shares' leads, then the one-chunk shares, then the trails in the same
    order, each pair cut from one share at about ratio : 1, covering
    exactly the shares' chunks."""
    from dotcache_amd.decode import _item_chunks, lead_trail_split, make_plan

    sp = np.array([40, 7, 300, 33, 1], dtype=np.int32)
    H, cpp = 2, 2
    last = np.array([64, 10, 33, 64, 5], dtype=np.int32)
    pi = make_plan(sp, H, device="cpu", chunks_per_page=cpp, target_items=32, last_page_tokens=last).host_items
    lt = lead_trail_split(pi, ratio, cpp)
    assert sorted(_chunks(pi, cpp)) == sorted(_chunks(lt, cpp))
    n_share = len(pi)
    lead, trail = lt[:n_share], lt[n_share:]
    big = _item_chunks(pi, cpp) >= 2
    assert len(trail) == int(big.sum()) and int(big.sum()) < n_share
    c_lead, c_trail = _item_chunks(lead[: len(trail)], cpp), _item_chunks(trail, cpp)
    assert np.array_equal(lead[: len(trail), :2], trail[:, :2])
    assert np.array_equal(lead[: len(trail), :2], pi[big, :2])
    assert np.all(np.abs(c_lead - ratio * c_trail) <= ratio + 1)
    assert np.array_equal(lead[len(trail):, :2], pi[~big, :2])


def _check_lead_trail_plan(lt, plain, sp, H, cpp, stride):
    """A lead-trail plan covers the plain plan's chunks once; its first
    n_share items (one per SIMD share) are followed by trails, trail j
    sharing item j's SIMD: either the rest of item j's share (same stream,
    the chunks right after the lead's) or, in a pair, a whole stream no
    longer than the whole-stream lead.  Returns the number of pairs."""
    from dotcache_amd.decode import _item_chunks

    it = lt.host_items
    assert sorted(_chunks(plain.host_items, cpp)) == sorted(_chunks(it, cpp))
    n_share = plain.n_items
    n_trail = len(it) - n_share
    assert 0 < n_trail <= n_share
    ch = _item_chunks(it, cpp)
    first = it[:, 2].astype(np.int64) * cpp + it[:, 5]
    stream = it[:, 0].astype(np.int64) * H + it[:, 1]
    n_items = np.bincount(stream, minlength=len(sp) * H)
    pairs = 0
    for j in range(n_trail):
        a, b = it[j], it[n_share + j]
        if stream[j] == stream[n_share + j]:
            assert first[n_share + j] == first[j] + ch[j]  # the trail starts where the lead ends
        else:
            pairs += 1
            assert n_items[stream[j]] == 1 and n_items[stream[n_share + j]] == 1
            assert a[4] == -1 and b[4] == -1 and ch[j] >= ch[n_share + j]
    lt.check(sp, H, stride, cpp)
    for seq, head, first, count in lt.host_merges:
        rows = np.flatnonzero((it[:, 0] == seq) & (it[:, 1] == head))
        assert sorted(it[rows, 4].tolist()) == list(range(first, first + count))
    return pairs


@pytest.mark.parametrize("ratio", [1.0, 1.6, 3.0])
def test_lead_trail_plans_cover_each_chunk_once(ratio):
    """make_plan(lead_ratio=...) on a small ragged batch."""
    from dotcache_amd.decode import make_plan

    sp = np.array([40, 7, 300, 33, 1], dtype=np.int32)
    H, cpp = 2, 2
    last = np.array([64, 10, 33, 64, 5], dtype=np.int32)
    plain = make_plan(sp, H, device="cpu", chunks_per_page=cpp, target_items=32, last_page_tokens=last)
    lt = make_plan(sp, H, device="cpu", chunks_per_page=cpp, target_items=64, last_page_tokens=last,
                   lead_ratio=ratio)
    _check_lead_trail_plan(lt, plain, sp, H, cpp, 300)


def test_lead_trail_plans_pair_short_streams():
    """The C4 batch (64 sequences, 256 to 32768 tokens, two KV heads): short
    streams share SIMDs in pairs, which lowers the largest modelled SIMD
    time below the plain lead-trail plan's and leaves those streams without
    a merge."""
    from dotcache_amd.decode import _item_chunks, _pair_time, lead_trail_split, make_plan, LONE_WAVE_RATE
    from dotcache_amd.workloads import SPECS, context_lengths

    ctx = context_lengths(SPECS["c4"], 0)
    sp = ((ctx + 63) // 64).astype(np.int32)
    last = (ctx - (sp - 1) * 64).astype(np.int32)
    H, cpp, n_simd = 2, 2, 1024
    plain = make_plan(sp, H, device="cpu", chunks_per_page=cpp, target_items=n_simd, last_page_tokens=last)
    lt = make_plan(sp, H, device="cpu", chunks_per_page=cpp, target_items=2 * n_simd, last_page_tokens=last,
                   lead_ratio=1.6)
    assert _check_lead_trail_plan(lt, plain, sp, H, cpp, int(sp.max())) > 0

    def worst(items):
        ch = _item_chunks(items, cpp).astype(float)
        nt = len(items) - n_simd
        return max(_pair_time(ch[j], ch[n_simd + j], 1.6) if j < nt else ch[j] / LONE_WAVE_RATE
                   for j in range(n_simd))

    assert worst(lt.host_items) < worst(lead_trail_split(plain.host_items, 1.6, cpp))
    assert lt.n_merges < len(sp) * H


@pytest.mark.parametrize("sp,H,target", [([6] * 6, 1, 32), ([6, 6, 1, 1, 1, 1], 1, 32), ([2] * 40, 1, 64),
                                         ([50, 1, 1, 1, 1, 2, 2], 2, 64), ([300, 3, 3, 9, 1], 4, 64)])
def test_lead_trail_plans_on_edge_batches(sp, H, target):
    """Lead-trail plans (with or without paired streams) on batches of only
    short streams, of one long stream among one-page ones, and with more
    shares than chunks to fill them: every chunk once, trails aligned."""
    from dotcache_amd.decode import make_plan

    sp = np.asarray(sp, dtype=np.int32)
    cpp = 2
    plain = make_plan(sp, H, device="cpu", chunks_per_page=cpp, target_items=target // 2)
    lt = make_plan(sp, H, device="cpu", chunks_per_page=cpp, target_items=target, lead_ratio=1.6)
    if len(lt.host_items) > plain.n_items:
        _check_lead_trail_plan(lt, plain, sp, H, cpp, int(sp.max()))
    else:
        assert sorted(_chunks(plain.host_items, cpp)) == sorted(_chunks(lt.host_items, cpp))
        lt.check(sp, H, int(sp.max()), cpp)


def test_plans_reused_within_a_chunk():
    """A plan depends on the last pages only through their chunk counts: a
    decode step that appends a token reuses the cached plan until a new
    32-token chunk starts; last-page token counts out of range raise."""
    from dotcache_amd.decode import make_plan

    sp = np.array([9, 4, 30], dtype=np.int32)
    kw = dict(device="cpu", chunks_per_page=2, target_items=24)
    a = make_plan(sp, 2, last_page_tokens=np.array([33, 64, 1], np.int32), **kw)
    b = make_plan(sp, 2, last_page_tokens=np.array([40, 63, 20], np.int32), **kw)
    c = make_plan(sp, 2, last_page_tokens=np.array([32, 64, 1], np.int32), **kw)
    assert a is b and a is not c
    for bad in ([0, 64, 1], [33, 65, 1]):
        with pytest.raises(ValueError):
            make_plan(sp, 2, last_page_tokens=np.array(bad, np.int32), **kw)
