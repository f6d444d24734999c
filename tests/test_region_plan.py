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
def test_lead_trail_plans_cover_each_chunk_once(ratio):
    """Lead-trail plans (instances at two waves per SIMD): the first half of
    the items are the SIMD shares' leads, the second half their trails in
    the same order, each pair cut from one share at about ratio : 1, and
    the chunks covered are exactly a plain plan's."""
    from dotcache_amd.decode import _item_chunks, make_plan

    sp = np.array([40, 7, 300, 33, 1], dtype=np.int32)
    H, cpp = 2, 2
    last = np.array([64, 10, 33, 64, 5], dtype=np.int32)
    plain = make_plan(sp, H, device="cpu", chunks_per_page=cpp, target_items=32, last_page_tokens=last)
    lt = make_plan(sp, H, device="cpu", chunks_per_page=cpp, target_items=64, last_page_tokens=last,
                   lead_ratio=ratio)
    assert sorted(_chunks(plain.host_items, cpp)) == sorted(_chunks(lt.host_items, cpp))
    n_share = plain.n_items
    lead, trail = lt.host_items[:n_share], lt.host_items[n_share:]
    # every share of two or more chunks became a (lead, trail) pair; those
    # leads come first, in order, then the one-chunk shares, then the
    # trails in the leads' order
    pi = plain.host_items
    big = _item_chunks(pi, cpp) >= 2
    assert len(trail) == int(big.sum()) and int(big.sum()) < n_share
    c_lead, c_trail = _item_chunks(lead[: len(trail)], cpp), _item_chunks(trail, cpp)
    assert np.array_equal(lead[: len(trail), :2], trail[:, :2])
    assert np.array_equal(lead[: len(trail), :2], pi[big, :2])
    assert np.all(np.abs(c_lead - ratio * c_trail) <= ratio + 1)
    assert np.array_equal(lead[len(trail):, :2], pi[~big, :2])
    lt.check(sp, H, 300, cpp)
    for seq, head, first, count in lt.host_merges:
        rows = np.flatnonzero((lt.host_items[:, 0] == seq) & (lt.host_items[:, 1] == head))
        assert sorted(lt.host_items[rows, 4].tolist()) == list(range(first, first + count))
