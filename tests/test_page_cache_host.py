"""The prepared-page cache's bookkeeping on the CPU (reference
``dotcache/page_cache.py:23-227``): byte budget, the three eviction
policies, hit/miss/eviction counters, and release of evicted pages to their
pool.  A stub preparer stands in for the device upload; the eviction orders
below are worked out by hand from the reference's ``_evict_one`` and
``_ensure_capacity`` (``page_cache.py:66-110``).  Also the pool's reuse of
freed blobs and ids, on a CPU-resident pool."""
import gc

import numpy as np
import pytest

from dotcache_amd.backends.hip_mi355x import PreparedPageHIP
from dotcache_amd.page_cache import PreparedPageCache
from dotcache_amd.tracing import ExecutionTrace
from oracle import dotcache_oracle as O
from tests.helpers import to_product_page

BLOB = 1024  # bytes per page in the stub pool


class StubPool:
    def __init__(self):
        self.next_id = 0
        self.live: set[int] = set()
        self.uploads = 0

    def blob_bytes(self, fmt, bits):
        return BLOB

    def free(self, pid):
        self.live.remove(pid)


def _stub_preparer(pool):
    def prepare(pages, *, trace=None):
        pool.uploads += 1
        out = []
        for p in pages:
            out.append(PreparedPageHIP(source_page=p, header=p.header, pool=pool, page_id=pool.next_id,
                                       host_to_device_nbytes=p.device_nbytes))
            pool.live.add(pool.next_id)
            pool.next_id += 1
        if trace is not None:
            trace.record_host_to_device(sum(p.device_nbytes for p in pages))
        return out
    return prepare


def _pages(n, seed=0):
    rng = np.random.default_rng(seed)
    return [to_product_page(O.encode_page(rng.normal(size=(16, 32)).astype(np.float32), head_dim=32, group_size=32,
                                          kind="K", bits=4, mode="M0")) for _ in range(n)]


def _cache(pool, **kw):
    return PreparedPageCache(preparer=_stub_preparer(pool), **kw)


def _cached_sources(cache, pages):
    return [i for i, p in enumerate(pages) if cache._entries.get(("hip", id(p))) is not None]


def test_fifo_budget_keeps_the_newest_and_releases_the_rest():
    pool = StubPool()
    pages = _pages(5)
    cache = _cache(pool, max_resident_bytes=3 * BLOB)
    trace = ExecutionTrace()
    for p in pages:
        cache.prepare_page(p, trace=trace)  # the caller keeps nothing
    gc.collect()
    assert _cached_sources(cache, pages) == [2, 3, 4]
    assert cache.size == 3 and cache.resident_bytes == 3 * BLOB
    assert trace.prepared_page_cache_misses == 5 and trace.prepared_page_cache_hits == 0
    assert trace.prepared_page_cache_evictions == 2 and trace.cache_evicted_bytes == 2 * BLOB
    assert trace.cache_resident_bytes == 3 * BLOB
    assert pool.live == {2, 3, 4}  # evicted blobs went back to the pool


@pytest.mark.parametrize("policy, kept", [("fifo", [1, 2, 3]), ("lru", [0, 2, 3]), ("pinned_recent_fifo", [1, 2, 3])])
def test_policies_choose_the_reference_victim(policy, kept):
    """a, b, c inserted; a hit; d inserted into a 3-page budget.  LRU drops
    b (a was touched); FIFO drops a, and so does pinned-recent FIFO with 2
    pinned (b and c, the newest when d arrives): a is the oldest unpinned."""
    pool = StubPool()
    pages = _pages(4)
    cache = _cache(pool, max_resident_bytes=3 * BLOB, policy=policy, pinned_recent_pages=2)
    cache.prepare_pages(pages[:3])
    trace = ExecutionTrace()
    cache.prepare_page(pages[0], trace=trace)
    assert trace.prepared_page_cache_hits == 1
    cache.prepare_page(pages[3])
    assert _cached_sources(cache, pages) == kept


def test_pinned_fallback_evicts_the_oldest_when_every_entry_is_pinned():
    pool = StubPool()
    pages = _pages(3)
    cache = _cache(pool, max_resident_bytes=BLOB, policy="pinned_recent_fifo", pinned_recent_pages=4)
    trace = ExecutionTrace()
    for p in pages:
        cache.prepare_page(p, trace=trace)
    assert _cached_sources(cache, pages) == [2]
    assert trace.prepared_page_cache_evictions == 2


def test_second_pass_is_all_hits_and_uploads_nothing():
    pool = StubPool()
    pages = _pages(6)
    cache = _cache(pool)
    first, second = ExecutionTrace(), ExecutionTrace()
    a = cache.prepare_pages(pages, trace=first)
    b = cache.prepare_pages(pages, trace=second)
    assert [x is y for x, y in zip(a, b)] == [True] * 6
    assert first.prepared_page_cache_misses == 6 and first.host_to_device_bytes > 0
    assert second.prepared_page_cache_hits == 6 and second.prepared_page_cache_misses == 0
    assert second.host_to_device_bytes == 0 and pool.uploads == 1
    assert second.cache_resident_bytes == cache.resident_bytes == 6 * BLOB
    assert all(cache.owns_prepared_page(p) for p in a)
    # an already-prepared page passes through as a hit
    t = ExecutionTrace()
    assert cache.prepare_page(a[2], trace=t) is a[2] and t.prepared_page_cache_hits == 1
    cache.clear()
    assert cache.size == 0 and cache.resident_bytes == 0 and not cache.owns_prepared_page(a[0])


def test_a_batch_larger_than_the_budget_returns_every_page():
    """Misses are inserted in order, each making room for itself, so the
    cache ends with the tail of the batch while the caller holds all of it."""
    pool = StubPool()
    pages = _pages(5)
    cache = _cache(pool, max_resident_bytes=2 * BLOB)
    out = cache.prepare_pages(pages)
    assert [p.source_page is s for p, s in zip(out, pages)] == [True] * 5
    assert _cached_sources(cache, pages) == [3, 4]
    assert pool.live == {0, 1, 2, 3, 4}  # the caller still holds the evicted ones
    del out
    gc.collect()
    assert pool.live == {3, 4}


def test_a_page_listed_twice_is_uploaded_once():
    pool = StubPool()
    pages = _pages(2)
    cache = _cache(pool)
    t = ExecutionTrace()
    out = cache.prepare_pages([pages[0], pages[1], pages[0]], trace=t)
    assert out[0] is out[2] and pool.next_id == 2
    assert cache.resident_bytes == 2 * BLOB
    assert t.prepared_page_cache_misses == 2 and t.prepared_page_cache_hits == 1


def test_zero_budget_keeps_only_the_newest_page():
    pool = StubPool()
    pages = _pages(2)
    cache = _cache(pool, max_resident_bytes=0)
    out = cache.prepare_pages(pages)
    cache.prepare_page(pages[1])
    assert len(out) == 2 and cache.size == 1  # room is made before insertion, as in the reference


def test_argument_checks():
    with pytest.raises(ValueError):
        PreparedPageCache(policy="random")
    with pytest.raises(ValueError):
        PreparedPageCache(max_resident_bytes=-1)
    with pytest.raises(ValueError):
        PreparedPageCache(pinned_recent_pages=-1)
    with pytest.raises(ValueError):
        PreparedPageCache().prepare_pages(_pages(1), backend="cpu_ref")


def test_default_preparer_needs_the_device():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(RuntimeError):
        PreparedPageCache().prepare_pages(_pages(1))


def test_pool_reuses_freed_blobs_and_ids():
    """Freed blobs take new pages (one upload, scattered into reused blobs),
    freed ids are handed out oldest-freed first, and the contents read back."""
    from dotcache_amd.page_pool import DevicePagePool, PoolGeometry

    rng = np.random.default_rng(5)
    pages = [to_product_page(O.encode_page(rng.normal(size=(64, 64)).astype(np.float32), head_dim=64, group_size=32,
                                           kind="K", bits=4, mode="M0")) for _ in range(4)]
    pool = DevicePagePool(PoolGeometry(64, 32, 64), device="cpu", reserve_bytes=1 << 16)
    ids = pool.upload_pages(pages)
    end = pool._next_block
    pool.free([ids[2], ids[0]])
    again = pool.upload_pages([pages[3], pages[1]])
    assert again.tolist() == [int(ids[2]), int(ids[0])] and pool._next_block == end
    more = pool.upload_pages([pages[0]])
    assert more.tolist() == [4] and pool._next_block > end
    live = {int(i): p for i, p in zip(ids, pages)}
    live.update({int(again[0]): pages[3], int(again[1]): pages[1], 4: pages[0]})
    for pid, p in live.items():
        d = pool.download_page(pid, kind="K")
        np.testing.assert_array_equal(d.payload, p.payload)
        np.testing.assert_array_equal(d.scales, p.scales)
        np.testing.assert_array_equal(d.bias, p.bias)
