"""The prepared-page cache on the device: the reference's cache-reuse test
(``tests/test_torch_mps_backend.py:581-627``) restated for hip_mi355x, and a
budget-bounded decode loop whose pool stays the size of the budget."""
import gc

import numpy as np
import pytest

from oracle import dotcache_oracle as O
from tests.helpers import to_product_page

pytestmark = pytest.mark.gpu


def _oracle_paged(x, kind):
    return O.encode_pages(x, tokens_per_page=64, head_dim=128, group_size=32, kind=kind, bits=4, mode="M0")


def _paged(x, kind):
    return [to_product_page(p) for p in _oracle_paged(x, kind)]


def test_prepared_page_cache_reuses_pages_across_decode_steps():
    from dotcache_amd import attention_runtime as rt
    from dotcache_amd.page_cache import PreparedPageCache
    from dotcache_amd.tracing import ExecutionTrace

    rng = np.random.default_rng(27)
    keys = rng.normal(size=(160, 128)).astype(np.float32)
    values = rng.normal(size=(160, 128)).astype(np.float32)
    qa, qb = rng.normal(size=(2, 128)).astype(np.float32)
    kp, vp = _paged(keys, "K"), _paged(values, "V")
    cache = PreparedPageCache()
    first, second = ExecutionTrace(), ExecutionTrace()
    la, _, oa = rt.decode_step(qa, kp, vp, backend="hip_mi355x", cache=cache, trace=first)
    lb, _, ob = rt.decode_step(qb, kp, vp, backend="hip_mi355x", cache=cache, trace=second)
    okp, ovp = _oracle_paged(keys, "K"), _oracle_paged(values, "V")
    for q, lg, out in ((qa, la, oa), (qb, lb, ob)):
        want = O.decode_step(q, okp, ovp)
        np.testing.assert_allclose(lg, want[0], atol=1e-4, rtol=1e-4)
        np.testing.assert_allclose(out, want[2], atol=1e-4, rtol=1e-4)
    total = len(kp) + len(vp)
    assert first.prepared_page_cache_misses == total and first.prepared_page_cache_hits == 0
    assert first.host_to_device_bytes > 0
    assert second.prepared_page_cache_hits == total and second.prepared_page_cache_misses == 0
    assert second.host_to_device_bytes == 0
    assert second.cache_resident_bytes == cache.resident_bytes


def test_budgeted_cache_keeps_the_pool_bounded():
    """Twenty steps over a sliding window of fresh pages with a 4-page
    budget: outputs match the oracle every step, the cache never exceeds its
    budget, and the pool's used blocks and id table stop growing once
    evicted pages come back to it."""
    from dotcache_amd import attention_runtime as rt
    from dotcache_amd.page_cache import PreparedPageCache
    from dotcache_amd.tracing import ExecutionTrace

    rng = np.random.default_rng(31)
    probe = _paged(rng.normal(size=(64, 128)).astype(np.float32), "K")[0]
    blob = rt.prepare_page(probe, backend="hip_mi355x").resident_nbytes
    cache = PreparedPageCache(max_resident_bytes=4 * blob, policy="lru")
    trace = ExecutionTrace()
    sizes = []
    for step in range(20):
        keys = rng.normal(size=(128, 128)).astype(np.float32)
        values = rng.normal(size=(128, 128)).astype(np.float32)
        q = rng.normal(size=(128,)).astype(np.float32)
        kp, vp = _paged(keys, "K"), _paged(values, "V")
        _, _, out = rt.decode_step(q, kp, vp, backend="hip_mi355x", cache=cache, trace=trace)
        want = O.decode_step(q, _oracle_paged(keys, "K"), _oracle_paged(values, "V"))[2]
        np.testing.assert_allclose(out, want, atol=1e-4, rtol=1e-4, err_msg=f"step {step}")
        assert cache.resident_bytes <= 4 * blob
        del kp, vp
        gc.collect()
        pool = next(iter(cache._entries.values())).pool
        sizes.append((pool._next_block, pool.n_pages))
    assert trace.prepared_page_cache_evictions == 20 * 4 - 4
    assert trace.cache_resident_bytes == 4 * blob
    assert sizes[-1] == sizes[2], sizes
