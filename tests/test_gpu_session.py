"""The paged decode session on the device against the oracle: the
reference's session tests (``tests/test_torch_mps_backend.py:630-706``)
restated for hip_mi355x."""
import numpy as np
import pytest

from oracle import dotcache_oracle as O
from tests.helpers import to_product_page

pytestmark = pytest.mark.gpu


def _oracle_paged(x, kind):
    return O.encode_pages(x, tokens_per_page=64, head_dim=128, group_size=32, kind=kind, bits=4, mode="M0")


def test_paged_decode_session_separates_preload_append_and_decode():
    from dotcache_amd.page_cache import PreparedPageCache
    from dotcache_amd.session_runtime import PagedDecodeSession
    from dotcache_amd.tracing import ExecutionTrace

    rng = np.random.default_rng(127)
    keys = rng.normal(size=(192, 128)).astype(np.float32)
    values = rng.normal(size=(192, 128)).astype(np.float32)
    q = rng.normal(size=(128,)).astype(np.float32)
    okp, ovp = _oracle_paged(keys, "K"), _oracle_paged(values, "V")
    kp, vp = [to_product_page(p) for p in okp], [to_product_page(p) for p in ovp]
    session = PagedDecodeSession(backend="hip_mi355x", cache=PreparedPageCache())
    pre, app, dec = ExecutionTrace(), ExecutionTrace(), ExecutionTrace()
    session.preload(kp[:2], vp[:2], trace=pre)
    session.append(kp[2:], vp[2:], trace=app)
    logits, weights, out = session.decode(q, trace=dec)
    want = O.decode_step(q, okp, ovp)
    np.testing.assert_allclose(logits, want[0], atol=1e-4, rtol=1e-4)
    np.testing.assert_allclose(weights, want[1], atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(out, want[2], atol=1e-4, rtol=1e-4)
    assert pre.host_to_device_bytes > 0 and app.host_to_device_bytes > 0
    assert dec.host_to_device_bytes == 0
    assert session.page_count == 3


def test_paged_decode_session_windowed_decode_matches_selected_page_reference():
    from dotcache_amd.page_cache import PreparedPageCache
    from dotcache_amd.session_runtime import PagedDecodeSession
    from dotcache_amd.tracing import ExecutionTrace

    rng = np.random.default_rng(128)
    keys = rng.normal(size=(320, 128)).astype(np.float32)
    values = rng.normal(size=(320, 128)).astype(np.float32)
    q = rng.normal(size=(128,)).astype(np.float32)
    okp, ovp = _oracle_paged(keys, "K"), _oracle_paged(values, "V")
    session = PagedDecodeSession(backend="hip_mi355x", cache=PreparedPageCache(), recent_window_tokens=64,
                                 sink_window_tokens=64)
    session.preload([to_product_page(p) for p in okp], [to_product_page(p) for p in ovp])
    t = ExecutionTrace()
    logits, weights, out = session.decode(q, trace=t)
    want = O.decode_step(q, [okp[0], okp[4]], [ovp[0], ovp[4]])
    np.testing.assert_allclose(logits, want[0], atol=1e-4, rtol=1e-4)
    np.testing.assert_allclose(weights, want[1], atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(out, want[2], atol=1e-4, rtol=1e-4)
    assert session.last_selected_indices == [0, 4]
    assert session.active_page_count == 2 and session.active_token_count == 128
    assert t.host_to_device_bytes == 0
