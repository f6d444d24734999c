"""Window page selection and session bookkeeping on the CPU (reference
``dotcache/session_runtime.py:192-216``, ``:442-480``, ``:483-560``;
``tests/test_torch_mps_backend.py:81-97``)."""
import numpy as np
import pytest

from dotcache_amd.session_runtime import (PagedDecodeSession, select_execution_page_indices,
                                          select_execution_page_pairs, select_window_page_indices)
from oracle import dotcache_oracle as O
from tests.helpers import to_product_page


def _paged(n_tokens, seed, kind, P=64):
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(n_tokens, 32)).astype(np.float32)
    return [to_product_page(p) for p in O.encode_pages(x, tokens_per_page=P, head_dim=32, group_size=32, kind=kind,
                                                       bits=4, mode="M0")]


def test_select_execution_page_pairs_keeps_sink_and_recent_pages():
    kp, vp = _paged(320, 20, "K"), _paged(320, 21, "V")
    sk, sv = select_execution_page_pairs(kp, vp, recent_window_tokens=64, sink_window_tokens=64)
    assert [p.header.token_start for p in sk] == [0, 256]
    assert [p.header.token_start for p in sv] == [0, 256]


@pytest.mark.parametrize("recent, sink, want", [
    (None, 0, [0, 1, 2, 3, 4]),   # no window: every page
    (64, 0, [3, 4]),              # end 300: [236, 300) touches pages 3 and 4
    (44, 0, [4]),                 # exactly the partial last page
    (None, 65, [0, 1]),           # the sink spills one token into page 1
    (1000, 0, [0, 1, 2, 3, 4]),   # a window longer than the context
    (1, 1, [0, 4]),
])
def test_window_indices_known_answers(recent, sink, want):
    kp = _paged(300, 3, "K")
    got = select_execution_page_indices(kp, recent_window_tokens=recent, sink_window_tokens=sink)
    assert got == want
    if recent or sink:
        assert select_window_page_indices(kp, recent_window_tokens=recent, sink_window_tokens=sink) == want


def test_shortlist_argument_checks():
    """The reference's errors: a shortlist needs a query, the mode must be
    sketch or envelope, the sketch size positive, key and value lists equal."""
    kp = _paged(128, 4, "K")
    with pytest.raises(ValueError, match="query_slice"):
        select_execution_page_indices(kp, relevance_top_k=1)
    with pytest.raises(ValueError, match="relevance_mode"):
        PagedDecodeSession(relevance_top_k=2, relevance_mode="dense")
    with pytest.raises(ValueError, match="sketch_size"):
        PagedDecodeSession(relevance_top_k=2, relevance_sketch_size=0)
    with pytest.raises(ValueError):
        select_execution_page_pairs(kp, kp[:1])


def test_session_bookkeeping_without_the_device():
    kp, vp = _paged(320, 5, "K"), _paged(320, 6, "V")
    s = PagedDecodeSession(recent_window_tokens=64, sink_window_tokens=64, relevance_sketch_size=4)
    with pytest.raises(ValueError, match="preloaded"):
        s.decode(np.zeros(32, np.float32))
    s.preload(kp[:3], vp[:3], prepare=False)
    s.append(kp[3:], vp[3:], prepare=False)
    assert s.page_count == 5
    assert s.execution_indices() == [0, 4]
    assert s.active_page_count == 2 and s.active_token_count == 128
    sk, sv = s.execution_pages()
    assert sk[1] is kp[4] and sv[0] is vp[0]
    with pytest.raises(ValueError):
        s.append(kp[:1], [], prepare=False)
    s.clear()
    assert s.page_count == 0
