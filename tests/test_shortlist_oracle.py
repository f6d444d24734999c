"""The shortlist oracle pinned on the CPU: the reference's known-answer
tests for page selection and summaries (``tests/test_torch_mps_backend.py``
of the reference, ``:65-200``) restated on oracle pages, and closed forms
(one-row sketch = mean of the dense rows, envelope = their min / max,
shortlist = brute-force best k, a shortlist that admits every page decodes
like ``decode_step``)."""
import numpy as np
import pytest

from oracle import dotcache_oracle as O
from oracle import shortlist_oracle as S


def _paged(x, kind, tpp=64, hd=32, meta=True):
    return O.encode_pages(x, tokens_per_page=tpp, head_dim=hd, group_size=min(32, hd), kind=kind, bits=4,
                          build_runtime_metadata=meta)


def test_encoder_stores_runtime_sketch_metadata():
    """Reference ``:65-78``: mean [hd], sketch [4, hd], min / max [hd], fp16 of the raw rows."""
    rng = np.random.default_rng(19)
    x = rng.normal(size=(64, 32)).astype(np.float32)
    p = _paged(x, "K")[0]
    assert p.runtime_page_mean.shape == (32,) and p.runtime_page_sketch.shape == (4, 32)
    assert p.runtime_page_min.shape == (32,) and p.runtime_page_max.shape == (32,)
    np.testing.assert_array_equal(p.runtime_page_sketch[1], x[16:32].mean(axis=0).astype(np.float16))
    np.testing.assert_array_equal(p.runtime_page_max, x.max(axis=0).astype(np.float16))


def test_relevant_old_page_is_admitted():
    """Reference ``:100-124``."""
    rng = np.random.default_rng(201)
    keys = rng.normal(size=(320, 32)).astype(np.float32) * 0.01
    keys[128:192, 0] = 10.0
    kp = _paged(keys, "K")
    q = np.zeros(32, np.float32)
    q[0] = 1.0
    summaries = [np.full(32, -1.0, np.float32) for _ in kp]
    summaries[2] = np.concatenate([[10.0], np.zeros(31)]).astype(np.float32)
    got = S.select_execution_page_indices(kp, recent_window_tokens=64, sink_window_tokens=64, query_slice=q,
                                          key_page_sketches=[s[None, :] for s in summaries], relevance_top_k=1)
    assert got == [0, 2, 4]


def test_chunk_sketch_keeps_local_signal():
    """Reference ``:127-138``: dense fallback (no stored sketch of 4 rows asked)."""
    x = np.zeros((64, 32), np.float32)
    x[:16, 0] = 8.0
    x[16:, 0] = -2.0
    p = _paged(x, "K", meta=False)[0]
    sk = S.sketch_key_page(p, sketch_size=4)
    assert sk.shape == (4, 32) and sk[0, 0] > 6.0 and sk[-1, 0] < -1.0


def test_chunked_sketch_beats_page_mean_and_envelope_admits_spike():
    """Reference ``:141-197``."""
    rng = np.random.default_rng(202)
    kp = _paged(rng.normal(size=(320, 32)).astype(np.float32) * 0.01, "K")
    q = np.zeros(32, np.float32)
    q[0] = 1.0
    mean_like = [np.full((1, 32), -1.0, np.float32) for _ in kp]
    chunked = [np.full((4, 32), -1.0, np.float32) for _ in kp]
    chunked[2][0, 0] = 10.0
    kw = dict(recent_window_tokens=64, sink_window_tokens=64, query_slice=q, relevance_top_k=1)
    assert S.select_execution_page_indices(kp, key_page_sketches=mean_like, **kw) != [0, 2, 4]
    assert S.select_execution_page_indices(kp, key_page_sketches=chunked, **kw) == [0, 2, 4]
    lo = [np.full(32, -1.0, np.float32) for _ in kp]
    hi = [np.full(32, -1.0, np.float32) for _ in kp]
    hi[2][0] = 10.0
    assert S.select_execution_page_indices(kp, key_page_minima=lo, key_page_maxima=hi, relevance_mode="envelope",
                                           **kw) == [0, 2, 4]


def test_summaries_are_the_dense_closed_forms_without_metadata():
    rng = np.random.default_rng(3)
    p = _paged(rng.normal(size=(50, 32)).astype(np.float32), "K", meta=False)[0]
    dense = O.decode_page(p)
    np.testing.assert_allclose(S.sketch_key_page(p, sketch_size=1)[0], dense.mean(axis=0), rtol=1e-6)
    lo, hi = S.envelope_key_page(p)
    np.testing.assert_array_equal(lo, dense.min(axis=0))
    np.testing.assert_array_equal(hi, dense.max(axis=0))
    sk = S.sketch_key_page(p, sketch_size=3)  # np.array_split(50, 3) = 17, 17, 16 rows
    np.testing.assert_allclose(sk[2], dense[34:].mean(axis=0), rtol=1e-6)


@pytest.mark.parametrize("mode", ["sketch", "envelope"])
def test_shortlist_is_the_brute_force_best_k(mode):
    rng = np.random.default_rng(11)
    kp = _paged(rng.normal(size=(64 * 12, 32)).astype(np.float32), "K", meta=False)
    q = rng.normal(size=32).astype(np.float32)
    sk = [S.sketch_key_page(p, sketch_size=2) for p in kp]
    env = [S.envelope_key_page(p) for p in kp]
    got = S.select_execution_page_indices(kp, recent_window_tokens=64, query_slice=q, key_page_sketches=sk,
                                          key_page_minima=[e[0] for e in env], key_page_maxima=[e[1] for e in env],
                                          relevance_top_k=4, relevance_mode=mode)
    score = [S.score_page_relevance(q, relevance_mode=mode, page_sketch=sk[i], page_min=env[i][0],
                                    page_max=env[i][1]) for i in range(11)]
    best = sorted(range(11), key=lambda i: -score[i])[:4]
    assert got == sorted(best + [11])


def test_session_that_admits_every_page_is_decode_step():
    rng = np.random.default_rng(12)
    kp = _paged(rng.normal(size=(64 * 4, 32)).astype(np.float32), "K")
    vp = _paged(rng.normal(size=(64 * 4, 32)).astype(np.float32), "V")
    q = rng.normal(size=32).astype(np.float32)
    s = S.Session(relevance_top_k=8, approximate_old_pages=True, relevance_sketch_size=4)
    s.append(kp, vp)
    want = O.decode_step(q, kp, vp)
    got = s.decode(q)
    for a, b in zip(got, want):
        np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-7)
