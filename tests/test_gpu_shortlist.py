"""Execution shortlist on the device against the oracle: the reference's
selection known answers (``tests/test_torch_mps_backend.py:100-233`` of the
reference) through the device scorer and top-k, page summaries from stored
metadata and from the device reduction of dequantised rows, relevance and
the tie rule of the ranking, and whole session decodes with a shortlist,
exact refine and the approximate fallback
(``:710-855`` restated against the oracle session)."""
import numpy as np
import pytest

from oracle import dotcache_oracle as O
from oracle import shortlist_oracle as S
from tests.helpers import to_product_page

pytestmark = pytest.mark.gpu


def _paged(x, kind, *, hd=32, tpp=64, meta=True, **fmt):
    fmt = {"bits": 4, **fmt}
    return O.encode_pages(x, tokens_per_page=tpp, head_dim=hd, group_size=32, kind=kind,
                          build_runtime_metadata=meta, **fmt)


def _prod(pages):
    return [to_product_page(p) for p in pages]


def test_reference_selection_known_answers_on_the_device():
    from dotcache_amd.session_runtime import select_execution_page_indices as sel

    rng = np.random.default_rng(201)
    kp = _prod(_paged(rng.normal(size=(320, 32)).astype(np.float32) * 0.01, "K"))
    q = np.zeros(32, np.float32)
    q[0] = 1.0
    kw = dict(recent_window_tokens=64, sink_window_tokens=64, query_slice=q, relevance_top_k=1)
    one = [np.full((1, 32), -1.0, np.float32) for _ in kp]
    one[2] = np.concatenate([[10.0], np.zeros(31)]).astype(np.float32)[None, :]
    assert sel(kp, key_page_sketches=one, **kw) == [0, 2, 4]
    mean_like = [np.full((1, 32), -1.0, np.float32) for _ in kp]
    chunked = [np.full((4, 32), -1.0, np.float32) for _ in kp]
    chunked[2][0, 0] = 10.0
    assert sel(kp, key_page_sketches=mean_like, **kw) != [0, 2, 4]
    assert sel(kp, key_page_sketches=chunked, **kw) == [0, 2, 4]
    lo = [np.full(32, -1.0, np.float32) for _ in kp]
    hi = [np.full(32, -1.0, np.float32) for _ in kp]
    hi[2][0] = 10.0
    assert sel(kp, key_page_minima=lo, key_page_maxima=hi, relevance_mode="envelope", **kw) == [0, 2, 4]
    # matrix form with a tail row (reference :200-233)
    kp8 = _prod(O.encode_pages(np.zeros((24, 8), np.float32), tokens_per_page=4, head_dim=8, group_size=8,
                               kind="K", bits=4))
    q8 = np.zeros(8, np.float32)
    q8[0] = 1.0
    mn = np.full((5, 8), -1.0, np.float32)
    mx = np.full((5, 8), -1.0, np.float32)
    mx[2, 0] = 10.0
    stats = {}
    got = sel(kp8, recent_window_tokens=4, sink_window_tokens=4, query_slice=q8, key_page_minima_matrix=mn,
              key_page_maxima_matrix=mx, tail_page_minimum=np.full(8, -1.0, np.float32),
              tail_page_maximum=np.full(8, -1.0, np.float32), relevance_top_k=1, relevance_mode="envelope",
              score_all_pages_with_matrices=True, score_all_pages_min_candidate_fraction=0.9,
              selector_stats_recorder=stats.update)
    assert got == [0, 2, 5]
    assert stats["used_score_all_pages"] is False and stats["candidate_pages"] == 4


@pytest.mark.parametrize("fmt", [dict(bits=4), dict(bits=8, scheme="symmetric"), dict(mode="M3")],
                         ids=["m0a4", "m0s8", "m3"])
@pytest.mark.parametrize("sketch_size", [1, 3, 4, 8])
def test_device_summaries_match_the_oracle(fmt, sketch_size):
    """Pages without stored metadata are reduced on the device; pages with
    it use the stored fp16 arrays by the reference's rules.  Pages of 64 and
    5 tokens (fewer tokens than sketch rows for sketch size 8)."""
    import torch

    from dotcache_amd.shortlist import key_page_summaries, value_page_means

    rng = np.random.default_rng(40 + sketch_size)
    x = rng.normal(size=(69, 64)).astype(np.float32) * 3.0
    for meta in (False, True):
        op = _paged(x, "K", hd=64, meta=meta, **fmt)
        dev = torch.device("cuda", 0)
        sk, lo, hi = key_page_summaries(_prod(op), sketch_size, device=dev)
        vm = value_page_means(_prod(op), device=dev)
        sk, lo, hi, vm = sk.cpu().numpy(), lo.cpu().numpy(), hi.cpu().numpy(), vm.cpu().numpy()
        for i, p in enumerate(op):
            want = S.sketch_key_page(p, sketch_size=sketch_size)
            r = want.shape[0]
            np.testing.assert_allclose(sk[i, :r], want, rtol=1e-5, atol=1e-5, err_msg=f"page {i} meta {meta}")
            for extra in range(r, sketch_size):
                np.testing.assert_array_equal(sk[i, extra], sk[i, r - 1])
            wlo, whi = S.envelope_key_page(p)
            np.testing.assert_array_equal(lo[i], wlo)
            np.testing.assert_array_equal(hi[i], whi)
            np.testing.assert_allclose(vm[i], S.summarize_value_page(p), rtol=1e-5, atol=1e-5)


def test_relevance_scores_and_the_tie_rule():
    import torch

    from dotcache_amd.shortlist import relevance_scores, select_top_k

    rng = np.random.default_rng(9)
    n, s, hd = 300, 3, 128
    sk = rng.normal(size=(n, s, hd)).astype(np.float32)
    lo = rng.normal(size=(n, hd)).astype(np.float32) - 1.0
    hi = lo + np.abs(rng.normal(size=(n, hd))).astype(np.float32)
    q = rng.normal(size=hd).astype(np.float32)
    dev = torch.device("cuda", 0)
    t = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    want = {"sketch": np.max(sk @ q, axis=1), "envelope": hi @ np.maximum(q, 0) + lo @ np.minimum(q, 0)}
    cand = rng.random(n) < 0.7
    for mode, w in want.items():
        got = relevance_scores(q, t(sk), t(lo), t(hi), mode)
        np.testing.assert_allclose(got.cpu().numpy(), w, rtol=1e-5, atol=1e-4)
        order = [i for i in sorted(np.flatnonzero(cand).tolist(), key=lambda i: -w[i])]
        k = 17
        assert w[order[k - 1]] - w[order[k]] > 1e-3  # a clear gap, so the set is fixed
        assert np.flatnonzero(select_top_k(got, cand, k)).tolist() == sorted(order[:k])
    # equal scores: the lower indices win, as in Python's stable sort
    eq = torch.full((50,), 2.0, device=dev)
    c = np.ones(50, dtype=bool)
    c[3] = False
    assert np.flatnonzero(select_top_k(eq, c, 5)).tolist() == [0, 1, 2, 4, 5]
    assert not select_top_k(eq, c, 0).any()


@pytest.mark.parametrize("cfg", [
    dict(relevance_top_k=2, relevance_sketch_size=4),
    dict(relevance_top_k=3, relevance_mode="envelope"),
    dict(relevance_top_k=4, exact_refine_top_k=2, relevance_sketch_size=1),
    dict(relevance_top_k=2, approximate_old_pages=True, relevance_sketch_size=4),
    dict(relevance_top_k=2, exact_refine_top_k=1, approximate_old_pages=True, relevance_mode="envelope"),
], ids=["sketch", "envelope", "refine", "fallback", "refine-fallback-envelope"])
@pytest.mark.parametrize("meta", [True, False], ids=["stored", "dense"])
def test_session_decode_with_shortlist_matches_the_oracle(cfg, meta):
    from dotcache_amd.session_runtime import PagedDecodeSession

    rng = np.random.default_rng(sum(map(ord, str(sorted(cfg.items())))) % 1000 + meta)
    hd, n = 64, 64 * 10 + 17
    keys = rng.normal(size=(n, hd)).astype(np.float32)
    keys[130:190, :8] += 4.0  # an old page the query likes
    vals = rng.normal(size=(n, hd)).astype(np.float32)
    kp, vp = _paged(keys, "K", hd=hd, meta=meta), _paged(vals, "V", hd=hd, meta=meta)
    q = rng.normal(size=hd).astype(np.float32)
    q[:8] += 1.0
    ref = S.Session(recent_window_tokens=64, sink_window_tokens=32, **cfg)
    ref.append(kp, vp)
    want_idx, _ = ref.plan(q)
    want = ref.decode(q)
    s = PagedDecodeSession(backend="hip_mi355x", recent_window_tokens=64, sink_window_tokens=32, **cfg)
    s.preload(_prod(kp[:4]), _prod(vp[:4]))
    s.append(_prod(kp[4:]), _prod(vp[4:]))
    got = s.decode(q)
    assert s.last_selected_indices == want_idx
    assert 2 < len(want_idx) < len(kp)
    for a, b, name in zip(got, want, ("logits", "weights", "output")):
        np.testing.assert_allclose(a, b, rtol=1e-4, atol=1e-4, err_msg=name)


def test_encode_page_stores_the_reference_runtime_metadata():
    """``encode_page`` (device encoder) carries the fp16 mean, 4-row chunk
    sketch, min and max of the raw rows, equal to the oracle's numpy
    restatement of reference ``encode.py:64-75``; a 3-token page has 3 rows."""
    from dotcache_amd.config import DotCacheConfig
    from dotcache_amd.encode import encode_page

    rng = np.random.default_rng(19)
    cfg = DotCacheConfig(head_dim=32, group_size=32, bits_k=4, tokens_per_page=64)
    for t in (64, 50, 3):
        x = rng.normal(size=(t, 32)).astype(np.float32)
        page = encode_page(x, cfg, kind="K")
        want = O.runtime_page_metadata(x)
        for name, arr in want.items():
            np.testing.assert_array_equal(getattr(page, name), arr, err_msg=f"{name} T={t}")
        assert page.runtime_page_sketch.shape == (min(4, t), 32)
    bare = encode_page(x, cfg, kind="K", build_runtime_metadata=False)
    assert bare.runtime_page_sketch is None and bare.runtime_page_mean is None


def test_select_top_k_across_tiles_with_ties():
    """Top-k over more than two LDS tiles of the kernel (4096 scores each) and
    a last tile that is not a multiple of 16, with equal scores on both sides
    of the tile boundaries: the selected set is Python's stable
    sorted(..., reverse=True)[:k] over the candidates."""
    import torch

    from dotcache_amd.shortlist import select_top_k

    rng = np.random.default_rng(77)
    n = 2 * 4096 + 37
    s = rng.integers(0, 40, size=n).astype(np.float32)  # many ties everywhere
    for b in (4096, 8192):
        s[b - 3: b + 3] = 17.0  # equal scores straddling each tile boundary
    s[-5:] = 39.0
    cand = rng.random(n) < 0.6
    cand[[4095, 4096, 8191, 8192]] = True
    got_scores = torch.from_numpy(s).cuda()
    for k in (1, 150, 700, int(cand.sum()), int(cand.sum()) + 5):
        order = sorted(np.flatnonzero(cand).tolist(), key=lambda i: s[i], reverse=True)
        want = sorted(order[:k])
        assert np.flatnonzero(select_top_k(got_scores, cand, k)).tolist() == want, k
