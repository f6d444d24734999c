"""CPU oracle of the execution shortlist -- TEST INFRASTRUCTURE ONLY.

Nothing in the product package may import this module; it is the checker of
``tests/``.  It restates, in numpy, reference ``dotcache/session_runtime.py``:

  * page summaries        ``sketch_key_page`` / ``summarize_value_page`` /
                          ``envelope_key_page`` (``:122-162``)
  * page relevance        ``score_page_relevance`` (``:165-186``)
  * window + shortlist    ``select_window_page_indices``,
                          ``select_execution_page_indices`` (``:189-439``,
                          the list-of-summaries form)
  * session plan / decode ``PagedDecodeSession._execution_plan``, ``decode``
                          and ``_decode_with_old_page_fallback`` (``:588-723``)

Pinned in ``tests/test_shortlist_oracle.py`` by the reference's known-answer
tests (``tests/test_torch_mps_backend.py:65-200``, ``:710-855``) restated,
and by closed forms: a one-row sketch is the mean of the dense rows, the
envelope is their min / max, the shortlist equals a brute-force choice of
the k best candidates, and a session whose shortlist admits every page
decodes exactly like ``decode_step``.
"""
from __future__ import annotations

import numpy as np

from . import dotcache_oracle as O


def sketch_key_page(page, *, sketch_size: int = 1) -> np.ndarray:
    """Reference ``session_runtime.py:122-137``."""
    if sketch_size <= 0:
        raise ValueError("sketch_size must be positive")
    if page.runtime_page_sketch is not None:
        stored = np.asarray(page.runtime_page_sketch, dtype=np.float32)
        if sketch_size == 1 and page.runtime_page_mean is not None:
            return np.asarray(page.runtime_page_mean, dtype=np.float32)[None, :]
        if stored.shape[0] == sketch_size:
            return stored
        if stored.shape[0] > sketch_size and sketch_size > 1:
            chunks = np.array_split(stored, sketch_size, axis=0)
            return np.stack([c.mean(axis=0) for c in chunks], axis=0).astype(np.float32)
    dense = O.decode_page(page)
    if sketch_size == 1:
        return dense.mean(axis=0, keepdims=True)
    chunks = np.array_split(dense, min(sketch_size, dense.shape[0]), axis=0)
    return np.stack([c.mean(axis=0) for c in chunks], axis=0).astype(np.float32)


def summarize_value_page(page) -> np.ndarray:
    """Reference ``session_runtime.py:144-148``."""
    if page.runtime_page_mean is not None:
        return np.asarray(page.runtime_page_mean, dtype=np.float32)
    return O.decode_page(page).mean(axis=0)


def envelope_key_page(page) -> tuple[np.ndarray, np.ndarray]:
    """Reference ``session_runtime.py:151-162``."""
    if page.runtime_page_min is not None and page.runtime_page_max is not None:
        return np.asarray(page.runtime_page_min, np.float32), np.asarray(page.runtime_page_max, np.float32)
    dense = O.decode_page(page)
    return dense.min(axis=0).astype(np.float32), dense.max(axis=0).astype(np.float32)


def score_page_relevance(query, *, relevance_mode, page_sketch=None, page_min=None, page_max=None) -> float:
    """Reference ``session_runtime.py:165-186``."""
    q = np.asarray(query, dtype=np.float32)
    if relevance_mode == "sketch":
        return float(np.max(np.asarray(page_sketch, dtype=np.float32) @ q))
    if relevance_mode == "envelope":
        return float(np.asarray(page_max, np.float32) @ np.maximum(q, 0.0)
                     + np.asarray(page_min, np.float32) @ np.minimum(q, 0.0))
    raise ValueError(f"unsupported relevance_mode: {relevance_mode}")


def select_window_page_indices(key_pages, *, recent_window_tokens=None, sink_window_tokens=0) -> list[int]:
    """Reference ``session_runtime.py:189-216``."""
    if not key_pages:
        return []
    end = max(p.header.token_start + p.header.token_count for p in key_pages)
    sink = max(0, sink_window_tokens)
    recent_start = end
    if recent_window_tokens is not None and recent_window_tokens > 0:
        recent_start = max(0, end - recent_window_tokens)
    out = set()
    for i, p in enumerate(key_pages):
        s, e = p.header.token_start, p.header.token_start + p.header.token_count
        if (sink > 0 and s < sink and e > 0) or (recent_window_tokens and recent_window_tokens > 0 and e > recent_start):
            out.add(i)
    return sorted(out)


def select_execution_page_indices(key_pages, *, recent_window_tokens=None, sink_window_tokens=0, query_slice=None,
                                  key_page_sketches=None, key_page_minima=None, key_page_maxima=None,
                                  relevance_top_k=0, relevance_mode="sketch") -> list[int]:
    """Reference ``session_runtime.py:219-439`` (list-of-summaries form)."""
    if not key_pages:
        return []
    chosen = set(select_window_page_indices(key_pages, recent_window_tokens=recent_window_tokens,
                                            sink_window_tokens=sink_window_tokens))
    if relevance_top_k > 0:
        if query_slice is None:
            raise ValueError("relevance gating requires query_slice")
        cand = [i for i in range(len(key_pages)) if i not in chosen]
        if cand:
            q = np.asarray(query_slice, dtype=np.float32)
            if relevance_mode == "sketch":
                sk = np.stack([np.asarray(key_page_sketches[i], dtype=np.float32) for i in cand], axis=0)
                scores = np.max(sk @ q, axis=1).astype(np.float32)
            elif relevance_mode == "envelope":
                mn = np.stack([np.asarray(key_page_minima[i], dtype=np.float32) for i in cand], axis=0)
                mx = np.stack([np.asarray(key_page_maxima[i], dtype=np.float32) for i in cand], axis=0)
                scores = (mx @ np.maximum(q, 0.0) + mn @ np.minimum(q, 0.0)).astype(np.float32)
            else:
                raise ValueError(f"unsupported relevance_mode: {relevance_mode}")
            ranked = [i for _, i in sorted(zip(scores.tolist(), cand), key=lambda it: it[0], reverse=True)]
            chosen.update(ranked[:relevance_top_k])
    if not chosen:
        return list(range(len(key_pages)))
    return sorted(chosen)


class Session:
    """Reference ``PagedDecodeSession`` (``session_runtime.py:483-723``) on
    oracle pages: summaries at append, shortlist, exact refine, and the
    approximate fallback for pages left out."""

    def __init__(self, *, recent_window_tokens=None, sink_window_tokens=0, relevance_top_k=0,
                 relevance_sketch_size=1, relevance_mode="sketch", exact_refine_top_k=0, approximate_old_pages=False):
        self.recent_window_tokens = recent_window_tokens
        self.sink_window_tokens = sink_window_tokens
        self.relevance_top_k = relevance_top_k
        self.relevance_sketch_size = relevance_sketch_size
        self.relevance_mode = relevance_mode
        self.exact_refine_top_k = exact_refine_top_k
        self.approximate_old_pages = approximate_old_pages
        self.key_pages, self.value_pages = [], []
        self.sketches, self.minima, self.maxima, self.value_means = [], [], [], []

    def append(self, key_pages, value_pages):
        self.key_pages += list(key_pages)
        self.value_pages += list(value_pages)
        for p in key_pages:
            self.sketches.append(sketch_key_page(p, sketch_size=self.relevance_sketch_size))
            lo, hi = envelope_key_page(p)
            self.minima.append(lo)
            self.maxima.append(hi)
        self.value_means += [summarize_value_page(p) for p in value_pages]

    def plan(self, query):
        """Reference ``_execution_plan`` (``:588-648``): (indices, exact logits of refined pages)."""
        stage1 = select_execution_page_indices(
            self.key_pages, recent_window_tokens=self.recent_window_tokens, sink_window_tokens=self.sink_window_tokens,
            query_slice=query, key_page_sketches=self.sketches, key_page_minima=self.minima,
            key_page_maxima=self.maxima, relevance_top_k=self.relevance_top_k, relevance_mode=self.relevance_mode)
        if query is None or self.exact_refine_top_k <= 0 or self.relevance_top_k <= 0 or not stage1:
            return stage1, {}
        base = set(select_window_page_indices(self.key_pages, recent_window_tokens=self.recent_window_tokens,
                                              sink_window_tokens=self.sink_window_tokens))
        cand = [i for i in stage1 if i not in base]
        if not cand or self.exact_refine_top_k >= len(cand):
            return stage1, {}
        logits = {i: O.score_page_ref(query, self.key_pages[i]) for i in cand}
        exact = sorted(((float(np.max(logits[i])), i) for i in cand), key=lambda it: it[0], reverse=True)
        chosen = [i for _, i in exact[: self.exact_refine_top_k]]
        return sorted(base.union(chosen)), {i: logits[i] for i in chosen}

    def decode(self, query):
        """Reference ``decode`` and ``_decode_with_old_page_fallback`` (``:650-723``)."""
        idx, refined = self.plan(query)
        if not self.approximate_old_pages or len(idx) == len(self.key_pages):
            return O.decode_step(query, [self.key_pages[i] for i in idx], [self.value_pages[i] for i in idx],
                                 page_logits=[refined.get(i) for i in idx])
        q = np.asarray(query, dtype=np.float32)
        exact = set(idx)
        all_logits, mx = [], -np.inf
        for i, p in enumerate(self.key_pages):
            if i in exact:
                lg = O.score_page_ref(q, p).astype(np.float32)
            else:
                s = score_page_relevance(q, relevance_mode=self.relevance_mode, page_sketch=self.sketches[i],
                                         page_min=self.minima[i], page_max=self.maxima[i])
                lg = np.full(p.header.token_count, s, dtype=np.float32)
            all_logits.append(lg)
            mx = max(mx, float(np.max(lg)))
        out = np.zeros(self.value_pages[0].header.head_dim, dtype=np.float32)
        weights, denom = [], 0.0
        for i, p in enumerate(self.key_pages):
            w = np.exp(all_logits[i] - mx).astype(np.float32)
            weights.append(w)
            denom += float(np.sum(w))
            if i in exact:
                out = O.mix_page_ref(w, self.value_pages[i], out_acc=out)
            else:
                out += float(np.sum(w)) * self.value_means[i]
        return (np.concatenate(all_logits), np.concatenate(weights) / np.float32(denom), out / np.float32(denom))
