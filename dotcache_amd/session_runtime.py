"""Paged decode session for ``hip_mi355x``: reference
``dotcache/session_runtime.py`` (``PagedDecodeSession``, ``:483-723``;
window selection and the execution shortlist, ``:122-480``).

A session holds a sequence's prepared key and value pages (on the device,
through an optional :class:`~dotcache_amd.page_cache.PreparedPageCache`),
grows by whole pages with ``append``, and decodes one query over the pages
its execution rule selects:

* the sink window (the first ``sink_window_tokens`` tokens) and the recent
  window (the last ``recent_window_tokens`` tokens), as whole pages;
* with ``relevance_top_k > 0``, also the ``relevance_top_k`` other pages
  whose summaries score highest against the query ("sketch": max over the
  page's sketch rows of row . q; "envelope": max . max(q, 0) + min . min(q, 0)).
  Summaries are kept on the device and scored and ranked there
  (:mod:`dotcache_amd.shortlist`);
* with ``exact_refine_top_k > 0``, the shortlisted pages are re-ranked by
  their exact maximum logit and only the best ``exact_refine_top_k`` kept;
* with ``approximate_old_pages``, pages left out still contribute: their
  logits are the page's relevance score for every token and their values
  the page mean (the reference's approximate fallback).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable, Sequence

import numpy as np

from . import attention_runtime as rt
from .attention_runtime import BackendName, PageLike
from .page_cache import PreparedPageCache
from .tracing import ExecutionTrace


def select_window_page_indices(key_pages: Sequence[PageLike], *, recent_window_tokens: int | None = None,
                               sink_window_tokens: int = 0) -> list[int]:
    """Indices of the pages that overlap the sink window ``[0, sink)`` or
    the recent window ``[end - recent, end)``, where ``end`` is the largest
    page end (reference ``session_runtime.py:189-216``)."""
    if not key_pages:
        return []
    end = max(p.header.token_start + p.header.token_count for p in key_pages)
    sink = max(0, int(sink_window_tokens))
    recent = int(recent_window_tokens) if recent_window_tokens is not None else 0
    recent_start = max(0, end - recent) if recent > 0 else end
    out = []
    for i, p in enumerate(key_pages):
        start = p.header.token_start
        stop = start + p.header.token_count
        if (sink > 0 and start < sink and stop > 0) or (recent > 0 and stop > recent_start):
            out.append(i)
    return out


def _stack_rows(arrays, n_rows: int | None = None) -> np.ndarray:
    """[n, rows, hd] from per-page [rows_i, hd] arrays; a page with fewer
    rows repeats its last one (which leaves its max over rows unchanged)."""
    mats = [np.atleast_2d(np.asarray(a, dtype=np.float32)) for a in arrays]
    rows = n_rows or max(m.shape[0] for m in mats)
    return np.stack([np.concatenate([m, np.repeat(m[-1:], rows - m.shape[0], axis=0)]) if m.shape[0] < rows else m
                     for m in mats])


def _device():
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("hip_mi355x is unavailable on this machine")
    return torch.device("cuda", torch.cuda.current_device())


def select_execution_page_indices(
    key_pages: Sequence[PageLike], *, recent_window_tokens: int | None = None, sink_window_tokens: int = 0,
    query_slice=None, key_page_sketches=None, key_page_sketch_matrix=None, tail_page_sketch=None,
    key_page_minima=None, key_page_minima_matrix=None, tail_page_minimum=None, key_page_maxima=None,
    key_page_maxima_matrix=None, tail_page_maximum=None, relevance_top_k: int = 0, relevance_mode: str = "sketch",
    stage_recorder: Callable | None = None, score_all_pages_with_matrices: bool = False,
    score_all_pages_min_candidate_fraction: float = 0.0, selector_stats_recorder: Callable | None = None,
) -> list[int]:
    """Reference ``session_runtime.py:219-439``: the window pages plus the
    ``relevance_top_k`` best-scoring other pages, scored and ranked on the
    device; every page when nothing is selected.  Summaries come as
    per-page lists or as matrices over all pages but the tail plus the
    tail's own row, as in the reference."""
    import torch

    from . import shortlist as sl

    if not key_pages:
        return []
    chosen = set(select_window_page_indices(key_pages, recent_window_tokens=recent_window_tokens,
                                            sink_window_tokens=sink_window_tokens))
    if relevance_top_k > 0:
        if query_slice is None:
            raise ValueError("relevance gating requires query_slice")
        n = len(key_pages)
        cand = np.ones(n, dtype=bool)
        cand[list(chosen)] = False
        if cand.any():
            frac = float(cand.sum()) / float(n)
            if selector_stats_recorder is not None:
                selector_stats_recorder({
                    "candidate_pages": int(cand.sum()), "total_pages": int(n), "candidate_fraction": frac,
                    "used_score_all_pages": bool(score_all_pages_with_matrices
                                                 and frac >= max(0.0, float(score_all_pages_min_candidate_fraction))),
                })
            hd = key_pages[0].header.head_dim
            if relevance_mode == "sketch":
                if key_page_sketch_matrix is not None:
                    rows = list(np.asarray(key_page_sketch_matrix, dtype=np.float32))
                    if len(rows) != (n - 1 if tail_page_sketch is not None else n):
                        raise ValueError("key_page_sketch_matrix must align with key_pages")
                    if tail_page_sketch is not None:
                        rows.append(np.asarray(tail_page_sketch, dtype=np.float32))
                else:
                    if key_page_sketches is None:
                        raise ValueError("sketch relevance gating requires key_page_sketches")
                    if len(key_page_sketches) != n:
                        raise ValueError("key_page_sketches must align with key_pages")
                    rows = key_page_sketches
                sk = _stack_rows(rows)
                zeros = np.zeros((n, hd), dtype=np.float32)
                mn = mx = zeros
            elif relevance_mode == "envelope":
                if key_page_minima_matrix is not None and key_page_maxima_matrix is not None:
                    mn_rows = list(np.asarray(key_page_minima_matrix, dtype=np.float32))
                    mx_rows = list(np.asarray(key_page_maxima_matrix, dtype=np.float32))
                    want = n - 1 if tail_page_minimum is not None and tail_page_maximum is not None else n
                    if len(mn_rows) != want or len(mx_rows) != want:
                        raise ValueError("page minima and maxima matrices must align with key_pages")
                    if want == n - 1:
                        mn_rows.append(np.asarray(tail_page_minimum, dtype=np.float32))
                        mx_rows.append(np.asarray(tail_page_maximum, dtype=np.float32))
                else:
                    if key_page_minima is None or key_page_maxima is None:
                        raise ValueError("envelope relevance gating requires page minima and maxima")
                    if len(key_page_minima) != n or len(key_page_maxima) != n:
                        raise ValueError("page minima and maxima must align with key_pages")
                    mn_rows, mx_rows = key_page_minima, key_page_maxima
                mn = np.stack([np.asarray(r, dtype=np.float32) for r in mn_rows])
                mx = np.stack([np.asarray(r, dtype=np.float32) for r in mx_rows])
                sk = np.zeros((n, 1, hd), dtype=np.float32)
            else:
                raise ValueError(f"unsupported relevance_mode: {relevance_mode}")
            dev = _device()
            scores = sl.relevance_scores(query_slice, torch.from_numpy(sk).to(dev), torch.from_numpy(mn).to(dev),
                                         torch.from_numpy(mx).to(dev), relevance_mode)
            chosen.update(np.flatnonzero(sl.select_top_k(scores, cand, relevance_top_k)).tolist())
    if not chosen:
        return list(range(len(key_pages)))
    return sorted(chosen)


def select_execution_page_pairs(key_pages: Sequence[PageLike], value_pages: Sequence[PageLike], *,
                                recent_window_tokens: int | None = None, sink_window_tokens: int = 0,
                                query_slice=None, key_page_sketches=None, key_page_minima=None, key_page_maxima=None,
                                relevance_top_k: int = 0, relevance_mode: str = "sketch") -> tuple[list, list]:
    """Reference ``session_runtime.py:442-480``: the selected key and value
    pages; every page when no window or shortlist is set."""
    if len(key_pages) != len(value_pages):
        raise ValueError("key_pages and value_pages must contain the same number of pages")
    if not key_pages:
        return [], []
    if (recent_window_tokens is None or recent_window_tokens <= 0) and sink_window_tokens <= 0 and relevance_top_k <= 0:
        return list(key_pages), list(value_pages)
    idx = select_execution_page_indices(
        key_pages, recent_window_tokens=recent_window_tokens, sink_window_tokens=sink_window_tokens,
        query_slice=query_slice, key_page_sketches=key_page_sketches, key_page_minima=key_page_minima,
        key_page_maxima=key_page_maxima, relevance_top_k=relevance_top_k, relevance_mode=relevance_mode)
    return [key_pages[i] for i in idx], [value_pages[i] for i in idx]


@dataclass(slots=True)
class PagedDecodeSession:
    """Reference ``PagedDecodeSession`` (``session_runtime.py:483-723``).
    Page summaries (``key_page_sketches [P, S, hd]``, ``key_page_minima`` /
    ``key_page_maxima [P, hd]``, ``value_page_summaries [P, hd]``) are
    device tensors, built at ``append`` when a shortlist or the approximate
    fallback needs them."""

    backend: BackendName = "auto"
    cache: PreparedPageCache | None = None
    recent_window_tokens: int | None = None
    sink_window_tokens: int = 0
    relevance_top_k: int = 0
    relevance_sketch_size: int = 1
    relevance_mode: str = "sketch"
    exact_refine_top_k: int = 0
    approximate_old_pages: bool = False
    key_pages: list = field(default_factory=list)
    value_pages: list = field(default_factory=list)
    key_page_sketches: object = None
    key_page_minima: object = None
    key_page_maxima: object = None
    value_page_summaries: object = None
    last_selected_indices: list = field(default_factory=list)

    def __post_init__(self) -> None:
        if self.relevance_mode not in ("sketch", "envelope"):
            raise ValueError(f"unsupported relevance_mode: {self.relevance_mode}")
        if int(self.relevance_sketch_size) <= 0:
            raise ValueError("sketch_size must be positive")

    @property
    def _needs_summaries(self) -> bool:
        return self.relevance_top_k > 0 or self.approximate_old_pages

    def clear(self) -> None:
        self.key_pages.clear()
        self.value_pages.clear()
        self.key_page_sketches = self.key_page_minima = self.key_page_maxima = self.value_page_summaries = None
        self.last_selected_indices.clear()
        if self.cache is not None:
            self.cache.clear()

    @property
    def page_count(self) -> int:
        return len(self.key_pages)

    @property
    def active_page_count(self) -> int:
        return len(self.execution_indices())

    @property
    def active_token_count(self) -> int:
        return sum(self.key_pages[i].header.token_count for i in self.execution_indices())

    def preload(self, key_pages: Sequence[PageLike], value_pages: Sequence[PageLike], *, prepare: bool = True,
                trace: ExecutionTrace | None = None) -> None:
        self.clear()
        self.append(key_pages, value_pages, prepare=prepare, trace=trace)

    def append(self, key_pages: Sequence[PageLike], value_pages: Sequence[PageLike], *, prepare: bool = True,
               trace: ExecutionTrace | None = None) -> None:
        """Add whole pages; with ``prepare`` they go to the device now, so
        ``decode`` moves no page bytes."""
        import torch

        from . import shortlist as sl

        if len(key_pages) != len(value_pages):
            raise ValueError("key_pages and value_pages must contain the same number of pages")
        if prepare and key_pages:
            key_pages = rt.prepare_pages(key_pages, backend=self.backend, cache=self.cache, trace=trace)
            value_pages = rt.prepare_pages(value_pages, backend=self.backend, cache=self.cache, trace=trace)
        if key_pages and self._needs_summaries:
            dev = _device()
            sk, lo, hi = sl.key_page_summaries(key_pages, int(self.relevance_sketch_size), device=dev, trace=trace)
            vm = sl.value_page_means(value_pages, device=dev, trace=trace)
            cat = lambda old, new: new if old is None else torch.cat([old, new])  # noqa: E731
            self.key_page_sketches = cat(self.key_page_sketches, sk)
            self.key_page_minima = cat(self.key_page_minima, lo)
            self.key_page_maxima = cat(self.key_page_maxima, hi)
            self.value_page_summaries = cat(self.value_page_summaries, vm)
        self.key_pages.extend(key_pages)
        self.value_pages.extend(value_pages)

    def _window(self) -> list[int]:
        return select_window_page_indices(self.key_pages, recent_window_tokens=self.recent_window_tokens,
                                          sink_window_tokens=self.sink_window_tokens)

    def _relevance(self, query_slice):
        from . import shortlist as sl

        return sl.relevance_scores(query_slice, self.key_page_sketches, self.key_page_minima, self.key_page_maxima,
                                   self.relevance_mode)

    def _stage1(self, query_slice) -> list[int]:
        from . import shortlist as sl

        if not self.key_pages:
            return []
        chosen = set(self._window())
        if self.relevance_top_k > 0:
            if query_slice is None:
                raise ValueError("relevance gating requires query_slice")
            cand = np.ones(len(self.key_pages), dtype=bool)
            cand[list(chosen)] = False
            if cand.any():
                sel = sl.select_top_k(self._relevance(query_slice), cand, self.relevance_top_k)
                chosen.update(np.flatnonzero(sel).tolist())
        return sorted(chosen) if chosen else list(range(len(self.key_pages)))

    def _execution_plan(self, query_slice=None, *, trace: ExecutionTrace | None = None):
        """Reference ``_execution_plan`` (``:588-648``): the selected indices
        and the exact logits of pages kept by the refine step."""
        stage1 = self._stage1(query_slice)
        if query_slice is None or self.exact_refine_top_k <= 0 or self.relevance_top_k <= 0 or not stage1:
            return stage1, {}
        base = set(self._window())
        cand = [i for i in stage1 if i not in base]
        if not cand or self.exact_refine_top_k >= len(cand):
            return stage1, {}
        logits = rt.score_pages(query_slice, [self.key_pages[i] for i in cand], backend=self.backend, trace=trace)
        ranked = sorted(((float(np.max(lg)), i) for lg, i in zip(logits, cand)), key=lambda it: it[0], reverse=True)
        chosen = [i for _, i in ranked[: self.exact_refine_top_k]]
        keep = set(chosen)
        refined = {i: np.asarray(lg, dtype=np.float32) for lg, i in zip(logits, cand) if i in keep}
        return sorted(base.union(chosen)), refined

    def execution_indices(self, query_slice=None, *, trace: ExecutionTrace | None = None) -> list[int]:
        return self._execution_plan(query_slice, trace=trace)[0]

    def execution_pages(self, query_slice=None) -> tuple[list[PageLike], list[PageLike]]:
        idx = self._stage1(query_slice)
        return [self.key_pages[i] for i in idx], [self.value_pages[i] for i in idx]

    def decode(self, query_slice, *, trace: ExecutionTrace | None = None) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        """(logits, weights, output) (reference ``session_runtime.py:650-672``)."""
        if not self.key_pages or not self.value_pages:
            raise ValueError("PagedDecodeSession requires preloaded pages before decode")
        idx, refined = self._execution_plan(query_slice, trace=trace)
        self.last_selected_indices = list(idx)
        if not self.approximate_old_pages or len(idx) == len(self.key_pages):
            return rt.decode_step_with_page_logits(query_slice, [self.key_pages[i] for i in idx],
                                                   [self.value_pages[i] for i in idx],
                                                   page_logits=[refined.get(i) for i in idx], backend=self.backend,
                                                   trace=trace)
        return self._decode_with_old_page_fallback(query_slice, idx, trace=trace)

    def _decode_with_old_page_fallback(self, query_slice, selected: Sequence[int], *,
                                       trace: ExecutionTrace | None = None):
        """Reference ``session_runtime.py:674-723``: exact logits and mix for
        the selected pages; for the others every token's logit is the page's
        relevance score and its value the page mean."""
        q = np.asarray(query_slice, dtype=np.float32)
        exact = set(selected)
        rel = self._relevance(q).cpu().numpy()
        means = self.value_page_summaries.cpu().numpy()
        ex = sorted(exact)
        ex_logits = dict(zip(ex, rt.score_pages(q, [self.key_pages[i] for i in ex], backend=self.backend, trace=trace)))
        all_logits, mx = [], -np.inf
        for i, p in enumerate(self.key_pages):
            lg = (np.asarray(ex_logits[i], dtype=np.float32) if i in exact
                  else np.full(p.header.token_count, rel[i], dtype=np.float32))
            all_logits.append(lg)
            if lg.size:
                mx = max(mx, float(np.max(lg)))
        if not np.isfinite(mx):
            raise ValueError("failed to compute logits for session decode")
        out = np.zeros(self.value_pages[0].header.head_dim, dtype=np.float32)
        weights, denom = [], 0.0
        for i, p in enumerate(self.key_pages):
            w = np.exp(all_logits[i] - mx).astype(np.float32)
            weights.append(w)
            denom += float(np.sum(w))
            if i in exact:
                out = rt.mix_page(w, self.value_pages[i], out_acc=out, backend=self.backend, trace=trace)
            else:
                out += float(np.sum(w)) * means[i]
        if denom <= 0.0:
            raise ValueError("invalid normalization denominator in session fallback decode")
        return (np.concatenate(all_logits).astype(np.float32),
                np.concatenate(weights).astype(np.float32) / np.float32(denom), out / np.float32(denom))
