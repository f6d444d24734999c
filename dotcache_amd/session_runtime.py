"""Paged decode session for ``hip_mi355x``: the exact-attention part of
reference ``dotcache/session_runtime.py`` (``PagedDecodeSession``,
``:483-723``; window selection, ``:192-216``, ``:442-480``).

A session holds a sequence's prepared key and value pages (on the device,
through an optional :class:`~dotcache_amd.page_cache.PreparedPageCache`),
grows by whole pages with ``append``, and decodes one query over the pages
the execution rule selects: all of them, or the pages that overlap the
sink window (the first ``sink_window_tokens`` tokens) or the recent window
(the last ``recent_window_tokens`` tokens).  Selection only picks whole
pages, so a windowed decode is exact attention over those pages.

The relevance shortlist of the reference (page sketches and envelopes,
``relevance_top_k``, ``exact_refine_top_k``, ``approximate_old_pages``) is
approximate attention and is not served: a session asked for it raises
ValueError at construction.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Sequence

import numpy as np

from . import attention_runtime as rt
from .attention_runtime import BackendName, PageLike
from .page_cache import PreparedPageCache
from .tracing import ExecutionTrace


def select_window_page_indices(key_pages: Sequence[PageLike], *, recent_window_tokens: int | None = None,
                               sink_window_tokens: int = 0) -> list[int]:
    """Indices of the pages that overlap the sink window ``[0, sink)`` or
    the recent window ``[end - recent, end)``, where ``end`` is the largest
    page end (reference ``session_runtime.py:192-216``)."""
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


def _check_no_shortlist(relevance_top_k: int) -> None:
    if int(relevance_top_k) > 0:
        raise ValueError("relevance shortlists are approximate attention and are not served by hip_mi355x")


def select_execution_page_indices(key_pages: Sequence[PageLike], *, recent_window_tokens: int | None = None,
                                  sink_window_tokens: int = 0, relevance_top_k: int = 0, **_shortlist) -> list[int]:
    """The window pages, or every page when no window selects any
    (reference ``session_runtime.py:219-439`` without the shortlist)."""
    _check_no_shortlist(relevance_top_k)
    if not key_pages:
        return []
    chosen = select_window_page_indices(key_pages, recent_window_tokens=recent_window_tokens,
                                        sink_window_tokens=sink_window_tokens)
    return chosen if chosen else list(range(len(key_pages)))


def select_execution_page_pairs(key_pages: Sequence[PageLike], value_pages: Sequence[PageLike], *,
                                recent_window_tokens: int | None = None, sink_window_tokens: int = 0,
                                relevance_top_k: int = 0, **_shortlist) -> tuple[list[PageLike], list[PageLike]]:
    """Reference ``session_runtime.py:442-480``: the selected key and value
    pages; every page when no window is set."""
    if len(key_pages) != len(value_pages):
        raise ValueError("key_pages and value_pages must contain the same number of pages")
    _check_no_shortlist(relevance_top_k)
    if not key_pages:
        return [], []
    if (recent_window_tokens is None or recent_window_tokens <= 0) and sink_window_tokens <= 0:
        return list(key_pages), list(value_pages)
    idx = select_execution_page_indices(key_pages, recent_window_tokens=recent_window_tokens,
                                        sink_window_tokens=sink_window_tokens)
    return [key_pages[i] for i in idx], [value_pages[i] for i in idx]


@dataclass(slots=True)
class PagedDecodeSession:
    """Reference ``PagedDecodeSession`` (``session_runtime.py:483-723``):
    preload / append / decode over prepared pages, exact attention only."""

    backend: BackendName = "auto"
    cache: PreparedPageCache | None = None
    recent_window_tokens: int | None = None
    sink_window_tokens: int = 0
    relevance_top_k: int = 0
    relevance_sketch_size: int = 1  # accepted for the reference's signature; used only by the shortlist
    relevance_mode: str = "sketch"  # likewise
    exact_refine_top_k: int = 0
    approximate_old_pages: bool = False
    key_pages: list = field(default_factory=list)
    value_pages: list = field(default_factory=list)
    last_selected_indices: list = field(default_factory=list)

    def __post_init__(self) -> None:
        _check_no_shortlist(self.relevance_top_k)
        if int(self.exact_refine_top_k) > 0 or self.approximate_old_pages:
            raise ValueError("exact refine and approximate old pages belong to the relevance shortlist, "
                             "which hip_mi355x does not serve")

    def clear(self) -> None:
        self.key_pages.clear()
        self.value_pages.clear()
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
        if len(key_pages) != len(value_pages):
            raise ValueError("key_pages and value_pages must contain the same number of pages")
        if prepare and key_pages:
            key_pages = rt.prepare_pages(key_pages, backend=self.backend, cache=self.cache, trace=trace)
            value_pages = rt.prepare_pages(value_pages, backend=self.backend, cache=self.cache, trace=trace)
        self.key_pages.extend(key_pages)
        self.value_pages.extend(value_pages)

    def execution_indices(self, query_slice=None, *, trace: ExecutionTrace | None = None) -> list[int]:
        if (self.recent_window_tokens is None or self.recent_window_tokens <= 0) and self.sink_window_tokens <= 0:
            return list(range(len(self.key_pages)))
        return select_execution_page_indices(self.key_pages, recent_window_tokens=self.recent_window_tokens,
                                             sink_window_tokens=self.sink_window_tokens)

    def execution_pages(self, query_slice=None) -> tuple[list[PageLike], list[PageLike]]:
        idx = self.execution_indices(query_slice)
        return [self.key_pages[i] for i in idx], [self.value_pages[i] for i in idx]

    def decode(self, query_slice, *, trace: ExecutionTrace | None = None) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        """(logits, weights, output) over the selected pages (reference
        ``session_runtime.py:643-666``)."""
        if not self.key_pages or not self.value_pages:
            raise ValueError("PagedDecodeSession requires preloaded pages before decode")
        idx = self.execution_indices(query_slice, trace=trace)
        self.last_selected_indices = list(idx)
        return rt.decode_step_with_page_logits(query_slice, [self.key_pages[i] for i in idx],
                                               [self.value_pages[i] for i in idx], backend=self.backend, trace=trace)
