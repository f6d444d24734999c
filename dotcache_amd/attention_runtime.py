"""Backend dispatch: the generic entry points of reference
``dotcache/attention_runtime.py:35-315`` for the ``hip_mi355x`` backend.

``BackendName`` here is ``"hip_mi355x"`` or ``"auto"``.  ``auto`` resolves
to ``hip_mi355x`` when a GPU and the library are present and otherwise raises
RuntimeError: this package ships no CPU path (the reference keeps its own
``cpu_ref``, and its ``_resolve_backend`` gains a ``hip_mi355x`` branch next
to it).  Errors follow the
reference: RuntimeError for an unavailable device, ValueError for an
unsupported page or bad shapes.
"""
from __future__ import annotations

from typing import Literal, Sequence

import numpy as np

from .backends import hip_mi355x as hip
from .backends.hip_mi355x import PreparedPageHIP
from .page_cache import PreparedPageCache
from .tracing import ExecutionTrace
from .types import EncodedPage

BackendName = Literal["hip_mi355x", "auto"]
PageLike = EncodedPage | PreparedPageHIP


def _resolve_backend(backend: BackendName, page: PageLike) -> Literal["hip_mi355x"]:
    """Reference ``attention_runtime.py:39-60`` for this backend."""
    if backend not in ("hip_mi355x", "auto"):
        raise ValueError(f"unknown backend {backend!r} (this package serves hip_mi355x)")
    if not hip.hip_available():
        raise RuntimeError("hip_mi355x is unavailable on this machine")
    if not hip.page_supported_hip(page):
        raise ValueError("page is unsupported by hip_mi355x in this phase")
    return "hip_mi355x"


def prepare_page(page: PageLike, *, backend: BackendName = "auto", cache: PreparedPageCache | None = None,
                 trace: ExecutionTrace | None = None) -> PreparedPageHIP:
    """Reference ``attention_runtime.py:72-87``: through ``cache`` when given."""
    _resolve_backend(backend, page)
    if cache is not None:
        return cache.prepare_page(page, backend="hip_mi355x", trace=trace)
    return hip.prepare_page_hip(page, trace=trace)


def prepare_pages(pages: Sequence[PageLike], *, backend: BackendName = "auto",
                  cache: PreparedPageCache | None = None, trace: ExecutionTrace | None = None) -> list[PreparedPageHIP]:
    """Reference ``attention_runtime.py:90-108``."""
    for p in pages:
        _resolve_backend(backend, p)
    if cache is not None:
        return cache.prepare_pages(list(pages), backend="hip_mi355x", trace=trace)
    return hip.prepare_pages_hip(pages, trace=trace)


def _cached(pages, backend, cache, trace):
    """Pages through ``cache`` when one is given, else unchanged (the
    backend prepares them per call)."""
    return list(pages) if cache is None else prepare_pages(pages, backend=backend, cache=cache, trace=trace)


def score_page(query_slice, page: PageLike, *, backend: BackendName = "auto", trace: ExecutionTrace | None = None) -> np.ndarray:
    _resolve_backend(backend, page)
    return hip.score_page_hip(query_slice, page, trace=trace)


def score_pages(query_slice, pages: Sequence[PageLike], *, backend: BackendName = "auto",
                cache: PreparedPageCache | None = None, trace: ExecutionTrace | None = None) -> list[np.ndarray]:
    if not pages:
        return []
    for p in pages:
        _resolve_backend(backend, p)
    return hip.score_pages_hip(query_slice, _cached(pages, backend, cache, trace), trace=trace)


def mix_page(attn_weights, page: PageLike, *, out_acc: np.ndarray | None = None, backend: BackendName = "auto",
             trace: ExecutionTrace | None = None) -> np.ndarray:
    _resolve_backend(backend, page)
    return hip.mix_page_hip(attn_weights, page, out_acc=out_acc, trace=trace)


def attention_step(query_slice, key_page: PageLike, value_page: PageLike, *, backend: BackendName = "auto",
                   cache: PreparedPageCache | None = None, trace: ExecutionTrace | None = None):
    """Reference ``attention_runtime.py:162-176``."""
    return decode_step(query_slice, [key_page], [value_page], backend=backend, cache=cache, trace=trace)


def decode_step(query_slice, key_pages: Sequence[PageLike], value_pages: Sequence[PageLike], *,
                backend: BackendName = "auto", cache: PreparedPageCache | None = None,
                trace: ExecutionTrace | None = None):
    """Reference ``attention_runtime.py:179-200``."""
    if len(key_pages) != len(value_pages):
        raise ValueError("key_pages and value_pages must contain the same number of pages")
    if not key_pages:
        raise ValueError("decode_step requires at least one page")
    return decode_step_with_page_logits(query_slice, key_pages, value_pages, backend=backend, cache=cache,
                                        trace=trace)


def decode_multi_query_step(query_slices, key_pages: Sequence[PageLike], value_pages: Sequence[PageLike], *,
                            backend: BackendName = "auto", cache: PreparedPageCache | None = None,
                            trace: ExecutionTrace | None = None):
    """Reference ``attention_runtime.py:203-257``."""
    queries = np.asarray(query_slices, dtype=np.float32)
    if queries.ndim != 2:
        raise ValueError("query_slices must have shape [query_count, head_dim]")
    if len(key_pages) != len(value_pages):
        raise ValueError("key_pages and value_pages must contain the same number of pages")
    if not key_pages:
        raise ValueError("decode_multi_query_step requires at least one page")
    for p in list(key_pages) + list(value_pages):
        _resolve_backend(backend, p)
    return hip.decode_multi_query_step_hip(queries, _cached(key_pages, backend, cache, trace),
                                           _cached(value_pages, backend, cache, trace), trace=trace)


def decode_step_with_page_logits(query_slice, key_pages: Sequence[PageLike], value_pages: Sequence[PageLike], *,
                                 page_logits=None, backend: BackendName = "auto",
                                 cache: PreparedPageCache | None = None, trace: ExecutionTrace | None = None):
    """Reference ``attention_runtime.py:260-315``: (logits, weights, output)."""
    if len(key_pages) != len(value_pages):
        raise ValueError("key_pages and value_pages must contain the same number of pages")
    if not key_pages:
        raise ValueError("decode_step requires at least one page")
    if page_logits is not None and len(page_logits) != len(key_pages):
        raise ValueError("page_logits must align with key_pages")
    for p in list(key_pages) + list(value_pages):
        _resolve_backend(backend, p)
    return hip.decode_step_hip(query_slice, _cached(key_pages, backend, cache, trace),
                               _cached(value_pages, backend, cache, trace), precomputed_page_logits=page_logits,
                               trace=trace)
