"""Execution shortlist on the device: page summaries, page relevance and a
stable top-k (reference ``dotcache/session_runtime.py:122-439``).

Summaries follow the reference's rules for where they come from: the fp16
runtime metadata an encoder stored with the page when it is there
(``runtime_page_mean`` / ``_sketch`` / ``_min`` / ``_max``), otherwise the
page's dequantised rows, reduced on the device by ``dc_page_summaries``
(the reference decodes the page densely on the host for that).  Relevance
(``dc_page_relevance``) and the top-k (``dc_select_top_k``) run on the
device; only the chosen page mask comes back to the host.
"""
from __future__ import annotations

import ctypes as C
from typing import Sequence

import numpy as np

from . import _lib
from .backends.hip_mi355x import PreparedPageHIP, prepare_pages_hip
from .page_pool import current_stream_ptr

MODES = {"sketch": 0, "envelope": 1}


def _torch():
    import torch

    return torch


def _source(page):
    return page.source_page if isinstance(page, PreparedPageHIP) else page


def stored_sketch(page, sketch_size: int) -> np.ndarray | None:
    """The sketch a page's stored metadata gives for ``sketch_size`` rows, or
    None when the dense rows are needed (reference ``session_runtime.py:122-131``)."""
    src = _source(page)
    if src.runtime_page_sketch is None:
        return None
    stored = np.asarray(src.runtime_page_sketch, dtype=np.float32)
    if sketch_size == 1 and src.runtime_page_mean is not None:
        return np.asarray(src.runtime_page_mean, dtype=np.float32)[None, :]
    if stored.shape[0] == sketch_size:
        return stored
    if stored.shape[0] > sketch_size > 1:
        return np.stack([c.mean(axis=0) for c in np.array_split(stored, sketch_size, axis=0)]).astype(np.float32)
    return None


def _dense_summaries(pages: Sequence, sketch_size: int, trace=None):
    """(mean [n, hd], sketch [n, S, hd], min, max) of the pages' dequantised
    rows, on the device, one ``dc_page_summaries`` launch per pool."""
    torch = _torch()
    prepared = prepare_pages_hip(list(pages), trace=trace)
    hd = prepared[0].header.head_dim
    dev = prepared[0].pool.device
    n = len(prepared)
    mean = torch.empty((n, hd), dtype=torch.float32, device=dev)
    sketch = torch.empty((n, sketch_size, hd), dtype=torch.float32, device=dev)
    lo = torch.empty((n, hd), dtype=torch.float32, device=dev)
    hi = torch.empty((n, hd), dtype=torch.float32, device=dev)
    by_pool: dict[int, list[int]] = {}
    for i, p in enumerate(prepared):
        by_pool.setdefault(id(p.pool), []).append(i)
    for idx in by_pool.values():
        pool = prepared[idx[0]].pool
        ids = torch.tensor([prepared[i].page_id for i in idx], dtype=torch.int32, device=dev)
        m = torch.empty((len(idx), hd), dtype=torch.float32, device=dev)
        s = torch.empty((len(idx), sketch_size, hd), dtype=torch.float32, device=dev)
        a = torch.empty((len(idx), hd), dtype=torch.float32, device=dev)
        b = torch.empty((len(idx), hd), dtype=torch.float32, device=dev)
        st = _lib.lib().dc_page_summaries(pool.c_pool(), C.c_void_p(ids.data_ptr()), len(idx), int(sketch_size),
                                          C.c_void_p(m.data_ptr()), C.c_void_p(s.data_ptr()), C.c_void_p(a.data_ptr()),
                                          C.c_void_p(b.data_ptr()), C.c_void_p(current_stream_ptr()))
        _lib.check(st, "dc_page_summaries")
        sel = torch.tensor(idx, dtype=torch.int64, device=dev)
        mean[sel], sketch[sel], lo[sel], hi[sel] = m, s, a, b
    return mean, sketch, lo, hi


def key_page_summaries(pages: Sequence, sketch_size: int, *, device, trace=None):
    """Device ``(sketch [n, S, hd], minima [n, hd], maxima [n, hd])`` of key
    pages (reference ``sketch_key_page`` / ``envelope_key_page``)."""
    torch = _torch()
    if sketch_size <= 0:
        raise ValueError("sketch_size must be positive")
    hd = _source(pages[0]).header.head_dim
    n = len(pages)
    sketch = torch.empty((n, sketch_size, hd), dtype=torch.float32, device=device)
    lo = torch.empty((n, hd), dtype=torch.float32, device=device)
    hi = torch.empty((n, hd), dtype=torch.float32, device=device)
    dense_idx = []
    for i, p in enumerate(pages):
        src = _source(p)
        sk = stored_sketch(p, sketch_size)
        has_env = src.runtime_page_min is not None and src.runtime_page_max is not None
        if sk is None or not has_env:
            dense_idx.append(i)
        if sk is not None:
            sketch[i] = torch.from_numpy(sk).to(device)
        if has_env:
            lo[i] = torch.from_numpy(np.asarray(src.runtime_page_min, np.float32)).to(device)
            hi[i] = torch.from_numpy(np.asarray(src.runtime_page_max, np.float32)).to(device)
    if dense_idx:
        _, dsk, dlo, dhi = _dense_summaries([pages[i] for i in dense_idx], sketch_size, trace)
        for j, i in enumerate(dense_idx):
            src = _source(pages[i])
            if stored_sketch(pages[i], sketch_size) is None:
                sketch[i] = dsk[j]
            if src.runtime_page_min is None or src.runtime_page_max is None:
                lo[i], hi[i] = dlo[j], dhi[j]
    return sketch, lo, hi


def value_page_means(pages: Sequence, *, device, trace=None):
    """Device ``[n, hd]`` page means of value pages (reference ``summarize_value_page``)."""
    torch = _torch()
    hd = _source(pages[0]).header.head_dim
    out = torch.empty((len(pages), hd), dtype=torch.float32, device=device)
    dense_idx = [i for i, p in enumerate(pages) if _source(p).runtime_page_mean is None]
    for i, p in enumerate(pages):
        if _source(p).runtime_page_mean is not None:
            out[i] = torch.from_numpy(np.asarray(_source(p).runtime_page_mean, np.float32)).to(device)
    if dense_idx:
        dmean, _, _, _ = _dense_summaries([pages[i] for i in dense_idx], 1, trace)
        for j, i in enumerate(dense_idx):
            out[i] = dmean[j]
    return out


def relevance_scores(query, sketch, minima, maxima, mode: str):
    """Device ``[n]`` relevance of every page (reference ``score_page_relevance``)."""
    torch = _torch()
    if mode not in MODES:
        raise ValueError(f"unsupported relevance_mode: {mode}")
    if sketch.dim() != 3:
        raise ValueError("sketch must have shape [n_pages, sketch_rows, head_dim]")
    n, S, hd = (int(x) for x in sketch.shape)
    for name, t in (("minima", minima), ("maxima", maxima)):
        if tuple(t.shape) != (n, hd) or t.dtype != torch.float32 or t.device != sketch.device:
            raise ValueError(f"{name} must be fp32 [n_pages, head_dim] on the sketch's device")
    if sketch.dtype != torch.float32:
        raise ValueError("sketch must be fp32")
    sketch, minima, maxima = sketch.contiguous(), minima.contiguous(), maxima.contiguous()
    q = torch.as_tensor(np.asarray(query, dtype=np.float32) if not isinstance(query, torch.Tensor) else query,
                        dtype=torch.float32, device=sketch.device).reshape(-1).contiguous()
    if q.numel() != hd:
        raise ValueError("query_slice must have shape [head_dim]")
    scores = torch.empty(n, dtype=torch.float32, device=sketch.device)
    st = _lib.lib().dc_page_relevance(C.c_void_p(sketch.data_ptr()), S, C.c_void_p(minima.data_ptr()),
                                      C.c_void_p(maxima.data_ptr()), MODES[mode], C.c_void_p(q.data_ptr()), hd, n,
                                      C.c_void_p(scores.data_ptr()), C.c_void_p(current_stream_ptr()))
    _lib.check(st, "dc_page_relevance")
    return scores


def select_top_k(scores, candidate: np.ndarray, k: int) -> np.ndarray:
    """Host bool mask of the ``k`` best candidates by device score,
    descending, ties to the lower index (reference
    ``session_runtime.py:425-436``)."""
    torch = _torch()
    n = int(scores.numel())
    candidate = np.asarray(candidate)
    if candidate.shape != (n,):
        raise ValueError(f"candidate mask must have one entry per score ({n}), got shape {candidate.shape}")
    if scores.dtype != torch.float32 or not scores.is_contiguous():
        raise ValueError("scores must be a contiguous fp32 tensor")
    cand = torch.from_numpy(np.ascontiguousarray(candidate, dtype=np.uint8)).to(scores.device)
    sel = torch.empty(n, dtype=torch.uint8, device=scores.device)
    st = _lib.lib().dc_select_top_k(C.c_void_p(scores.data_ptr()), C.c_void_p(cand.data_ptr()), n, int(k),
                                    C.c_void_p(sel.data_ptr()), C.c_void_p(current_stream_ptr()))
    _lib.check(st, "dc_select_top_k")
    return sel.cpu().numpy().astype(bool)
