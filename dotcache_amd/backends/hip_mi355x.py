"""``hip_mi355x`` backend: the reference's per-backend function set served by
hand-written gfx950 kernels.

Same names, argument meanings and error behaviour as the ``torch_cuda``
backend of the reference (``dotcache/backends/torch_cuda.py:26-168``, whose
behaviour is ``dotcache/backends/torch_mps.py``), with ``_cuda`` replaced by
``_hip``:

=====================================================  ==============================================
hip_mi355x                                             reference
=====================================================  ==============================================
``hip_available``                                      ``cuda_available`` (torch_cuda.py:29-30)
``page_supported_hip``                                 ``page_supported_cuda`` (torch_cuda.py:33-34)
``prepare_page_hip`` / ``prepare_pages_hip``           torch_cuda.py:37-50
``score_page_hip`` / ``score_pages_hip``               torch_cuda.py:53-68
``mix_page_hip``                                       torch_cuda.py:71-78
``decode_step_hip``                                    torch_cuda.py:81-96
``decode_multi_query_step_hip(_tensor)``               torch_cuda.py:99-112, :161-168
``decode_grouped_multiquery_step_(prepared_)hip_tensor``  torch_cuda.py:115-143
``..._prepared_hip_tensor_output_only``                torch_cuda.py:146-158
``PreparedPageHIP``                                    ``PreparedPageCUDA`` (torch_cuda.py:26)
=====================================================  ==============================================

Prepared pages live in a :class:`~dotcache_amd.page_pool.DevicePagePool`
(one per page geometry) instead of per-page tensors.  Unlike the reference's
torch path, every M0 scheme (affine and symmetric) and code width (2, 3, 4,
8 bits) and every M3 escape dtype run on the device -- nothing falls back to
the CPU.  Every function raises RuntimeError when the HIP library or a GPU is
missing.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Any, Sequence

import numpy as np

from .. import _lib
from ..decode import decode_paged
from ..page_pool import DevicePagePool, PoolGeometry, current_stream_ptr, page_format_of
from ..tracing import ExecutionTrace
from ..types import EncodedPage, PageHeader

DEVICE_TYPE = "hip"
_pools: dict[tuple, DevicePagePool] = {}


def _torch():
    import torch

    return torch


@dataclass(slots=True)
class PreparedPageHIP:
    """A page resident in a device pool (reference ``PreparedPageTorch``,
    ``torch_mps.py:107-134``): header, source page, and where it lives."""

    source_page: EncodedPage
    header: PageHeader
    pool: DevicePagePool
    page_id: int
    host_to_device_nbytes: int = 0
    device_type: str = DEVICE_TYPE

    @property
    def payload_nbytes(self) -> int:
        return self.source_page.payload_nbytes

    @property
    def metadata_nbytes(self) -> int:
        return self.source_page.metadata_nbytes

    @property
    def resident_nbytes(self) -> int:
        return self.pool.blob_bytes(*page_format_of(self.header.mode_default, self.header.quant_scheme,
                                                    self.header.bits, self.header.escape_dtype))

    def __del__(self) -> None:
        # the blob goes back to its pool with the last reference, as a torch
        # page's tensors do; work already queued on the stream still reads it
        # first (a later upload into the slot is ordered after it)
        try:
            self.pool.free(self.page_id)
        except Exception:  # interpreter shutdown, or the pool released it already
            pass


PageLike = EncodedPage | PreparedPageHIP


def hip_available() -> bool:
    """True when a GPU is visible and libdotcache_hip.so loads."""
    try:
        torch = _torch()
        if not torch.cuda.is_available():
            return False
        _lib.lib()
        return True
    except Exception:
        return False


def _require() -> None:
    torch = _torch()
    if not torch.cuda.is_available():
        raise RuntimeError("hip_mi355x is unavailable on this machine (no GPU visible)")
    _lib.lib()


def _source(page: PageLike) -> EncodedPage:
    return page.source_page if isinstance(page, PreparedPageHIP) else page


def page_supported_hip(page: PageLike) -> bool:
    """Which pages this backend can hold (cf. reference ``torch_mps.py:1018-1074``)."""
    src = _source(page)
    h = src.header
    if h.layout not in ("group_major", "token_major"):
        return False
    if int(h.group_size) <= 0 or int(h.num_groups) <= 0:
        return False
    if int(h.group_size) * int(h.num_groups) != int(h.padded_head_dim):
        return False
    if h.token_count > 65535:
        return False
    if h.mode_default == "M3":
        if src.escape_payload is None:
            return False
        if h.escape_dtype == "int8":
            return src.escape_scales is not None
        return h.escape_dtype in ("float16", "float32")
    if h.mode_default == "M0":
        if src.payload is None or src.scales is None or h.bits not in (2, 3, 4, 8):
            return False
        if h.quant_scheme == "affine":
            return src.bias is not None
        return h.quant_scheme == "symmetric"
    return False


def _capacity(token_count: int) -> int:
    return max(64, 1 << (max(int(token_count), 1) - 1).bit_length())


def pool_for(head_dim: int, group_size: int, capacity: int, layout: str, device=None, kind: str = "K") -> DevicePagePool:
    """The module-level pool for one page geometry and kind (created on
    first use).  Key and value pages live in separate pools, so a pool's
    format mask names the formats of one role only and the decode kernel
    is chosen for the key and value formats actually present."""
    torch = _torch()
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    key = (head_dim, group_size, capacity, layout, str(dev), kind)
    pool = _pools.get(key)
    if pool is None:
        pool = DevicePagePool(PoolGeometry(head_dim, group_size, capacity, layout), device=dev)
        _pools[key] = pool
    return pool


def clear_prepared_pools() -> None:
    _pools.clear()


def prepare_pages_hip(pages: Sequence[PageLike], *, trace: ExecutionTrace | None = None,
                      pool: DevicePagePool | None = None) -> list[PreparedPageHIP]:
    """Upload host pages into a device pool (one copy per page format);
    already-prepared pages pass through.  Reference ``prepare_pages_cuda``."""
    _require()
    out: list[PreparedPageHIP | None] = [None] * len(pages)
    todo: dict[tuple, list[int]] = {}
    for i, p in enumerate(pages):
        if isinstance(p, PreparedPageHIP) and (pool is None or p.pool is pool):
            out[i] = p
            continue
        src = _source(p)
        if not page_supported_hip(src):
            raise ValueError("page is unsupported by hip_mi355x in this phase")
        h = src.header
        key = (h.head_dim, h.group_size, h.layout, h.kind)
        todo.setdefault(key, []).append(i)
    for (hd, gs, layout, kind), idx in todo.items():
        cap = _capacity(max(_source(pages[i]).header.token_count for i in idx))
        target = pool if pool is not None else pool_for(hd, gs, cap, layout, kind=kind)
        srcs = [_source(pages[i]) for i in idx]
        ids = target.upload_pages(srcs)
        for i, pid, src in zip(idx, ids.tolist(), srcs):
            nbytes = src.device_nbytes
            out[i] = PreparedPageHIP(source_page=src, header=src.header, pool=target, page_id=int(pid),
                                     host_to_device_nbytes=nbytes)
            if trace is not None:
                trace.record_host_to_device(nbytes)
    return out  # type: ignore[return-value]


def prepare_page_hip(page: PageLike, *, trace: ExecutionTrace | None = None) -> PreparedPageHIP:
    return prepare_pages_hip([page], trace=trace)[0]


def _one_pool(pages: Sequence[PageLike], trace=None) -> tuple[DevicePagePool, np.ndarray, list[PreparedPageHIP]]:
    """Prepared pages that all live in one pool (re-preparing into the
    largest-capacity pool when they do not)."""
    prepared = prepare_pages_hip(pages, trace=trace)
    pools = {id(p.pool): p.pool for p in prepared}
    if len(pools) > 1:
        target = max(pools.values(), key=lambda pl: pl.geometry.page_capacity)
        prepared = prepare_pages_hip([p.source_page if p.pool is not target else p for p in prepared], trace=trace,
                                     pool=target)
    pool = prepared[0].pool
    return pool, np.asarray([p.page_id for p in prepared], dtype=np.int32), prepared


def _one_pool_with_capacity(pages, capacity: int, trace=None):
    src = [_source(p) for p in pages]
    h = src[0].header
    pool = pool_for(h.head_dim, h.group_size, capacity, h.layout, kind=h.kind)
    prepared = prepare_pages_hip(src, trace=trace, pool=pool)
    return pool, np.asarray([p.page_id for p in prepared], dtype=np.int32), prepared


def _record_reads(trace: ExecutionTrace | None, prepared: Sequence[PreparedPageHIP], name: str) -> None:
    if trace is None:
        return
    trace.record_call(name)
    for p in prepared:
        trace.record_page_read(p.payload_nbytes, p.metadata_nbytes)
        trace.record_device_read(p.source_page.device_nbytes)


def _queries_tensor(q, hd: int, device):
    torch = _torch()
    t = q if isinstance(q, torch.Tensor) else torch.as_tensor(np.asarray(q, dtype=np.float32))
    t = t.to(device=device, dtype=torch.float32)
    if t.dim() == 1:
        t = t[None, :]
    if t.shape[-1] != hd:
        raise ValueError("query head_dim does not match the pages")
    return t.contiguous()


def _score_tensor(queries, pool: DevicePagePool, ids: np.ndarray, score=None):
    """logits [n_queries, total_tokens] on the device.  With ``score`` (a
    bool mask over the pages), only those pages are scored; the columns of
    the others are left unwritten."""
    torch = _torch()
    dev = pool.device
    tok = pool.tokens_of(ids)
    offsets = np.zeros(ids.size + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(tok)
    total = int(offsets[-1])
    q = _queries_tensor(queries, pool.geometry.head_dim, dev)
    logits = torch.empty((q.shape[0], total), dtype=torch.float32, device=dev)
    sel_ids, sel_off = (ids, offsets) if score is None else (ids[score], offsets[:-1][score])
    if sel_ids.size:
        ids_d = torch.from_numpy(np.ascontiguousarray(sel_ids)).to(dev)
        off_d = torch.from_numpy(np.ascontiguousarray(sel_off)).to(dev)
        st = _lib.lib().dc_score_pages(pool.c_pool(), C.c_void_p(ids_d.data_ptr()), C.c_void_p(off_d.data_ptr()),
                                       sel_ids.size, C.c_void_p(q.data_ptr()), q.shape[0],
                                       C.c_void_p(logits.data_ptr()), total, C.c_void_p(current_stream_ptr()))
        _lib.check(st, "dc_score_pages")
    return logits, offsets


def _mix_tensor(weights, pool: DevicePagePool, ids: np.ndarray, out=None):
    """out [n_queries, head_dim] (+)= weights [n_queries, total_tokens] @ V."""
    torch = _torch()
    dev = pool.device
    tok = pool.tokens_of(ids)
    offsets = np.zeros(ids.size + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(tok)
    w = weights if isinstance(weights, torch.Tensor) else torch.as_tensor(np.asarray(weights, dtype=np.float32))
    w = w.to(device=dev, dtype=torch.float32)
    if w.dim() == 1:
        w = w[None, :]
    w = w.contiguous()
    if w.shape[1] != int(offsets[-1]):
        raise ValueError("attn_weights must have shape [token_count]")
    acc = 1
    if out is None:
        out = torch.empty((w.shape[0], pool.geometry.head_dim), dtype=torch.float32, device=dev)
        acc = 0
    ids_d = torch.from_numpy(ids).to(dev)
    off_d = torch.from_numpy(offsets).to(dev)
    st = _lib.lib().dc_mix_pages(pool.c_pool(), C.c_void_p(ids_d.data_ptr()), C.c_void_p(off_d.data_ptr()), ids.size,
                                 C.c_void_p(w.data_ptr()), w.shape[0], w.shape[1], C.c_void_p(out.data_ptr()), acc,
                                 C.c_void_p(current_stream_ptr()))
    _lib.check(st, "dc_mix_pages")
    return out


def _softmax_(x) -> None:
    st = _lib.lib().dc_softmax_rows(C.c_void_p(x.data_ptr()), x.shape[0], x.shape[1], x.stride(0),
                                    C.c_void_p(current_stream_ptr()))
    _lib.check(st, "dc_softmax_rows")


def score_page_hip(query_slice: np.ndarray | Any, page: PageLike, *, trace: ExecutionTrace | None = None) -> np.ndarray:
    """Logits ``[token_count]`` of one page -- reference ``score_page_cuda``."""
    pool, ids, prepared = _one_pool([page], trace)
    _record_reads(trace, prepared, "score_page")
    logits, _ = _score_tensor(query_slice, pool, ids)
    return logits[0].cpu().numpy()


def score_pages_hip(query_slice: np.ndarray | Any, pages: Sequence[PageLike], *,
                    trace: ExecutionTrace | None = None) -> list[np.ndarray]:
    """Per-page logits in one launch -- reference ``score_pages_cuda``."""
    if not pages:
        return []
    pool, ids, prepared = _one_pool(pages, trace)
    _record_reads(trace, prepared, "score_pages")
    logits, offsets = _score_tensor(query_slice, pool, ids)
    flat = logits[0].cpu().numpy()
    return [flat[offsets[i]: offsets[i + 1]].copy() for i in range(ids.size)]


def mix_page_hip(attn_weights: np.ndarray | Any, page: PageLike, *, out_acc: np.ndarray | None = None,
                 trace: ExecutionTrace | None = None) -> np.ndarray:
    """``out_acc + weights @ V(page)`` -- reference ``mix_page_cuda``."""
    torch = _torch()
    pool, ids, prepared = _one_pool([page], trace)
    _record_reads(trace, prepared, "mix_page")
    hd = pool.geometry.head_dim
    out = None
    if out_acc is not None:
        acc = np.asarray(out_acc, dtype=np.float32)
        if acc.shape != (hd,):
            raise ValueError("out_acc must have shape [head_dim]")
        out = torch.from_numpy(acc.copy()).to(pool.device)[None, :]
    return _mix_tensor(attn_weights, pool, ids, out)[0].cpu().numpy()


def _pair_pools(key_pages, value_pages, trace):
    if len(key_pages) != len(value_pages):
        raise ValueError("key_pages and value_pages must contain the same number of pages")
    if not key_pages:
        raise ValueError("decode_step requires at least one page")
    kpool, kid, kprep = _one_pool(key_pages, trace)
    vpool, vid, vprep = _one_pool(value_pages, trace)
    if not np.array_equal(kpool.tokens_of(kid), vpool.tokens_of(vid)):
        raise ValueError("key and value pages must hold the same token counts")
    return kpool, vpool, kid, vid, kprep + vprep


def decode_multi_query_step_hip_tensor(query_slices, key_pages, value_pages, *, precomputed_page_logits=None,
                                       trace: ExecutionTrace | None = None):
    """(logits [Q, T], weights [Q, T], output [Q, head_dim]) as device tensors.

    ``precomputed_page_logits[i]``, when not None, is used as page i's logits
    and page i's key bytes are not read (reference
    ``decode_step_with_page_logits``, dotcache/attention_runtime.py:298-303,
    and its device path dotcache/backends/torch_mps.py:2690-2700); the trace
    counts the key pages scored and every value page."""
    torch = _torch()
    kpool, vpool, kid, vid, prepared = _pair_pools(key_pages, value_pages, trace)
    kprep, vprep = prepared[:kid.size], prepared[kid.size:]
    cached = [None] * kid.size
    if precomputed_page_logits is not None:
        if len(precomputed_page_logits) != kid.size:
            raise ValueError("precomputed_page_logits must align with key_pages")
        cached = list(precomputed_page_logits)
    score = np.asarray([c is None for c in cached], dtype=bool)
    kread = [p for p, s in zip(kprep, score) if s]
    _record_reads(trace, kread + list(vprep), "decode_multi_query_step")
    logits, offsets = _score_tensor(query_slices, kpool, kid, score=None if score.all() else score)
    for i, c in enumerate(cached):
        if c is None:
            continue
        c = torch.as_tensor(np.asarray(c, dtype=np.float32) if not isinstance(c, torch.Tensor) else c,
                            dtype=torch.float32, device=kpool.device)
        n = int(offsets[i + 1] - offsets[i])
        if c.numel() != n:
            raise ValueError("precomputed page logits must have shape [token_count]")
        logits[:, offsets[i]: offsets[i + 1]] = c.reshape(1, n)
    weights = logits.clone()
    _softmax_(weights)
    out = _mix_tensor(weights, vpool, vid)
    return logits, weights, out


def decode_step_hip(query_slice, key_pages, value_pages, *, precomputed_page_logits=None,
                    trace: ExecutionTrace | None = None) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(logits, weights, output) for one query -- reference ``decode_step_cuda``."""
    q = np.asarray(query_slice, dtype=np.float32) if not hasattr(query_slice, "device") else query_slice
    logits, weights, out = decode_multi_query_step_hip_tensor(q, key_pages, value_pages,
                                                              precomputed_page_logits=precomputed_page_logits, trace=trace)
    return logits[0].cpu().numpy(), weights[0].cpu().numpy(), out[0].cpu().numpy()


def decode_multi_query_step_hip(query_slices, key_pages, value_pages, *, trace: ExecutionTrace | None = None):
    q = np.asarray(query_slices, dtype=np.float32) if not hasattr(query_slices, "device") else query_slices
    if getattr(q, "ndim", 2) != 2:
        raise ValueError("query_slices must have shape [query_count, head_dim]")
    logits, weights, out = decode_multi_query_step_hip_tensor(q, key_pages, value_pages, trace=trace)
    return logits.cpu().numpy(), weights.cpu().numpy(), out.cpu().numpy()


def _grouped_inputs(query_groups, key_pages_by_group, value_pages_by_group):
    if not key_pages_by_group or not value_pages_by_group:
        raise ValueError("grouped decode requires non-empty key/value page groups")
    if len(key_pages_by_group) != len(value_pages_by_group):
        raise ValueError("key_pages_by_group and value_pages_by_group must have the same group count")
    if len(query_groups) != len(key_pages_by_group):
        raise ValueError("query_groups must align with key/value group count")
    if not key_pages_by_group[0]:
        raise ValueError("grouped decode requires at least one key page per group")


def decode_grouped_multiquery_step_prepared_hip_tensor(query_groups, key_pages_by_group, value_pages_by_group, *,
                                                       trace: ExecutionTrace | None = None, **_ignored):
    """Per KV group: (logits [G, Q, T], weights [G, Q, T], output [G, Q, head_dim])
    -- reference ``decode_grouped_multiquery_step_prepared_cuda_tensor``
    (``torch_cuda.py:131-143`` over ``torch_mps.py:4110-4273``).  One batched
    pass for all groups: one grouped score launch, one softmax over the
    G x Q rows, one grouped mix launch.  Groups must hold the same token
    counts, as in the reference."""
    torch = _torch()
    _grouped_inputs(query_groups, key_pages_by_group, value_pages_by_group)
    G = len(key_pages_by_group)
    counts = [len(g) for g in key_pages_by_group]
    if counts != [len(g) for g in value_pages_by_group]:
        raise ValueError("key_pages_by_group and value_pages_by_group must align")
    flat_k = [p for grp in key_pages_by_group for p in grp]
    flat_v = [p for grp in value_pages_by_group for p in grp]
    kpool, kids, kprep = _one_pool(flat_k, trace)
    vpool, vids, vprep = _one_pool(flat_v, trace)
    _record_reads(trace, kprep + vprep, "decode_grouped_multiquery_step")
    ktok, vtok = kpool.tokens_of(kids), vpool.tokens_of(vids)
    if not np.array_equal(ktok, vtok):
        raise ValueError("key and value pages must hold the same token counts")
    bounds = np.zeros(G + 1, dtype=np.int64)
    bounds[1:] = np.cumsum(counts)
    totals = [int(ktok[bounds[g]:bounds[g + 1]].sum()) for g in range(G)]
    dev = kpool.device
    q = torch.stack([_queries_tensor(x, kpool.geometry.head_dim, dev) for x in query_groups]).contiguous()  # [G, Q, hd]
    Q, hd = int(q.shape[1]), int(q.shape[2])
    if len(set(totals)) != 1:
        raise ValueError("all query groups must have the same query count and token count for batched grouped decode")
    T = totals[0]
    # first token of every page within its group, the group of every page
    starts = np.zeros(len(kids), dtype=np.int32)
    for g in range(G):
        seg = ktok[bounds[g]:bounds[g + 1]]
        starts[bounds[g]:bounds[g + 1]] = np.cumsum(seg) - seg
    page_group = np.repeat(np.arange(G, dtype=np.int32), counts)
    kids_d, vids_d = torch.from_numpy(kids).to(dev), torch.from_numpy(vids).to(dev)
    off_d = torch.from_numpy(starts).to(dev)
    grp_d = torch.from_numpy(page_group).to(dev)
    gp_d = torch.from_numpy(bounds.astype(np.int32)).to(dev)
    logits = torch.empty((G, Q, T), dtype=torch.float32, device=dev)
    stream = C.c_void_p(current_stream_ptr())
    L = _lib.lib()
    _lib.check(L.dc_score_pages_grouped(kpool.c_pool(), C.c_void_p(kids_d.data_ptr()), C.c_void_p(off_d.data_ptr()),
                                        C.c_void_p(grp_d.data_ptr()), G, len(kids), C.c_void_p(q.data_ptr()), Q,
                                        C.c_void_p(logits.data_ptr()), T, stream), "dc_score_pages_grouped")
    weights = logits.clone()
    _lib.check(L.dc_softmax_rows(C.c_void_p(weights.data_ptr()), G * Q, T, T, stream), "dc_softmax_rows")
    out = torch.empty((G, Q, hd), dtype=torch.float32, device=dev)
    _lib.check(L.dc_mix_pages_grouped(vpool.c_pool(), C.c_void_p(vids_d.data_ptr()), C.c_void_p(off_d.data_ptr()),
                                      C.c_void_p(gp_d.data_ptr()), G, len(vids), C.c_void_p(weights.data_ptr()), Q, T,
                                      C.c_void_p(out.data_ptr()), 0, stream), "dc_mix_pages_grouped")
    return logits, weights, out


decode_grouped_multiquery_step_hip_tensor = decode_grouped_multiquery_step_prepared_hip_tensor


def decode_grouped_multiquery_step_prepared_hip_tensor_output_only(query_groups, key_pages_by_group,
                                                                   value_pages_by_group, *,
                                                                   trace: ExecutionTrace | None = None,
                                                                   pages_per_split: int | None = None, **_ignored):
    """Output ``[G, Q, head_dim]`` only, from the fused score + online softmax
    + mix kernel -- reference
    ``decode_grouped_multiquery_step_prepared_cuda_tensor_output_only``.
    Groups may have different page counts."""
    torch = _torch()
    _grouped_inputs(query_groups, key_pages_by_group, value_pages_by_group)
    G = len(key_pages_by_group)
    flat_k = [p for grp in key_pages_by_group for p in grp]
    flat_v = [p for grp in value_pages_by_group for p in grp]
    counts = [len(g) for g in key_pages_by_group]
    if counts != [len(g) for g in value_pages_by_group]:
        raise ValueError("key_pages_by_group and value_pages_by_group must align")
    kpool, kids, kprep = _one_pool(flat_k, trace)
    vpool, vids, vprep = _one_pool(flat_v, trace)
    if vpool.geometry.page_capacity != kpool.geometry.page_capacity:
        vpool, vids, vprep = _one_pool_with_capacity(flat_v, kpool.geometry.page_capacity, trace)
    _record_reads(trace, kprep + vprep, "decode_grouped_output_only")
    width = max(counts)
    kt = np.zeros((G, 1, width), dtype=np.int32)  # one "sequence" per group with one KV head
    vt = np.zeros((G, 1, width), dtype=np.int32)
    off = 0
    for g, n in enumerate(counts):
        kt[g, 0, :n] = kids[off: off + n]
        vt[g, 0, :n] = vids[off: off + n]
        off += n
    dev = kpool.device
    q = torch.stack([_queries_tensor(x, kpool.geometry.head_dim, dev) for x in query_groups])  # [G, Q, hd]
    out = decode_paged(kpool, torch.from_numpy(kt).to(dev), torch.from_numpy(vt).to(dev),
                       np.asarray(counts, dtype=np.int32), q[:, None].contiguous(), pages_per_split=pages_per_split,
                       v_pool=vpool)
    return out[:, 0]
