"""Device-resident page pool: one HBM byte arena of page blobs plus an 8-byte
descriptor per page.

This is the MI355X successor of the reference's prepared-page residency
(``dotcache/page_cache.py:23-227`` and the batched uploads of
``dotcache/backends/torch_mps.py:1257-1524``): instead of one torch tensor
view per page and per-chunk caches, every page is a blob at a 256-byte
aligned offset of a single arena, addressed by a page id.  Page tables are
plain int32 arrays of page ids, so a decode batch of ragged sequences whose
pages are scattered across the arena runs in one kernel launch.

Blob layout (also in ``include/dotcache_hip.h``): M0 pages hold the
reference's group_major payload ``[G][C][W]`` uint32, then scales ``[C][G]``
fp16, then (affine) biases ``[C][G]`` fp16; M3 pages hold escape rows
``[C][head_dim]``.  ``C`` is the pool's page capacity, so a partially filled
tail page is appended to in place.

torch provides the device allocation and the stream; all page arithmetic is
in ``libdotcache_hip.so``.
"""
from __future__ import annotations

import ctypes as C
from collections import deque
from dataclasses import dataclass

import numpy as np

from . import _lib
from .types import EncodedPage, PageHeader, words_per_group

DESC_DTYPE = np.dtype([("block", "<u4"), ("tokens", "<u2"), ("format", "u1"), ("bits", "u1")])

_SCHEME_FMT = {"affine": _lib.FMT_M0_AFFINE, "symmetric": _lib.FMT_M0_SYMMETRIC}
_ESCAPE_FMT = {"float16": _lib.FMT_M3_F16, "float32": _lib.FMT_M3_F32, "int8": _lib.FMT_M3_I8}
_TORCH_DT = {}


def _torch():
    import torch

    return torch


def set_encode_path(path: str) -> None:
    """``"auto"`` (the wavefront encode kernel where the geometry fits it)
    or ``"general"`` (the one-thread-per-group kernel only)."""
    paths = {"auto": 0, "general": 1}
    if path not in paths:
        raise ValueError("encode path must be 'auto' or 'general'")
    _lib.check(_lib.lib().dc_set_encode_path(paths[path]), "dc_set_encode_path")


def page_format_of(mode: str, scheme: str, bits: int, escape_dtype: str = "float16") -> tuple[int, int]:
    """(dc_page_format, bits) for a page mode; ValueError if this backend cannot hold it."""
    if mode == "M3":
        if escape_dtype not in _ESCAPE_FMT:
            raise ValueError(f"unsupported escape dtype {escape_dtype}")
        return _ESCAPE_FMT[escape_dtype], 0
    if mode == "M0":
        if scheme not in _SCHEME_FMT:
            raise ValueError(f"M0 scheme {scheme} is not supported by hip_mi355x")
        if bits not in (2, 3, 4, 8):
            raise ValueError(f"M0 bits={bits} is not supported by hip_mi355x")
        return _SCHEME_FMT[scheme], int(bits)
    raise ValueError(f"page mode {mode} is not supported by hip_mi355x")


def dtype_code(t) -> int:
    torch = _torch()
    if t.dtype == torch.float32:
        return _lib.DT_F32
    if t.dtype == torch.float16:
        return _lib.DT_F16
    if t.dtype == torch.bfloat16:
        return _lib.DT_BF16
    raise ValueError(f"unsupported tensor dtype {t.dtype}")


def current_stream_ptr() -> int:
    return int(_torch().cuda.current_stream().cuda_stream)


@dataclass(frozen=True)
class PoolGeometry:
    head_dim: int
    group_size: int
    page_capacity: int
    layout: str = "group_major"

    @property
    def num_groups(self) -> int:
        return -(-self.head_dim // self.group_size)

    def c(self) -> _lib.PageGeometry:
        return _lib.geometry(self.head_dim, self.group_size, self.page_capacity, self.layout)


class DevicePagePool:
    """Arena + descriptor table on one device.

    ``reserve_bytes`` sizes the arena up front; it grows (by re-allocation
    and a device copy) when a batch of pages does not fit.  A page keeps its
    id while it is live; freed blobs and freed ids are reused by later pages
    (blobs of the same size, ids oldest-freed first), so a pool whose pages
    come and go stays the size of its live set.  Reuse is ordered on the
    current stream: work queued before a free still reads the old page.
    """

    def __init__(self, geometry: PoolGeometry, *, device="cuda", reserve_bytes: int = 64 << 20, reserve_pages: int = 4096):
        torch = _torch()
        if geometry.page_capacity > 65535:
            raise ValueError("page_capacity exceeds 65535")
        self.geometry = geometry
        self.device = torch.device(device)
        # zero-filled so never-written token slots of a partial page hold finite values
        self.arena = torch.zeros(max(int(reserve_bytes), 256), dtype=torch.uint8, device=self.device)
        self.format_mask = 0
        self._next_block = 0
        self._free: dict[int, list[int]] = {}
        self._host_desc = np.zeros(max(int(reserve_pages), 16), dtype=DESC_DTYPE)
        self._n_pages = 0
        self._free_ids: deque[int] = deque()
        self._dev_desc = None
        self._dirty_ids: set[int] = set()  # descriptors changed since the last device upload
        # bumped on every descriptor change: page records gathered at one
        # version are stale at any other
        self.desc_version = 0
        self.headers: dict[int, PageHeader] = {}
        self._blob_size: dict[int, int] = {}
        self._live = np.zeros(self._host_desc.shape[0], dtype=bool)

    # ---- bookkeeping -----------------------------------------------------
    @property
    def n_pages(self) -> int:
        return self._n_pages

    def blob_bytes(self, fmt: int, bits: int) -> int:
        return _lib.page_blob_bytes(fmt, bits, self.geometry.c())

    def _ensure_arena(self, end_block: int) -> None:
        need = end_block * 256
        if need <= self.arena.numel():
            return
        torch = _torch()
        new = torch.zeros(max(need, 2 * self.arena.numel()), dtype=torch.uint8, device=self.device)
        used = self._next_block * 256
        if used:
            new[:used].copy_(self.arena[:used])
        self.arena = new

    def _new_id(self) -> int:
        if self._free_ids:
            return self._free_ids.popleft()
        if self._n_pages == self._host_desc.shape[0]:
            grown = np.zeros(2 * self._host_desc.shape[0], dtype=DESC_DTYPE)
            grown[: self._n_pages] = self._host_desc[: self._n_pages]
            self._host_desc = grown
            live = np.zeros(grown.shape[0], dtype=bool)
            live[: self._n_pages] = self._live[: self._n_pages]
            self._live = live
        pid = self._n_pages
        self._n_pages += 1
        return pid

    def allocate(self, fmt: int, bits: int, count: int = 1, *, tokens: int = 0) -> np.ndarray:
        """Allocate ``count`` page blobs of one format; returns int32 page ids.
        Fresh blobs are contiguous, so a batch upload is one copy."""
        nbytes = self.blob_bytes(fmt, bits)
        nblk = nbytes // 256
        ids = np.empty(count, dtype=np.int32)
        free = self._free.get(nblk, [])
        fresh = max(0, count - len(free))
        self._ensure_arena(self._next_block + fresh * nblk)
        for i in range(count):
            if free:
                block = free.pop()
            else:
                block = self._next_block
                self._next_block += nblk
            pid = self._new_id()
            self._host_desc[pid] = (block, tokens, fmt, bits)
            self.format_mask |= _lib.format_bit(fmt, bits)
            self._live[pid] = True
            self._blob_size[pid] = nblk
            ids[i] = pid
        self._dirty_ids.update(ids.tolist())
        self.desc_version += 1
        return ids

    def free(self, page_ids) -> None:
        for pid in np.atleast_1d(np.asarray(page_ids, dtype=np.int64)):
            pid = int(pid)
            if not self._live[pid]:
                raise RuntimeError(f"page {pid} is not live")
            self._live[pid] = False
            nblk = self._blob_size.pop(pid)
            self._free.setdefault(nblk, []).append(int(self._host_desc[pid]["block"]))
            self._host_desc[pid] = (0, 0, 0, 0)
            self.headers.pop(pid, None)
            self._dirty_ids.add(pid)
            self._free_ids.append(pid)
            self.desc_version += 1

    def set_tokens(self, page_ids, tokens) -> None:
        ids = np.atleast_1d(np.asarray(page_ids, dtype=np.int64)).ravel()
        tok = np.broadcast_to(np.asarray(tokens, dtype=np.int64).ravel() if np.ndim(tokens) else tokens, ids.shape)
        if np.any(tok < 0) or np.any(tok > self.geometry.page_capacity):
            raise ValueError("token count outside [0, page_capacity]")
        self._host_desc["tokens"][ids] = tok
        for pid, t in zip(ids.tolist(), tok.tolist()):
            h = self.headers.get(pid)
            if h is not None:
                h.token_count = int(t)
        self._dirty_ids.update(ids.tolist())
        self.desc_version += 1

    def desc(self, page_id: int):
        return self._host_desc[int(page_id)]

    def tokens_of(self, page_ids) -> np.ndarray:
        return self._host_desc["tokens"][np.asarray(page_ids, dtype=np.int64)].astype(np.int64)

    def descs_of(self, page_ids) -> np.ndarray:
        """Host copies of these pages' ``dc_page_desc`` records (``DESC_DTYPE``)."""
        return self._host_desc[np.asarray(page_ids, dtype=np.int64)].copy()

    def formats_of(self, page_ids) -> np.ndarray:
        """The ``_lib.FMT_*`` format of each page id (same shape)."""
        return self._host_desc["format"][np.asarray(page_ids, dtype=np.int64)].astype(np.int64)

    def format_mask_of(self, page_ids) -> int:
        """``dc_pool.format_mask`` bits of the formats these pages hold (a
        subset of :attr:`format_mask`)."""
        ids = np.unique(np.asarray(page_ids, dtype=np.int64).ravel())
        if ids.size == 0:
            return 0
        d = self._host_desc[ids]
        mask = 0
        for fmt, bits in set(zip(d["format"].tolist(), d["bits"].tolist())):
            mask |= _lib.format_bit(int(fmt), int(bits))
        return mask

    def validate_ids(self, page_ids) -> None:
        ids = np.asarray(page_ids, dtype=np.int64).ravel()
        if ids.size and (ids.min() < 0 or ids.max() >= self._n_pages or not self._live[ids].all()):
            raise ValueError("page table names a page that is not live in this pool")

    def device_descs(self):
        """Device copy of the descriptor table, sized like the host table.
        Changed descriptors are copied up by index; the whole table only
        when the host table has outgrown the device copy."""
        torch = _torch()
        cap = self._host_desc.shape[0]
        if self._dev_desc is None or self._dev_desc.numel() < cap:
            raw = self._host_desc.view(np.int64).copy()
            self._dev_desc = torch.from_numpy(raw).to(self.device, non_blocking=False)
            self._dirty_ids.clear()
        elif self._dirty_ids:
            ids = np.fromiter(sorted(self._dirty_ids), dtype=np.int64, count=len(self._dirty_ids))
            vals = torch.from_numpy(self._host_desc[ids].view(np.int64).copy()).to(self.device, non_blocking=False)
            self._dev_desc[torch.from_numpy(ids).to(self.device)] = vals
            self._dirty_ids.clear()
        return self._dev_desc

    def c_pool(self) -> _lib.Pool:
        descs = self.device_descs()
        return _lib.Pool(
            C.c_void_p(self.arena.data_ptr()), self.arena.numel(), C.c_void_p(descs.data_ptr()), self._n_pages,
            self.geometry.c(), self.format_mask,
        )

    # ---- host <-> device pages --------------------------------------------
    def _check_page_geometry(self, page: EncodedPage) -> None:
        h = page.header
        if h.head_dim != self.geometry.head_dim or h.group_size != self.geometry.group_size:
            raise ValueError("page head_dim / group_size do not match the pool geometry")
        if h.layout != self.geometry.layout:
            raise ValueError("page layout does not match the pool geometry")
        if h.token_count > self.geometry.page_capacity:
            raise ValueError("page has more tokens than the pool's page capacity")

    def _blob_from_page(self, page: EncodedPage, fmt: int, bits: int) -> np.ndarray:
        g = self.geometry
        cap = g.page_capacity
        h = page.header
        T = h.token_count
        blob = np.zeros(self.blob_bytes(fmt, bits), dtype=np.uint8)
        if h.mode_default == "M0":
            G = g.num_groups
            W = words_per_group(g.group_size, bits)
            pay = np.zeros((G, cap, W) if g.layout == "group_major" else (cap, G, W), dtype=np.uint32)
            if g.layout == "group_major":
                pay[:, :T, :] = page.payload
            else:
                pay[:T] = page.payload
            pb = pay.view(np.uint8).ravel()
            blob[: pb.size] = pb
            off = -(-pb.size // 16) * 16
            sc = np.zeros((cap, G), dtype=np.float16)
            sc[:T] = page.scales
            blob[off: off + sc.nbytes] = sc.view(np.uint8).ravel()
            if fmt == _lib.FMT_M0_AFFINE:
                off2 = off + -(-sc.nbytes // 16) * 16
                bs = np.zeros((cap, G), dtype=np.float16)
                bs[:T] = page.bias
                blob[off2: off2 + bs.nbytes] = bs.view(np.uint8).ravel()
        else:
            esc = np.asarray(page.escape_payload)
            rows = np.zeros((cap, g.head_dim), dtype=esc.dtype)
            rows[:T] = esc
            rb = rows.view(np.uint8).ravel()
            blob[: rb.size] = rb
            if fmt == _lib.FMT_M3_I8:
                off = -(-rb.size // 16) * 16
                rs = np.zeros(cap, dtype=np.float16)
                rs[:T] = page.escape_scales
                blob[off: off + rs.nbytes] = rs.view(np.uint8).ravel()
        return blob

    def upload_pages(self, pages: list[EncodedPage]) -> np.ndarray:
        """Copy host pages into new blobs; returns their page ids.  Pages are
        grouped by blob size so each group is one host-to-device copy."""
        torch = _torch()
        ids = np.empty(len(pages), dtype=np.int32)
        by_fmt: dict[tuple[int, int], list[int]] = {}
        for i, p in enumerate(pages):
            self._check_page_geometry(p)
            by_fmt.setdefault(page_format_of(p.header.mode_default, p.header.quant_scheme, p.header.bits, p.header.escape_dtype), []).append(i)
        for (fmt, bits), idx in by_fmt.items():
            nblk = self.blob_bytes(fmt, bits) // 256
            host = np.concatenate([self._blob_from_page(pages[i], fmt, bits) for i in idx])
            src = torch.from_numpy(host)
            if self.device.type == "cuda":
                src = src.pin_memory()
            free = self._free.get(nblk, [])
            n_old = min(len(free), len(idx))
            blocks = [free.pop() for _ in range(n_old)]
            start = self._next_block
            self._ensure_arena(start + (len(idx) - n_old) * nblk)
            blocks += [start + j * nblk for j in range(len(idx) - n_old)]
            self._next_block = start + (len(idx) - n_old) * nblk
            for i, block in zip(idx, blocks):
                pid = self._new_id()
                self._host_desc[pid] = (block, pages[i].header.token_count, fmt, bits)
                self.format_mask |= _lib.format_bit(fmt, bits)
                self._live[pid] = True
                self._blob_size[pid] = nblk
                self.headers[pid] = PageHeader.from_dict(pages[i].header.to_dict())
                self._dirty_ids.add(pid)
                self.desc_version += 1
                ids[i] = pid
            if n_old == 0:  # fresh contiguous blocks: one copy
                self.arena[start * 256: start * 256 + host.size].copy_(src, non_blocking=False)
            else:  # one upload, then a scatter of 256-byte rows into the reused blobs
                staged = src.to(self.device, non_blocking=False).view(-1, 256)
                rows = (np.asarray(blocks, dtype=np.int64)[:, None] + np.arange(nblk)).ravel()
                used = self.arena[: self._next_block * 256].view(-1, 256)
                used.index_copy_(0, torch.from_numpy(rows).to(self.device), staged)
        return ids

    def header_of(self, page_id: int, kind: str = "K") -> PageHeader:
        """A reference page header for a page written on the device (by
        ``encode_rows``), from its descriptor and the pool geometry."""
        d = self._host_desc[int(page_id)]
        fmt, bits = int(d["format"]), int(d["bits"])
        g = self.geometry
        m0 = fmt in (_lib.FMT_M0_AFFINE, _lib.FMT_M0_SYMMETRIC)
        b = bits if m0 else 4
        esc = {_lib.FMT_M3_F32: "float32", _lib.FMT_M3_I8: "int8"}.get(fmt, "float16")
        return PageHeader(layer_id=0, kv_head_id=0, kind=kind, token_start=0, token_count=int(d["tokens"]),
                          head_dim=g.head_dim, padded_head_dim=g.num_groups * g.group_size, group_size=g.group_size,
                          num_groups=g.num_groups, bits=b, words_per_group=words_per_group(g.group_size, b),
                          mode_default="M0" if m0 else "M3", layout=g.layout,
                          quant_scheme="symmetric" if fmt == _lib.FMT_M0_SYMMETRIC else "affine", escape_dtype=esc)

    def download_page(self, page_id: int, header: PageHeader | None = None, *, kind: str = "K") -> EncodedPage:
        """Read one page back into a host :class:`EncodedPage` (reference
        layout).  The header is ``header``, the one stored at upload, or one
        made from the descriptor (``kind`` names K or V pages)."""
        d = self._host_desc[int(page_id)]
        fmt, bits, T = int(d["format"]), int(d["bits"]), int(d["tokens"])
        g = self.geometry
        cap = g.page_capacity
        start = int(d["block"]) * 256
        blob = self.arena[start: start + self.blob_bytes(fmt, bits)].cpu().numpy()
        h = header or self.headers.get(int(page_id)) or self.header_of(page_id, kind)
        h = PageHeader.from_dict(h.to_dict())
        h.token_count = T
        if fmt in (_lib.FMT_M0_AFFINE, _lib.FMT_M0_SYMMETRIC):
            G = g.num_groups
            W = words_per_group(g.group_size, bits)
            n = G * cap * W * 4
            pay = blob[:n].view(np.uint32).reshape((G, cap, W) if g.layout == "group_major" else (cap, G, W))
            pay = pay[:, :T, :].copy() if g.layout == "group_major" else pay[:T].copy()
            off = -(-n // 16) * 16
            sc = blob[off: off + cap * G * 2].view(np.float16).reshape(cap, G)[:T].copy()
            bias = None
            if fmt == _lib.FMT_M0_AFFINE:
                off2 = off + -(-(cap * G * 2) // 16) * 16
                bias = blob[off2: off2 + cap * G * 2].view(np.float16).reshape(cap, G)[:T].copy()
            return EncodedPage(header=h, payload=pay, scales=sc, bias=bias)
        dt = {_lib.FMT_M3_F16: np.float16, _lib.FMT_M3_F32: np.float32, _lib.FMT_M3_I8: np.int8}[fmt]
        n = cap * g.head_dim * np.dtype(dt).itemsize
        rows = blob[:n].view(dt).reshape(cap, g.head_dim)[:T].copy()
        rs = None
        if fmt == _lib.FMT_M3_I8:
            off = -(-n // 16) * 16
            rs = blob[off: off + cap * 2].view(np.float16)[:T].copy()
        return EncodedPage(header=h, escape_payload=rows, escape_scales=rs)

    # ---- device encode ------------------------------------------------------
    def encode_rows(self, values, page_ids, slots) -> None:
        """Encode device rows ``values [n, head_dim]`` into (page, slot) pairs
        with ``dc_encode_rows``.  ``page_ids`` / ``slots``: device or host
        int32 arrays of length n.  Token counts are not changed."""
        torch = _torch()
        if values.dim() != 2 or values.shape[1] != self.geometry.head_dim:
            raise ValueError("values must have shape [n, head_dim]")
        if values.stride(1) != 1:
            values = values.contiguous()
        n = values.shape[0]
        pid = torch.as_tensor(page_ids, dtype=torch.int32, device=self.device).contiguous()
        slot = torch.as_tensor(slots, dtype=torch.int32, device=self.device).contiguous()
        if pid.numel() != n or slot.numel() != n:
            raise ValueError("page_ids and slots must have one entry per row")
        pool = self.c_pool()
        st = _lib.lib().dc_encode_rows(
            C.c_void_p(values.data_ptr()), dtype_code(values), n, values.stride(0), C.c_void_p(pid.data_ptr()),
            C.c_void_p(slot.data_ptr()), pool, C.c_void_p(current_stream_ptr()),
        )
        _lib.check(st, "dc_encode_rows")

    def encode_rows_with(self, v_pool: "DevicePagePool", k_values, v_values, k_page_ids, k_slots, v_page_ids,
                         v_slots) -> None:
        """Keys into this pool and values into ``v_pool`` in one launch
        (``dc_encode_rows_kv``): the per-step append of new tokens.  Both
        value arrays are ``[n, head_dim]`` of one dtype and row stride."""
        torch = _torch()
        hd = self.geometry.head_dim
        if v_pool.geometry.head_dim != hd:
            raise ValueError("key and value pools must share head_dim")
        if k_values.dim() != 2 or k_values.shape[1] != hd or tuple(v_values.shape) != tuple(k_values.shape):
            raise ValueError("key and value rows must have the same shape [n, head_dim]")
        if k_values.dtype != v_values.dtype:
            raise ValueError("key and value rows must have the same dtype")
        k_values, v_values = k_values.contiguous(), v_values.contiguous()
        n = k_values.shape[0]
        ids = [torch.as_tensor(x, dtype=torch.int32, device=self.device).contiguous()
               for x in (k_page_ids, k_slots, v_page_ids, v_slots)]
        if any(t.numel() != n for t in ids):
            raise ValueError("page_ids and slots must have one entry per row")
        st = _lib.lib().dc_encode_rows_kv(
            C.c_void_p(k_values.data_ptr()), C.c_void_p(v_values.data_ptr()), dtype_code(k_values), n, hd,
            *(C.c_void_p(t.data_ptr()) for t in ids), self.c_pool(), v_pool.c_pool(), C.c_void_p(current_stream_ptr()))
        _lib.check(st, "dc_encode_rows_kv")

    def read_bytes(self, page_ids) -> int:
        """Compressed bytes a reader fetches for these pages (valid tokens only)."""
        return int(self.read_bytes_each(page_ids).sum())

    def read_bytes_each(self, page_ids) -> np.ndarray:
        """int64 array shaped like ``page_ids``: each page's compressed bytes
        a reader fetches (valid tokens only)."""
        ids = np.asarray(page_ids, dtype=np.int64)
        if ids.size == 0:
            return np.zeros(ids.shape, dtype=np.int64)
        d = self._host_desc[ids.ravel()]
        key = (d["format"].astype(np.int64) << 32) | (d["bits"].astype(np.int64) << 16) | d["tokens"].astype(np.int64)
        uniq, inv = np.unique(key, return_inverse=True)
        geo = self.geometry.c()
        each = np.array([_lib.page_read_bytes(int(u >> 32), int((u >> 16) & 0xFFFF), int(u & 0xFFFF), geo)
                         for u in uniq], dtype=np.int64)
        return each[inv.ravel()].reshape(ids.shape)
