"""Block-table KV cache for a paged serving engine: vLLM block ids mapped
to device pages.

MI355X counterpart of the reference's vLLM adapter cache (reference
``dotcache/integrations/vllm_adapter/block_cache.py:92-551``).  The
reference keeps a ``ModelPagedKVCache`` per model and, beside it, one host
``EncodedPage`` per (layer, KV head, block id), re-encoded with numpy on
every appended token.  Here a block id owns device pages directly:

* a live (partially filled) block is an escape (M3) page per KV head,
  written row by row by ``dc_encode_rows``, plus its rows in fp32 in HBM;
* when its last slot is written the block is encoded, on the device, into
  a page of the layer's mode (``DotCacheConfig.resolve_page_mode``) from
  the fp32 rows -- bit-identical to the reference's ``encode_page`` of the
  block -- and the escape pages are released.

``write_slots`` takes rows with a vLLM-style slot mapping (``block_id *
block_size + offset``), and ``decode_block_tables`` decodes a batch of
sequences given by block tables and context lengths in one launch: the
page tables are gathered from the block map on the device.  The
reference's single-sequence interface (``sync_layer_blocks``,
``append_step``, ``append_tokens_torch``, ``decode_layer``,
``block_entry``) is built on these two.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .config import DotCacheConfig
from .decode import decode_paged, plan_decode, workspace_bytes
from .encode import resolve_encode_spec
from .kv_cache import default_q_head_to_kv_head
from .page_pool import DevicePagePool, PoolGeometry, page_format_of
from .types import EncodedPage


def _torch():
    import torch

    return torch


@dataclass(frozen=True)
class VllmBlockKey:
    """Reference ``block_cache.py:16-21``."""
    layer_id: int
    kv_head_id: int
    block_id: int
    kind: str


@dataclass
class VllmBlockEntry:
    """Reference ``block_cache.py:24-30``; ``page`` is read back from the
    device when the entry is requested."""
    key: VllmBlockKey
    page: EncodedPage
    finalized: bool
    token_count: int
    token_start: int


class DeviceVllmPagedKVCache:
    """Pages of ``num_hidden_layers`` layers addressed by block id.

    Rows may be numpy arrays or torch tensors (fp32, fp16, bf16), read as
    fp32.  ``block_size`` equals ``config.tokens_per_page``, as in the
    reference (``block_cache.py:103-104``).
    """

    def __init__(self, *, config: DotCacheConfig, num_hidden_layers: int, num_attention_heads: int,
                 num_key_value_heads: int, block_size: int, device="cuda", reserve_blocks: int = 64):
        torch = _torch()
        if config.tokens_per_page != block_size:
            raise ValueError("DotCache tokens_per_page must equal the vLLM block_size for this phase")
        q_map = default_q_head_to_kv_head(num_attention_heads, num_key_value_heads)
        if num_attention_heads // num_key_value_heads > 16:
            raise ValueError("at most 16 query heads per KV head")
        self.config = config
        self.block_size = int(block_size)
        self.num_hidden_layers = int(num_hidden_layers)
        self.num_attention_heads = int(num_attention_heads)
        self.num_key_value_heads = int(num_key_value_heads)
        self.device = torch.device(device)
        self.default_q_head_to_kv_head = q_map
        L, H, P, hd = self.num_hidden_layers, self.num_key_value_heads, self.block_size, config.head_dim
        self._specs = {kind: resolve_encode_spec(config, kind=kind) for kind in ("K", "V")}
        self._live_fmt = {kind: page_format_of("M3", "affine", 4, self._specs[kind]["escape_dtype"]) for kind in ("K", "V")}
        self._pools = {}
        for kind in ("K", "V"):
            geo = PoolGeometry(hd, config.group_size, P, self._specs[kind]["layout"])
            probe = DevicePagePool(geo, device=self.device, reserve_bytes=256, reserve_pages=16)
            blob = max(probe.blob_bytes(*self._page_format(kind, 0, 0)), probe.blob_bytes(*self._live_fmt[kind]))
            self._pools[kind] = DevicePagePool(geo, device=self.device, reserve_bytes=L * H * reserve_blocks * blob + (1 << 20),
                                               reserve_pages=L * H * reserve_blocks + 16)
        self.k_pool, self.v_pool = self._pools["K"], self._pools["V"]
        n = max(int(reserve_blocks), 1)
        # per layer, per block id: page id of each KV head (-1: none), tokens written, finalised, first token
        self._map = {kind: [np.full((n, H), -1, dtype=np.int32) for _ in range(L)] for kind in ("K", "V")}
        self._fill = [np.zeros(n, dtype=np.int32) for _ in range(L)]
        self._final = [np.zeros(n, dtype=bool) for _ in range(L)]
        self._start = [np.full(n, -1, dtype=np.int64) for _ in range(L)]
        self._rows = [dict() for _ in range(L)]     # live block id -> fp32 rows [2, H, P, hd] on the device
        self._dev_map = [None] * L                   # device copies of the K / V maps, rebuilt when they change
        # the single-sequence view of the reference interface: block ids in token order, cached length
        self._seq_blocks = [[] for _ in range(L)]
        self._seq_len = np.zeros(L, dtype=np.int64)
        self._workspace = None

    # ---- formats and small helpers ------------------------------------------
    def _page_format(self, kind: str, layer_id: int, kv_head_id: int) -> tuple[int, int]:
        spec = self._specs[kind]
        mode = self.config.resolve_page_mode(kind=kind, layer_id=layer_id, kv_head_id=kv_head_id)
        return page_format_of(mode, spec["scheme"], spec["bits"], spec["escape_dtype"])

    def _check_layer(self, layer_id: int) -> int:
        lid = int(layer_id)
        if not 0 <= lid < self.num_hidden_layers:
            raise ValueError(f"layer_id {layer_id} out of range")
        return lid

    def _as_rows(self, x, name: str):
        """``x [n, H, hd]`` as fp32 on the device."""
        torch = _torch()
        t = x if isinstance(x, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(np.asarray(x, dtype=np.float32)))
        t = t.to(device=self.device, dtype=torch.float32)
        if t.dim() != 3 or t.shape[1] != self.num_key_value_heads or t.shape[2] != self.config.head_dim:
            raise ValueError(f"{name} must have shape [tokens, {self.num_key_value_heads}, {self.config.head_dim}]")
        return t

    def _grow(self, lid: int, block_id: int) -> None:
        n = self._fill[lid].shape[0]
        if block_id < n:
            return
        m = max(2 * n, block_id + 1)
        for kind in ("K", "V"):
            grown = np.full((m, self.num_key_value_heads), -1, dtype=np.int32)
            grown[:n] = self._map[kind][lid]
            self._map[kind][lid] = grown
        self._fill[lid] = np.concatenate([self._fill[lid], np.zeros(m - n, dtype=np.int32)])
        self._final[lid] = np.concatenate([self._final[lid], np.zeros(m - n, dtype=bool)])
        self._start[lid] = np.concatenate([self._start[lid], np.full(m - n, -1, dtype=np.int64)])

    def _release(self, lid: int, block_id: int) -> None:
        for kind in ("K", "V"):
            ids = self._map[kind][lid][block_id]
            live = ids[ids >= 0]
            if len(live):
                self._pools[kind].free(live)
            ids[:] = -1
        self._fill[lid][block_id] = 0
        self._final[lid][block_id] = False
        self._start[lid][block_id] = -1
        self._rows[lid].pop(block_id, None)
        self._dev_map[lid] = None

    # ---- the serving interface -------------------------------------------------
    def write_slots(self, layer_id: int, key_rows, value_rows, slot_mapping, *, token_start: int | None = None) -> None:
        """Write ``[n, H, hd]`` rows to ``slot_mapping[i] = block * block_size
        + offset``.  Within a block, slots are written in order from its
        fill (a block whose offset 0 is written again starts over).  A block
        whose last slot is written is finalised.  ``token_start`` (optional)
        is the absolute position of row 0, kept for page headers."""
        torch = _torch()
        lid = self._check_layer(layer_id)
        keys = self._as_rows(key_rows, "key_rows")
        values = self._as_rows(value_rows, "value_rows")
        if keys.shape[0] != values.shape[0]:
            raise ValueError("key_rows and value_rows must hold the same number of tokens")
        slots = np.asarray(slot_mapping.detach().cpu().numpy() if isinstance(slot_mapping, torch.Tensor) else slot_mapping,
                           dtype=np.int64).reshape(-1)
        if slots.shape[0] != keys.shape[0]:
            raise ValueError("slot_mapping needs one slot per row")
        if np.any(slots < 0):
            raise ValueError("slots must be non-negative")
        P, H, hd = self.block_size, self.num_key_value_heads, self.config.head_dim
        i = 0
        n = slots.shape[0]
        while i < n:  # runs of consecutive slots of one block
            blk, off = int(slots[i] // P), int(slots[i] % P)
            j = i + 1
            while j < n and slots[j] == slots[j - 1] + 1 and slots[j] // P == blk:
                j += 1
            self._grow(lid, blk)
            if off == 0 and self._fill[lid][blk] > 0:
                self._release(lid, blk)  # a block id reused from its first slot
            if off != self._fill[lid][blk]:
                raise ValueError(f"block {blk} holds {int(self._fill[lid][blk])} tokens; slot offset {off} is out of order")
            self._write_run(lid, blk, off, keys[i:j], values[i:j], None if token_start is None else int(token_start) + i)
            i = j

    def _write_run(self, lid: int, blk: int, off: int, keys, values, start: int | None) -> None:
        torch = _torch()
        P, H, hd = self.block_size, self.num_key_value_heads, self.config.head_dim
        m = int(keys.shape[0])
        if self._final[lid][blk]:
            raise ValueError(f"block {blk} is full")
        if blk not in self._rows[lid]:
            self._rows[lid][blk] = torch.zeros((2, H, P, hd), dtype=torch.float32, device=self.device)
            for kind in ("K", "V"):
                self._map[kind][lid][blk] = self._pools[kind].allocate(*self._live_fmt[kind], H, tokens=0)
            self._dev_map[lid] = None
        if off == 0:
            self._start[lid][blk] = -1 if start is None else start
        rows = self._rows[lid][blk]
        for k, (kind, x) in enumerate((("K", keys), ("V", values))):
            xt = x.transpose(0, 1)  # [H, m, hd]
            rows[k, :, off:off + m].copy_(xt)
            ids = self._map[kind][lid][blk]
            self._pools[kind].encode_rows(xt.reshape(H * m, hd), np.repeat(ids, m), np.tile(np.arange(off, off + m), H))
            self._pools[kind].set_tokens(ids, off + m)
        self._fill[lid][blk] = off + m
        if off + m == P:
            self._finalise(lid, blk)

    def _finalise(self, lid: int, blk: int) -> None:
        P, H, hd = self.block_size, self.num_key_value_heads, self.config.head_dim
        rows = self._rows[lid].pop(blk)
        for k, kind in enumerate(("K", "V")):
            pool = self._pools[kind]
            old = self._map[kind][lid][blk].copy()
            new = np.empty(H, dtype=np.int32)
            for h in range(H):
                new[h] = pool.allocate(*self._page_format(kind, lid, h), 1, tokens=P)[0]
            pool.encode_rows(rows[k].reshape(H * P, hd), np.repeat(new, P), np.tile(np.arange(P), H))
            pool.free(old)
            self._map[kind][lid][blk] = new
        self._final[lid][blk] = True
        self._dev_map[lid] = None

    def decode_block_tables(self, layer_id: int, queries, block_tables, context_lens, q_head_to_kv_head=None, *,
                            query_scale: float = 1.0):
        """Attention of ``queries [B, Hq, hd]`` over sequences given as
        ``block_tables [B, W]`` block ids and ``context_lens [B]``: one
        decode launch for the batch.  Block b of a sequence holds tokens
        ``[b * block_size, ...)``; its token count is the block's fill."""
        torch = _torch()
        lid = self._check_layer(layer_id)
        B, Hq, H, hd, P = None, self.num_attention_heads, self.num_key_value_heads, self.config.head_dim, self.block_size
        q = queries if isinstance(queries, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(np.asarray(queries, dtype=np.float32)))
        q = q.to(self.device)
        if q.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            q = q.float()
        B = int(q.shape[0])
        if q.dim() != 3 or tuple(q.shape[1:]) != (Hq, hd):
            raise ValueError(f"queries must have shape [batch, {Hq}, {hd}]")
        lens = np.asarray(context_lens.detach().cpu().numpy() if isinstance(context_lens, torch.Tensor) else context_lens,
                          dtype=np.int64).reshape(-1)
        if lens.shape != (B,) or np.any(lens <= 0):
            raise ValueError("context_lens needs one positive length per sequence")
        bt = block_tables if isinstance(block_tables, torch.Tensor) else torch.from_numpy(np.asarray(block_tables, dtype=np.int64))
        if bt.dim() != 2 or bt.shape[0] != B:
            raise ValueError("block_tables must have shape [batch, max_blocks]")
        n_blocks = -(-lens // P)
        if np.any(n_blocks > bt.shape[1]):
            raise ValueError("a context length needs more blocks than its block-table row holds")
        bt_host = bt.detach().cpu().numpy().astype(np.int64)
        nmap = self._fill[lid].shape[0]
        for b in range(B):
            used = bt_host[b, : n_blocks[b]]
            if np.any(used < 0) or np.any(used >= nmap) or np.any(self._map["K"][lid][np.clip(used, 0, nmap - 1), 0] < 0):
                raise ValueError(f"sequence {b} names a block with no pages in layer {lid}")
            if int(self._fill[lid][used].sum()) != int(lens[b]):
                raise ValueError(f"sequence {b}: its blocks hold {int(self._fill[lid][used].sum())} tokens, context_lens says {int(lens[b])}")
        if self._dev_map[lid] is None:
            self._dev_map[lid] = tuple(torch.from_numpy(self._map[kind][lid].astype(np.int32)).to(self.device) for kind in ("K", "V"))
        idx = torch.from_numpy(np.clip(bt_host, 0, nmap - 1)).to(self.device)
        k_table = self._dev_map[lid][0][idx].permute(0, 2, 1).contiguous()  # [B, H, W] page ids
        v_table = self._dev_map[lid][1][idx].permute(0, 2, 1).contiguous()
        qmap = self.default_q_head_to_kv_head if q_head_to_kv_head is None else np.asarray(q_head_to_kv_head, dtype=np.int64)
        if qmap.shape != (Hq,) or np.any(qmap < 0) or np.any(qmap >= H) or np.any(np.bincount(qmap, minlength=H) != Hq // H):
            raise ValueError("q_head_to_kv_head must give every KV head the same number of query heads")
        order = np.argsort(qmap, kind="stable")
        contiguous = np.array_equal(order, np.arange(Hq))
        order_t = torch.from_numpy(order).to(self.device)
        qg = (q if contiguous else q[:, order_t]).reshape(B, H, Hq // H, hd)
        seq_pages = n_blocks.astype(np.int32)
        last_tokens = np.asarray([self._fill[lid][bt_host[b, n_blocks[b] - 1]] for b in range(B)], dtype=np.int32)
        # (a sequence's live block is an fp16 page: the split-K merge attends
        # it, and the decode launch takes the instance of the full blocks)
        kt = self._map["K"][lid][np.clip(bt_host, 0, nmap - 1)].transpose(0, 2, 1)
        vt = self._map["V"][lid][np.clip(bt_host, 0, nmap - 1)].transpose(0, 2, 1)
        plan, masks = plan_decode(self.k_pool, self.v_pool, kt, vt, seq_pages, Hq // H, device=self.device,
                                  last_page_tokens=last_tokens)
        need = workspace_bytes(plan, Hq // H, hd)
        if self._workspace is None or self._workspace.numel() < need:
            self._workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=self.device)
        out = decode_paged(self.k_pool, k_table, v_table, seq_pages, qg, query_scale=query_scale, plan=plan,
                           workspace=self._workspace, validate=False, v_pool=self.v_pool,
                           page_masks=masks).reshape(B, Hq, hd)
        if contiguous:
            return out
        res = torch.empty_like(out)
        res[:, order_t] = out
        return res

    # ---- the reference's single-sequence interface --------------------------
    def sync_layer_blocks(self, layer_id: int, key_blocks, value_blocks, *, block_ids=None,
                          live_block_token_count: int = 0) -> None:
        """Replace layer ``layer_id`` with ``[H, n_blocks, block_size, hd]``
        blocks (reference ``block_cache.py:152-301``): all full, or the last
        one live with ``live_block_token_count`` tokens."""
        torch = _torch()
        lid = self._check_layer(layer_id)
        P, H, hd = self.block_size, self.num_key_value_heads, self.config.head_dim
        kb = [key_blocks, value_blocks]
        for i, x in enumerate(kb):
            t = x if isinstance(x, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(np.asarray(x, dtype=np.float32)))
            t = t.to(device=self.device, dtype=torch.float32)
            if t.dim() == 5:
                if t.shape[0] != 1:
                    raise ValueError("batch dimension must be 1")
                t = t[0]
            if t.dim() != 4 or t.shape[0] != H or t.shape[2] != P or t.shape[3] != hd:
                raise ValueError(f"{'key' if i == 0 else 'value'}_blocks must have shape [kv_heads, block_count, block_size, head_dim]")
            kb[i] = t
        keys, values = kb
        if keys.shape[1] != values.shape[1]:
            raise ValueError("key_blocks and value_blocks must contain the same number of blocks")
        n = int(keys.shape[1])
        ids = list(range(n)) if block_ids is None else [int(b) for b in block_ids]
        if len(ids) != n:
            raise ValueError("block_ids must align with the number of blocks")
        if len(set(ids)) != n:
            raise ValueError("block_ids must be unique")
        if not 0 <= int(live_block_token_count) <= P:
            raise ValueError("live_block_token_count must be in [0, block_size]")
        self.clear_layer(lid)
        live = int(live_block_token_count)
        finalised = n if live in (0, P) else n - 1
        for i, blk in enumerate(ids):
            cnt = P if i < finalised else live
            slots = blk * P + np.arange(cnt)
            self.write_slots(lid, keys[:, i, :cnt].transpose(0, 1), values[:, i, :cnt].transpose(0, 1), slots,
                             token_start=i * P)
        self._seq_blocks[lid] = ids
        self._seq_len[lid] = finalised * P + (live if finalised < n else 0)

    def append_step(self, layer_id: int, key_step, value_step, token_index: int) -> None:
        """Append ``[H, n, hd]`` rows at ``token_index`` (the cached length);
        token t goes to block ``t // block_size`` (reference
        ``block_cache.py:303-325``, ``:456-517``)."""
        torch = _torch()
        lid = self._check_layer(layer_id)
        rows = []
        for name, x in (("key_step", key_step), ("value_step", value_step)):
            t = x if isinstance(x, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(np.asarray(x, dtype=np.float32)))
            t = t.to(device=self.device, dtype=torch.float32)
            if t.dim() == 4:
                if t.shape[0] != 1:
                    raise ValueError(f"{name} batch dimension must be 1")
                t = t[0]
            if t.dim() != 3 or t.shape[0] != self.num_key_value_heads or t.shape[2] != self.config.head_dim:
                raise ValueError(f"{name} must have shape [kv_heads, token_count, head_dim]")
            rows.append(t)
        if rows[0].shape[1] != rows[1].shape[1]:
            raise ValueError("key_step and value_step token counts must match")
        if int(token_index) != int(self._seq_len[lid]):
            raise ValueError(f"layer {lid} expected token_index {int(self._seq_len[lid])}, received {token_index}")
        n = int(rows[0].shape[1])
        pos = int(token_index) + np.arange(n)
        seq = self._seq_blocks[lid]
        live = seq[-1] if seq and self._fill[lid][seq[-1]] < self.block_size else None
        for blk in np.unique(pos // self.block_size).tolist():
            if blk == live:
                continue
            if blk in seq:
                raise ValueError(f"token {int(pos[0])} maps to block {blk}, which already holds earlier tokens of layer {lid}")
            seq.append(blk)
        self.write_slots(lid, rows[0].transpose(0, 1), rows[1].transpose(0, 1), pos, token_start=int(token_index))
        self._seq_len[lid] += n

    append_step_torch = append_step

    def append_tokens_torch(self, layer_id: int, key_rows, value_rows, token_positions) -> None:
        """``[n, H, hd]`` rows at contiguous positions, appended in chunks
        that end on block boundaries (reference ``block_cache.py:420-454``)."""
        torch = _torch()
        pos = token_positions.reshape(-1).detach().cpu().numpy().astype(np.int64) if isinstance(token_positions, torch.Tensor) \
            else np.asarray(token_positions, dtype=np.int64).reshape(-1)
        if pos.size == 0:
            return
        if not np.array_equal(pos, np.arange(int(pos[0]), int(pos[0]) + pos.size)):
            raise ValueError("token positions must be contiguous (one sequence)")
        k = self._as_rows(key_rows, "key_rows").transpose(0, 1)
        v = self._as_rows(value_rows, "value_rows").transpose(0, 1)
        off = 0
        while off < pos.size:
            t = int(pos[off])
            m = min(self.block_size - t % self.block_size, pos.size - off)
            self.append_step(layer_id, k[:, off:off + m], v[:, off:off + m], t)
            off += m

    def decode_layer_torch(self, layer_id: int, query_step, q_head_to_kv_head=None, *, query_scale: float = 1.0):
        """The layer's sequence (its blocks in token order) decoded for
        ``query_step [Hq, hd]``; fp32 ``[Hq, hd]`` on the device (reference
        ``block_cache.py:519-551``)."""
        torch = _torch()
        lid = self._check_layer(layer_id)
        if self._seq_len[lid] == 0:
            raise ValueError(f"layer {lid} has no cached tokens to decode against")
        q = query_step if isinstance(query_step, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(np.asarray(query_step, dtype=np.float32)))
        table = np.asarray(self._seq_blocks[lid], dtype=np.int64)[None]
        return self.decode_block_tables(lid, q.reshape(1, *q.shape[-2:]), table, [int(self._seq_len[lid])],
                                        q_head_to_kv_head, query_scale=query_scale)[0]

    def decode_layer(self, layer_id: int, query_step, q_head_to_kv_head=None, *, query_scale: float = 1.0) -> np.ndarray:
        return self.decode_layer_torch(layer_id, query_step, q_head_to_kv_head, query_scale=query_scale).cpu().numpy()

    # ---- entries and bookkeeping ----------------------------------------------
    def block_entry(self, layer_id: int, kv_head_id: int, block_id: int, kind: str) -> VllmBlockEntry:
        """The page of one (layer, KV head, block), read back from the device."""
        lid, h, blk = self._check_layer(layer_id), int(kv_head_id), int(block_id)
        if kind not in ("K", "V"):
            raise ValueError("kind must be K or V")
        if blk >= self._fill[lid].shape[0] or self._map[kind][lid][blk, h] < 0:
            raise KeyError(VllmBlockKey(lid, h, blk, kind))
        pool = self._pools[kind]
        pid = int(self._map[kind][lid][blk, h])
        header = pool.header_of(pid, kind)
        start = int(self._start[lid][blk])
        header.layer_id, header.kv_head_id, header.token_start = lid, h, max(start, 0)
        page = pool.download_page(pid, header, kind=kind)
        return VllmBlockEntry(key=VllmBlockKey(lid, h, blk, kind), page=page, finalized=bool(self._final[lid][blk]),
                              token_count=int(self._fill[lid][blk]), token_start=max(start, 0))

    def block_entries_for_layer(self, layer_id: int, *, kind: str) -> list[VllmBlockEntry]:
        lid = self._check_layer(layer_id)
        blocks = np.flatnonzero(self._fill[lid] > 0).tolist()
        return [self.block_entry(lid, h, b, kind) for h in range(self.num_key_value_heads) for b in blocks]

    def clear_layer(self, layer_id: int) -> None:
        lid = self._check_layer(layer_id)
        for blk in np.flatnonzero((self._map["K"][lid][:, 0] >= 0) | (self._fill[lid] > 0)).tolist():
            self._release(lid, blk)
        self._seq_blocks[lid] = []
        self._seq_len[lid] = 0

    def clear(self) -> None:
        for lid in range(self.num_hidden_layers):
            self.clear_layer(lid)

    @property
    def resident_bytes(self) -> int:
        """Bytes of every block's pages (valid tokens only)."""
        total = 0
        for lid in range(self.num_hidden_layers):
            for kind in ("K", "V"):
                ids = self._map[kind][lid]
                total += self._pools[kind].read_bytes(ids[ids >= 0])
        return total


__all__ = ["DeviceVllmPagedKVCache", "VllmBlockEntry", "VllmBlockKey"]
