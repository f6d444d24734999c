"""Device-resident paged KV cache of a decoder: prefill ingest, per-step
append into an exact tail page, page finalise and decode, all on the GPU.

MI355X counterpart of the reference's ``ModelPagedKVCache`` lifecycle
(reference ``dotcache/model_kv_cache.py:3609-3691`` ingest_prefill_cache,
``:3830-3902`` append_step with the tail builder of ``:718-880``,
``:4099-4134`` decode_layer).  The reference keeps the tail rows on the
host (or in a torch tail page) and encodes a full page with numpy after a
device-to-host copy.  Here every (layer, sequence, KV head) stream owns:

* its finalised pages: ids in a :class:`~dotcache_amd.page_pool.DevicePagePool`
  (one pool for keys, one for values), encoded on the device by
  ``dc_encode_rows``;
* a tail page in the escape format (M3), written row by row as tokens
  arrive, which decode attends like any other page;
* the tail's rows in fp32 on the device, from which the full page is
  encoded when the tail fills -- so a finalised page is bit-identical to
  the reference's ``encode_page`` of the same fp32 rows
  (``model_kv_cache.py:788-830``).

Page modes are chosen as the reference's numpy cache chooses them.  A kind
without mode or policy overrides takes ``DotCacheConfig.resolve_page_mode``.
A kind with any override takes ``choose_page_mode`` under the stream's layer
policy (reference ``model_kv_cache.py:3164-3185`` for prefill pages,
``:789-810`` for pages finalised by ``append_step``), with the token age
``sequence_length - token_start - 1`` of the page: young pages of a tier
policy become M3 (the recent window), and the header fields
``policy_id`` / ``sensitivity_tier`` / ``fallback_reason`` / ``age_bucket``
record the choice.  Page statistics (``observe_page``) are computed on the
device, only when a candidate needs them.  Several sequences
(``batch_size``) share the pools and decode in one launch per layer.
"""
from __future__ import annotations

import numpy as np

from .config import DotCacheConfig, observe_page
from .decode import decode_paged, plan_decode, workspace_bytes
from .encode import make_header, resolve_encode_spec
from .page_pool import DevicePagePool, PoolGeometry, page_format_of


def _torch():
    import torch

    return torch


def default_q_head_to_kv_head(num_attention_heads: int, num_key_value_heads: int) -> np.ndarray:
    """Query head q reads KV head ``q // (Hq / Hkv)`` (reference
    ``model_kv_cache.py:85-95``)."""
    if num_attention_heads % num_key_value_heads:
        raise ValueError("num_attention_heads must be a multiple of num_key_value_heads")
    group = num_attention_heads // num_key_value_heads
    return np.arange(num_attention_heads, dtype=np.int64) // group


class DevicePagedKVCache:
    """Paged, compressed KV cache of ``num_hidden_layers`` layers for
    ``batch_size`` sequences, resident in HBM.

    Tensors passed in may be numpy arrays or torch tensors (fp32, fp16 or
    bf16); they are read as fp32.  Shapes carry a leading batch dimension
    when ``batch_size > 1``, as in the reference's ``[1, heads, tokens,
    head_dim]`` with batch 1.
    """

    def __init__(self, config: DotCacheConfig, *, num_hidden_layers: int, num_attention_heads: int,
                 num_key_value_heads: int, batch_size: int = 1, device="cuda",
                 reserve_pages_per_stream: int = 16):
        torch = _torch()
        if num_hidden_layers <= 0 or num_key_value_heads <= 0 or batch_size <= 0:
            raise ValueError("num_hidden_layers, num_key_value_heads and batch_size must be positive")
        q_map = default_q_head_to_kv_head(num_attention_heads, num_key_value_heads)
        if num_attention_heads // num_key_value_heads > 16:
            raise ValueError("at most 16 query heads per KV head")
        self.config = config
        self.num_hidden_layers = int(num_hidden_layers)
        self.num_attention_heads = int(num_attention_heads)
        self.num_key_value_heads = int(num_key_value_heads)
        self.batch_size = int(batch_size)
        self.device = torch.device(device)
        self.q_head_to_kv_head = q_map
        L, B, H, P, hd = self.num_hidden_layers, self.batch_size, self.num_key_value_heads, config.tokens_per_page, config.head_dim
        self._specs = {kind: resolve_encode_spec(config, kind=kind) for kind in ("K", "V")}
        self._tail_fmt = {kind: page_format_of("M3", "affine", 4, self._specs[kind]["escape_dtype"]) for kind in ("K", "V")}
        streams = L * B * H
        pools = {}
        for kind in ("K", "V"):
            geo = PoolGeometry(hd, config.group_size, P, self._specs[kind]["layout"])
            probe = DevicePagePool(geo, device=self.device, reserve_bytes=256, reserve_pages=16)
            per_stream = reserve_pages_per_stream * max(probe.blob_bytes(*self._page_format(kind, 0, 0)),
                                                        probe.blob_bytes(*self._tail_fmt[kind]))
            pools[kind] = DevicePagePool(geo, device=self.device, reserve_bytes=streams * per_stream + (1 << 20),
                                         reserve_pages=streams * (reserve_pages_per_stream + 1))
        self.k_pool, self.v_pool = pools["K"], pools["V"]
        # finalised page ids per (layer, sequence, head); the tail page of each stream
        self._pages = {kind: [[[[] for _ in range(H)] for _ in range(B)] for _ in range(L)] for kind in ("K", "V")}
        self._tail_page = {kind: np.full((L, B, H), -1, dtype=np.int64) for kind in ("K", "V")}
        self._tail_rows = {kind: torch.zeros((L, B, H, P, hd), dtype=torch.float32, device=self.device)
                           for kind in ("K", "V")}
        self._seq_len = np.zeros((L, B), dtype=np.int64)    # tokens cached per (layer, sequence)
        self._tail_start = np.zeros((L, B), dtype=np.int64)  # absolute index of each tail's first token
        self._tables = [None] * L  # (k_table, v_table, seq_pages) on the device, rebuilt when pages change
        self._host_tables = [None] * L  # the same tables on the host
        self._spec_memo: dict = {}
        self._workspace = None

    # ---- formats -----------------------------------------------------------
    def _page_format(self, kind: str, layer_id: int, kv_head_id: int) -> tuple[int, int]:
        spec = self._specs[kind]
        mode = self.config.resolve_page_mode(kind=kind, layer_id=layer_id, kv_head_id=kv_head_id)
        return page_format_of(mode, spec["scheme"], spec["bits"], spec["escape_dtype"])

    def _page_spec(self, kind: str, layer_id: int, kv_head_id: int, token_start: int, sequence_length: int,
                   rows) -> dict:
        """Encode spec (mode, bits, scheme, escape dtype, policy header
        fields) of one full page whose fp32 device rows are ``rows [P, hd]``:
        ``choose_page_mode`` when the kind has overrides, else the layer's
        resolved mode (reference ``model_kv_cache.py:3164-3185``)."""
        cfg = self.config
        if not cfg.chooses_page_modes(kind):  # the mode depends on (kind, layer, head) only
            key = (kind, int(layer_id), int(kv_head_id))
            hit = self._spec_memo.get(key)
            if hit is None:
                mode = cfg.resolve_page_mode(kind=kind, layer_id=layer_id, kv_head_id=kv_head_id)
                hit = self._spec_memo[key] = resolve_encode_spec(cfg, kind=kind, mode=mode)
            return hit
        chosen = cfg.select_page_mode(kind=kind, layer_id=layer_id, kv_head_id=kv_head_id, token_start=token_start,
                                      sequence_length=sequence_length, stats=lambda: observe_page(rows))
        if chosen.mode not in ("M0", "M3"):
            raise ValueError(f"the {kind} page policy of layer {layer_id} chose mode {chosen.mode} "
                             f"(token_start {token_start}), which hip_mi355x does not encode")
        return resolve_encode_spec(cfg, kind=kind, page_mode=chosen)

    def _pool(self, kind: str) -> DevicePagePool:
        return self.k_pool if kind == "K" else self.v_pool

    # ---- input normalisation ------------------------------------------------
    def _rows(self, x, *, tokens: int | None, name: str):
        """``x`` as fp32 device ``[B, H, T, hd]``."""
        torch = _torch()
        t = x if isinstance(x, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(np.asarray(x, dtype=np.float32)))
        t = t.to(device=self.device, dtype=torch.float32)
        if t.dim() == 3 and self.batch_size == 1:
            t = t.unsqueeze(0)
        B, H, hd = self.batch_size, self.num_key_value_heads, self.config.head_dim
        if t.dim() != 4 or t.shape[0] != B or t.shape[1] != H or t.shape[3] != hd:
            raise ValueError(f"{name} must have shape [{B}, {H}, tokens, {hd}]" + (" or [H, tokens, head_dim]" if B == 1 else ""))
        if tokens is not None and t.shape[2] != tokens:
            raise ValueError(f"{name} must hold {tokens} tokens")
        return t

    def _check_layer(self, layer_id: int) -> int:
        lid = int(layer_id)
        if not 0 <= lid < self.num_hidden_layers:
            raise ValueError(f"layer_id {layer_id} out of range")
        return lid

    # ---- writes ------------------------------------------------------------
    def _encode(self, kind: str, rows, page_ids: np.ndarray, slots: np.ndarray) -> None:
        if len(page_ids):
            self._pool(kind).encode_rows(rows, page_ids.astype(np.int32), slots.astype(np.int32))

    def _finalise_pages(self, kind: str, layer_id: int, rows, token_stream: np.ndarray, token_starts: np.ndarray,
                        sequence_lengths: np.ndarray) -> None:
        """Encode full pages: ``rows [n_pages * P, hd]`` fp32, page i of
        stream ``token_stream[i]`` (index b * H + h) starting at absolute
        token ``token_starts[i]`` of a context of ``sequence_lengths[i]``
        tokens (the page-mode choice reads both)."""
        P, H = self.config.tokens_per_page, self.num_key_value_heads
        pool = self._pool(kind)
        n = len(token_stream)
        specs = [self._page_spec(kind, layer_id, int(s) % H, int(t0), int(sl), rows[i * P:(i + 1) * P])
                 for i, (s, t0, sl) in enumerate(zip(token_stream, token_starts, sequence_lengths))]
        fmts = [page_format_of(sp["mode"], sp["scheme"], sp["bits"], sp["escape_dtype"]) for sp in specs]
        ids = np.empty(n, dtype=np.int64)
        for fmt_bits in set(fmts):
            sel = [i for i in range(n) if fmts[i] == fmt_bits]
            ids[sel] = pool.allocate(*fmt_bits, len(sel), tokens=P)
        self._encode(kind, rows, np.repeat(ids, P), np.tile(np.arange(P), n))
        for i, (pid, s) in enumerate(zip(ids.tolist(), token_stream.tolist())):
            self._pages[kind][layer_id][s // H][s % H].append(pid)
            pool.headers[pid] = make_header(self.config, specs[i], kind=kind, layer_id=layer_id, kv_head_id=s % H,
                                            token_start=int(token_starts[i]), token_count=P)

    def _write_tail(self, kind: str, layer_id: int, rows, first_slot: int) -> None:
        """Rows ``[B, H, n, hd]`` into tail slots ``first_slot ..`` of every
        stream of the layer (fp32 copy and escape page)."""
        B, H, n = int(rows.shape[0]), int(rows.shape[1]), int(rows.shape[2])
        if n == 0:
            return
        tp = self._tail_page[kind][layer_id]
        pool = self._pool(kind)
        missing = np.argwhere(tp < 0)
        if len(missing):
            ids = pool.allocate(*self._tail_fmt[kind], len(missing), tokens=0)
            tp[missing[:, 0], missing[:, 1]] = ids
        self._tail_rows[kind][layer_id, :, :, first_slot: first_slot + n].copy_(rows)
        flat = rows.reshape(B * H * n, -1)
        page_ids = np.repeat(tp.reshape(-1), n)
        slots = np.tile(np.arange(first_slot, first_slot + n), B * H)
        self._encode(kind, flat, page_ids, slots)
        pool.set_tokens(tp.reshape(-1), first_slot + n)

    # ---- the reference's entry points ---------------------------------------
    def ingest_prefill_cache(self, layer_id: int, layer_k, layer_v, *, context_length: int | None = None) -> None:
        """Store a prefill's K/V ``[B, H, T, hd]`` for layer ``layer_id``:
        full pages are encoded on the device, the remaining ``T % P`` rows
        become the tail (reference ``model_kv_cache.py:3609-3691``)."""
        lid = self._check_layer(layer_id)
        keys = self._rows(layer_k, tokens=None, name="layer_k")
        values = self._rows(layer_v, tokens=int(keys.shape[2]), name="layer_v")
        T = int(keys.shape[2])
        ctx = T if context_length is None else int(context_length)
        if ctx < T:
            raise ValueError("context_length must be at least the stored prefill cache length")
        self.clear_layer(lid)
        B, H, P, hd = self.batch_size, self.num_key_value_heads, self.config.tokens_per_page, self.config.head_dim
        full = (T // P) * P
        if full:
            # page-major rows: stream (b, h), page i, slot j; page i starts at
            # absolute token ctx - T + i P of a ctx-token context
            streams = np.repeat(np.arange(B * H), full // P)
            starts = np.tile((ctx - T) + P * np.arange(full // P), B * H)
            for kind, x in (("K", keys), ("V", values)):
                self._finalise_pages(kind, lid, x[:, :, :full].reshape(B * H * full, hd), streams, starts,
                                     np.full(len(streams), ctx))
        for kind, x in (("K", keys), ("V", values)):
            self._write_tail(kind, lid, x[:, :, full:], 0)
        self._seq_len[lid, :] = ctx
        self._tail_start[lid, :] = ctx - T + full
        self._tables[lid] = None

    def append_step(self, layer_id: int, key_step, value_step, token_index: int) -> None:
        """Append ``[B, H, n, hd]`` new rows at absolute position
        ``token_index`` (which must equal the cached length); each tail that
        fills is encoded into a page of the layer's mode and reset
        (reference ``model_kv_cache.py:3830-3902`` and ``:756-830``)."""
        lid = self._check_layer(layer_id)
        keys = self._rows(key_step, tokens=None, name="key_step")
        values = self._rows(value_step, tokens=int(keys.shape[2]), name="value_step")
        if np.any(self._seq_len[lid] != int(token_index)):
            raise ValueError(f"layer {lid} expected token_index {int(self._seq_len[lid, 0])}, received {token_index}")
        B, H, P, hd = self.batch_size, self.num_key_value_heads, self.config.tokens_per_page, self.config.head_dim
        n = int(keys.shape[2])
        done = 0
        while done < n:
            fill = int(self._seq_len[lid, 0] - self._tail_start[lid, 0])
            take = min(P - fill, n - done)
            for kind, x in (("K", keys), ("V", values)):
                self._write_tail(kind, lid, x[:, :, done: done + take], fill)
            done += take
            self._seq_len[lid, :] += take
            if fill + take == P:  # every stream's tail is full: encode it into a page
                # the page's context is the whole step's (reference
                # model_kv_cache.py:3887-3892 passes token_index + n)
                streams = np.arange(B * H)
                starts = np.repeat(self._tail_start[lid], H)
                for kind in ("K", "V"):
                    rows = self._tail_rows[kind][lid].reshape(B * H * P, hd)
                    self._finalise_pages(kind, lid, rows, streams, starts, np.full(B * H, int(token_index) + n))
                    self._pool(kind).set_tokens(self._tail_page[kind][lid].reshape(-1), 0)
                self._tail_start[lid, :] = self._seq_len[lid, :]
            self._tables[lid] = None

    def decode_layer(self, layer_id: int, query_step, q_head_to_kv_head=None, *, query_scale: float = 1.0):
        """Attention of ``query_step [B, Hq, hd]`` over layer ``layer_id``'s
        cached tokens (pages + tail); query head q reads KV head
        ``q_head_to_kv_head[q]`` (default ``q // (Hq / Hkv)``), every KV head
        serving the same number of query heads.  Returns fp32 ``[B, Hq, hd]``
        on the device (reference ``model_kv_cache.py:4099-4134``)."""
        torch = _torch()
        lid = self._check_layer(layer_id)
        q = query_step if isinstance(query_step, torch.Tensor) else torch.from_numpy(
            np.ascontiguousarray(np.asarray(query_step, dtype=np.float32)))
        q = q.to(self.device)
        if q.dim() == 2 and self.batch_size == 1:
            q = q.unsqueeze(0)
        B, Hq, H, hd = self.batch_size, self.num_attention_heads, self.num_key_value_heads, self.config.head_dim
        if q.dim() != 3 or tuple(q.shape) != (B, Hq, hd):
            raise ValueError(f"query_step must have shape [{B}, {Hq}, {hd}]")
        if q.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            q = q.float()
        if np.any(self._seq_len[lid] == 0):
            raise ValueError(f"layer {lid} has no cached tokens to decode against")
        qmap = self.q_head_to_kv_head if q_head_to_kv_head is None else np.asarray(q_head_to_kv_head, dtype=np.int64)
        if qmap.shape != (Hq,) or np.any(qmap < 0) or np.any(qmap >= H):
            raise ValueError(f"q_head_to_kv_head must map {Hq} query heads to KV heads in [0, {H})")
        if np.any(np.bincount(qmap, minlength=H) != Hq // H):
            raise ValueError("every KV head must serve the same number of query heads")
        order = np.argsort(qmap, kind="stable")  # query heads grouped by KV head
        contiguous = np.array_equal(order, np.arange(Hq))
        k_table, v_table, seq_pages, last_tokens = self._layer_tables(lid)
        kt, vt = self._host_tables[lid]
        qg = q if contiguous else q[:, torch.from_numpy(order).to(self.device)]
        queries = qg.reshape(B, H, Hq // H, hd)
        # The fp16 tail page (and any young exact pages right before it) is
        # attended by the split-K merge, so the decode launch takes the kernel
        # instance of the other pages' formats (region plan, merge windows).
        plan, masks = plan_decode(self.k_pool, self.v_pool, kt, vt, seq_pages, Hq // H, device=self.device,
                                  last_page_tokens=last_tokens)
        need = workspace_bytes(plan, Hq // H, hd)
        if self._workspace is None or self._workspace.numel() < need:
            self._workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=self.device)
        out = decode_paged(self.k_pool, k_table, v_table, seq_pages, queries, query_scale=query_scale, plan=plan,
                           workspace=self._workspace, validate=False, v_pool=self.v_pool, page_masks=masks)
        out = out.reshape(B, Hq, hd)
        if contiguous:
            return out
        res = torch.empty_like(out)
        res[:, torch.from_numpy(order).to(self.device)] = out
        return res

    # ---- bookkeeping -------------------------------------------------------
    def _layer_tables(self, lid: int):
        """Device page tables of a layer (each stream's pages, then its tail
        page when the tail holds tokens), the page counts and the tokens in
        each sequence's last page."""
        torch = _torch()
        if self._tables[lid] is None:
            B, H = self.batch_size, self.num_key_value_heads
            has_tail = (self._seq_len[lid] - self._tail_start[lid]) > 0
            counts = np.array([len(self._pages["K"][lid][b][0]) + int(has_tail[b]) for b in range(B)], dtype=np.int32)
            stride = max(int(counts.max()), 1)
            tabs, host = {}, {}
            for kind in ("K", "V"):
                t = np.zeros((B, H, stride), dtype=np.int32)
                for b in range(B):
                    for h in range(H):
                        ids = self._pages[kind][lid][b][h] + ([int(self._tail_page[kind][lid, b, h])] if has_tail[b] else [])
                        t[b, h, : len(ids)] = ids
                tabs[kind] = torch.from_numpy(t).to(self.device)
                host[kind] = t
                if kind == "K":
                    last = self.k_pool.tokens_of(t[np.arange(B), 0, np.maximum(counts - 1, 0)]).astype(np.int32)
            self._tables[lid] = (tabs["K"], tabs["V"], counts, last)
            self._host_tables[lid] = (host["K"], host["V"])
        return self._tables[lid]

    def clear_layer(self, layer_id: int) -> None:
        """Drop every cached token of a layer (pages are returned to the pools)."""
        lid = self._check_layer(layer_id)
        for kind in ("K", "V"):
            pool = self._pool(kind)
            for b in range(self.batch_size):
                for h in range(self.num_key_value_heads):
                    ids = self._pages[kind][lid][b][h]
                    if ids:
                        pool.free(ids)
                    self._pages[kind][lid][b][h] = []
            tp = self._tail_page[kind][lid]
            live = tp[tp >= 0]
            if len(live):
                pool.set_tokens(live, 0)
        self._seq_len[lid, :] = 0
        self._tail_start[lid, :] = 0
        self._tables[lid] = None

    def sequence_length(self, layer_id: int) -> int:
        return int(self._seq_len[self._check_layer(layer_id), 0])

    def page_ids(self, layer_id: int, sequence: int, kv_head_id: int, kind: str = "K") -> list[int]:
        """Finalised page ids of one stream, oldest first (the tail excluded)."""
        return list(self._pages[kind][self._check_layer(layer_id)][int(sequence)][int(kv_head_id)])

    def page(self, layer_id: int, sequence: int, kv_head_id: int, index: int, kind: str = "K"):
        """Finalised page ``index`` of one stream as a host ``EncodedPage``
        with the header the reference's cache gives it (token_start, mode
        and the policy fields)."""
        pid = self.page_ids(layer_id, sequence, kv_head_id, kind)[index]
        return self._pool(kind).download_page(pid, kind=kind)

    def tail_page_id(self, layer_id: int, sequence: int, kv_head_id: int, kind: str = "K") -> int:
        return int(self._tail_page[kind][self._check_layer(layer_id), int(sequence), int(kv_head_id)])

    def resident_bytes(self) -> int:
        """Compressed bytes a decode of every layer reads (pages + tails)."""
        total = 0
        for lid in range(self.num_hidden_layers):
            if self._seq_len[lid, 0] == 0:
                continue
            k_table, v_table, counts, _ = self._layer_tables(lid)
            kt, vt = k_table.cpu().numpy(), v_table.cpu().numpy()
            for b in range(self.batch_size):
                total += self.k_pool.read_bytes(kt[b, :, : counts[b]]) + self.v_pool.read_bytes(vt[b, :, : counts[b]])
        return total


__all__ = ["DevicePagedKVCache", "default_q_head_to_kv_head"]
