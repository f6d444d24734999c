"""Seeded synthetic decode workloads shaped like the BASELINE configurations.

Each workload builds, on the device, every layer's key and value pages
(encoded by the HIP encoder straight into device pools, no host round trip)
and per-layer ragged page tables whose page ids are a random permutation of
the pool, then exposes one decode step = one ``dc_decode_paged`` launch per
layer.  Data is synthetic (no checkpoints): K, V ~ N(0, 1) or Student-t
(df 4), optional fixed outlier channels per KV head scaled x16.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import _lib
from .config import PageModeSpec, choose_page_mode, make_explicit_policy
from .decode import (DecodePlan, chunks_per_page, decode_paged, gather_records, launch_lead_ratio, launch_target_items,
                     make_plan, make_region_plan, merge_partials, page_costs, workspace_bytes)
from .page_pool import DevicePagePool, PoolGeometry


def _torch():
    import torch

    return torch


@dataclass(frozen=True)
class PageFormat:
    mode: str              # "M0" or "M3"
    scheme: str = "affine"
    bits: int = 4
    group_size: int = 32

    @property
    def fmt(self) -> tuple[int, int]:
        if self.mode == "M3":
            return _lib.FMT_M3_F16, 0
        return (_lib.FMT_M0_AFFINE if self.scheme == "affine" else _lib.FMT_M0_SYMMETRIC), self.bits


@dataclass(frozen=True)
class WorkloadSpec:
    name: str
    n_layers: int
    n_q_heads: int
    n_kv_heads: int
    head_dim: int
    batch: int
    page_size: int
    key: PageFormat
    value: PageFormat
    context: int = 0                       # fixed context per sequence
    ragged: tuple[int, int] | None = None  # log-uniform [lo, hi] context lengths
    key_m3_fraction: float = 0.0           # sensitivity map: fraction of (layer, kv head) key streams kept M3
    recent_window: int = 0                 # newest tokens kept as fp16 (M3) pages
    outlier_channels: int = 0
    distribution: str = "normal"
    append: bool = False                   # per-step encode/append of the new token
    replicas: int = 1                      # independent KV sets cycled step by step (working set past the MALL)
    description: str = ""

    @property
    def gqa(self) -> int:
        return self.n_q_heads // self.n_kv_heads


SPECS = {
    "c1": WorkloadSpec("c1_cpu_plumbing", 1, 1, 1, 64, 1, 64, PageFormat("M0", "symmetric", 4, 32),
                       PageFormat("M0", "symmetric", 4, 32), context=1024,
                       description="1 layer, 1 q / 1 kv head, hd 64, 16 pages, M0 symmetric 4-bit g32"),
    "c2": WorkloadSpec("c2_llama32_1b", 16, 32, 8, 64, 1, 64, PageFormat("M0", "affine", 4, 32),
                       PageFormat("M0", "affine", 4, 32), context=4096, replicas=8,
                       description="Llama-3.2-1B-shaped: 16 L, 32 q / 8 kv, hd 64, ctx 4096, M0 affine 4-bit g32; "
                                   "8 KV sets (336 MB) cycled step by step, past the 256 MB MALL"),
    "c3": WorkloadSpec("c3_qwen25_7b_gqa", 28, 28, 4, 128, 8, 64, PageFormat("M3"),
                       PageFormat("M0", "symmetric", 4, 32), context=16384, outlier_channels=4,
                       description="Qwen2.5-7B-shaped: 28 L, 28 q / 4 kv (GQA 7), hd 128, batch 8 x 16384, "
                                   "K M3 fp16, V M0 symmetric 4-bit g32"),
    "c4": WorkloadSpec("c4_ragged_qwen25_1p5b", 28, 12, 2, 128, 64, 64, PageFormat("M0", "affine", 4, 32),
                       PageFormat("M0", "symmetric", 8, 64), ragged=(256, 32768), key_m3_fraction=0.12,
                       description="Qwen2.5-1.5B-shaped ragged batch of 64, log-uniform 256..32768, ~12% key "
                                   "streams M3, K M0 affine 4-bit g32, V M0 symmetric 8-bit g64"),
    "c5": WorkloadSpec("c5_qwen35_4b_long", 8, 16, 4, 256, 4, 128, PageFormat("M0", "affine", 4, 32),
                       PageFormat("M0", "affine", 4, 32), context=131072, recent_window=128,
                       distribution="student_t4", append=True,
                       description="Qwen3.5-4B-shaped full-attention layers: 8 L, 16 q / 4 kv, hd 256, batch 4 x "
                                   "131072, page 128, M0 affine 4-bit g32 + 128-token fp16 window, per-step append"),
}


def context_lengths(spec: WorkloadSpec, seed: int) -> np.ndarray:
    if spec.ragged is None:
        return np.full(spec.batch, spec.context, dtype=np.int64)
    rng = np.random.default_rng(seed)
    lo, hi = spec.ragged
    return np.exp(rng.uniform(np.log(lo), np.log(hi), size=spec.batch)).astype(np.int64)


def key_m3_map(spec: WorkloadSpec, seed: int) -> np.ndarray:
    """[n_layers, n_kv_heads] bool: key streams kept exact (selective key precision)."""
    if spec.key_m3_fraction <= 0:
        return np.zeros((spec.n_layers, spec.n_kv_heads), dtype=bool)
    rng = np.random.default_rng(seed + 17)
    return rng.random((spec.n_layers, spec.n_kv_heads)) < spec.key_m3_fraction


@dataclass
class LayerTables:
    k_table: object        # device int32 [B, H, stride]
    v_table: object
    seq_pages: np.ndarray  # [B]
    tail_k: np.ndarray | None = None  # [B, H] page ids receiving appended tokens
    tail_v: np.ndarray | None = None


@dataclass
class Workload:
    spec: WorkloadSpec
    seed: int
    lengths: np.ndarray
    k_pool: DevicePagePool
    v_pool: DevicePagePool
    layers: list[LayerTables]
    queries: list              # per layer [B, H, Q, hd] bf16
    new_k: list = field(default_factory=list)  # per layer [B*H, hd] rows to append
    new_v: list = field(default_factory=list)
    plan: DecodePlan | None = None  # layer 0's plan (every layer's when a split is given)
    plans: list = field(default_factory=list)  # per layer: items of near-equal cost under its page formats
    lead_ratios: list = field(default_factory=list)  # per layer: the plan's lead/trail ratio (None: plain)
    records: list = field(default_factory=list)  # per layer: page records of its plan (PageRecords)
    outs: list = field(default_factory=list)
    workspace: object = None
    k_page_ids_by_layer: list = field(default_factory=list)
    v_page_ids_by_layer: list = field(default_factory=list)
    attended: np.ndarray | None = None
    graph: object = None  # captured HIP graphs of one whole step, one per replica
    next_replica: int = 0
    tail_k_dev: list = field(default_factory=list)
    tail_v_dev: list = field(default_factory=list)
    slot_dev: object = None

    @property
    def query_scale(self) -> float:
        return 1.0 / float(np.sqrt(self.spec.head_dim))

    @property
    def replicas(self) -> int:
        return self.spec.replicas

    def replica_layers(self, r: int) -> range:
        """Layer indices of KV set ``r``: a step attends one set's layers."""
        L = self.spec.n_layers
        return range(r * L, (r + 1) * L)

    def algorithmic_bytes_per_step(self) -> int:
        """Compressed bytes one decode step reads (all layers of one KV set,
        all sequences): codes + fp16 scales / biases + fp16 escape rows for
        valid tokens, plus the two int32 page-table entries per page."""
        total = 0
        for l in self.replica_layers(0):
            total += self.k_pool.read_bytes(self.k_page_ids_by_layer[l])
            total += self.v_pool.read_bytes(self.v_page_ids_by_layer[l])
            total += 8 * len(self.k_page_ids_by_layer[l])
        return total

    def window_bytes_per_step(self) -> int:
        """Of :meth:`algorithmic_bytes_per_step`, the bytes of the pages the
        merges attend (plans with merge windows), which no decode launch
        reads: their fp16 keys and values and table entries."""
        total = 0
        for l in self.replica_layers(0):
            plan = self.plans[l]
            if plan.host_windows is None:
                continue
            kt = self.layers[l].k_table.cpu().numpy()
            vt = self.layers[l].v_table.cpu().numpy()
            for (seq, head, _, _), (pb, pe) in zip(plan.host_merges, plan.host_windows):
                total += self.k_pool.read_bytes(kt[seq, head, pb:pe]) + self.v_pool.read_bytes(vt[seq, head, pb:pe])
                total += 8 * int(pe - pb)
        return total

    def token_positions_per_step(self) -> int:
        """(sequence, layer, context token) positions attended per step."""
        return int(np.sum(self.attended_lengths())) * self.spec.n_layers

    def attended_lengths(self) -> np.ndarray:
        """Context tokens each sequence attends per layer (after any append)."""
        return self.attended

    def step(self) -> None:
        """One decode step: per layer of the next KV set (round robin over
        the replicas), (append) + the fused decode kernel + the split-K merge
        kernel.  Replays that set's captured graph when :meth:`capture` has
        been called."""
        r = self.next_replica
        self.next_replica = (r + 1) % self.replicas
        if self.graph is not None:
            self.graph[r].replay()
            return
        self.step_replica(r)

    def step_replica(self, r: int) -> None:
        for l in self.replica_layers(r):
            self.decode_layer(l)
            self.merge_kernel(l)

    def decode_layer(self, l: int) -> None:
        """(Append and) the decode kernel of layer ``l``, partials left in
        the workspace for the merge."""
        if self.spec.append:
            self._append(l)
        self.decode_kernel(l)

    def merge_kernel(self, l: int) -> None:
        lt = self.layers[l]
        merge_partials(self.plans[l], self.outs[l], self.workspace,
                       window=(self.k_pool, self.v_pool, lt.k_table, lt.v_table, self.queries[l], self.query_scale),
                       records=self.records[l] if self.records else None)

    def decode_kernel(self, l: int) -> None:
        """Layer ``l``'s decode kernel alone (``dc_decode_paged_records``
        without the merge).  The layer's page records are gathered again
        first if its tables or the pools changed since."""
        lt = self.layers[l]
        rec = self.records[l] if self.records else None
        if rec is not None and not rec.fresh_for(self.plans[l], lt.k_table, lt.v_table, self.k_pool, self.v_pool):
            rec = self.records[l] = gather_records(self.k_pool, lt.k_table, lt.v_table, lt.seq_pages, self.plans[l],
                                                   v_pool=self.v_pool)
        decode_paged(self.k_pool, lt.k_table, lt.v_table, lt.seq_pages, self.queries[l],
                     query_scale=self.query_scale, plan=self.plans[l], out=self.outs[l], workspace=self.workspace,
                     validate=False, v_pool=self.v_pool, merge=False, records=rec)

    def capture(self) -> None:
        """Capture one whole step (every layer's append, decode and merge
        kernels) as a HIP graph; :meth:`step` then replays it, so a decode
        loop costs one host launch per step.  Pools, tables, plan and
        buffers must not be reallocated afterwards."""
        self.graph = None
        self.graph = [self.capture_fn(lambda r=r: self.step_replica(r)) for r in range(self.replicas)]

    def capture_fn(self, fn):
        """``fn`` (a sequence of this workload's kernel launches) captured as
        a HIP graph, after one eager warm-up run on a side stream."""
        torch = _torch()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # warm-up: descriptor tables and plan uploaded before capture
            fn()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        torch.cuda.synchronize()
        return g

    def _append(self, l: int) -> None:
        """Encode this step's new K / V row of every (sequence, KV head) into
        slot 0 of its tail page (the steady-state cost of one append; the
        tail holds exactly that one token)."""
        self.k_pool.encode_rows_with(self.v_pool, self.new_k[l], self.new_v[l], self.tail_k_dev[l], self.slot_dev,
                                     self.tail_v_dev[l], self.slot_dev)


def _gen(shape, gen, dist: str, device):
    torch = _torch()
    x = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    if dist == "student_t4":
        # t(4) = Z / sqrt(chi2_4 / 4), chi2_4 = sum of 4 squared normals
        chi = torch.zeros(shape[:-1] + (1,), device=device)
        for _ in range(4):
            chi += torch.randn(shape[:-1] + (1,), generator=gen, device=device) ** 2
        x = x / torch.sqrt(chi / 4.0)
    return x


def build_workload(name: str, *, seed: int = 0, device="cuda", layers: int | None = None, batch: int | None = None,
                   context: int | None = None, pages_per_split: int | None = None,
                   scatter_pages: bool = True, key_bits: int | None = None,
                   replicas: int | None = None, window: str = "merge",
                   front_items: int | None = None, lead_ratio: float | None | str = "auto") -> Workload:
    """Encode every layer's pages on the device and build its page tables.
    ``layers`` / ``batch`` / ``context`` shrink the workload for tests (one
    KV set unless ``replicas`` says otherwise); ``replicas`` sets the number
    of independent KV sets the steps cycle through;
    ``scatter_pages=False`` keeps each sequence's pages in allocation order;
    ``key_bits`` re-codes the configuration's M0 key pages at that width
    (a variant named ``<workload>_k<bits>``); ``window`` (fill plans of a
    workload with an exact recent window): ``"merge"`` attends the window's
    fp16 pages in the split-K merge (``make_region_plan(window_merge=True)``),
    ``"launch"`` in a decode launch of its own ahead of the rest
    (``front_items`` items, default one per chunk), either way keeping the
    decode launch to the kernel instance of its 4-bit pages; ``"none"``
    decodes them with the rest in one launch; ``lead_ratio`` (fill plans):
    "auto" plans lead-trail items where the instance runs two waves per
    SIMD (``launch_lead_ratio``), a number that ratio there, None never."""
    if window not in ("merge", "launch", "none"):
        raise ValueError("window must be 'merge', 'launch' or 'none'")
    torch = _torch()
    spec = SPECS[name]
    if key_bits is not None and key_bits != spec.key.bits:
        from dataclasses import replace

        if spec.key.mode != "M0" or key_bits not in (2, 3, 4, 8):
            raise ValueError("key_bits re-codes M0 key pages at 2, 3, 4 or 8 bits")
        spec = replace(spec, name=f"{spec.name}_k{key_bits}", key=replace(spec.key, bits=key_bits))
    if layers is not None or batch is not None or context is not None:
        from dataclasses import replace

        spec = replace(spec, n_layers=layers or spec.n_layers, batch=batch or spec.batch,
                       context=context or spec.context,
                       ragged=None if (context and spec.ragged) else spec.ragged, replicas=1)
    if replicas is not None:
        from dataclasses import replace

        if int(replicas) < 1:
            raise ValueError("replicas must be at least 1")
        spec = replace(spec, replicas=int(replicas))
    dev = torch.device(device)
    B, H, Q, hd, P = spec.batch, spec.n_kv_heads, spec.gqa, spec.head_dim, spec.page_size
    lengths = context_lengths(spec, seed)
    if spec.ragged is not None and batch is not None:
        lengths = lengths[:B]
    n_pages = (lengths + P - 1) // P
    stride = int(n_pages.max()) + (1 if spec.append else 0)
    kgeo = PoolGeometry(hd, spec.key.group_size, P)
    vgeo = PoolGeometry(hd, spec.value.group_size, P)
    m3map = key_m3_map(spec, seed)
    n_sets = spec.n_layers * spec.replicas  # layer sets built: every layer of every replica
    total_pages = int(n_pages.sum()) * H * n_sets

    def pool_bytes(fmt, geo):
        f, b = fmt
        return total_pages * _lib.page_blob_bytes(f, b, geo.c())

    kres = max(pool_bytes(spec.key.fmt, kgeo), pool_bytes((_lib.FMT_M3_F16, 0), kgeo) if m3map.any() else 0)
    k_pool = DevicePagePool(kgeo, device=dev, reserve_bytes=kres + (64 << 20), reserve_pages=total_pages + 1024)
    v_pool = DevicePagePool(vgeo, device=dev, reserve_bytes=pool_bytes(spec.value.fmt, vgeo) + (64 << 20),
                            reserve_pages=total_pages + 1024)
    rng = np.random.default_rng(seed + 5)
    gen = torch.Generator(device=dev)
    tables: list[LayerTables] = []
    queries, new_k, new_v = [], [], []
    kids_by_layer, vids_by_layer = [], []
    kids_tables, vids_tables = [], []
    attended = lengths.copy()
    for l in range(n_sets):
        gen.manual_seed(seed * 1000 + l)
        kt = np.zeros((B, H, stride), dtype=np.int32)
        vt = np.zeros((B, H, stride), dtype=np.int32)
        layer_k_ids, layer_v_ids = [], []
        for h in range(H):
            kfmt = PageFormat("M3") if m3map[l % spec.n_layers, h] else spec.key
            nph = int(n_pages.sum())
            kid = k_pool.allocate(*kfmt.fmt, nph)
            vid = v_pool.allocate(*spec.value.fmt, nph)
            # scatter each (sequence, head)'s pages across the pool
            perm = rng.permutation(nph) if scatter_pages else np.arange(nph)
            kid, vid = kid[perm], vid[perm]
            off = 0
            for b in range(B):
                n = int(n_pages[b])
                kt[b, h, :n] = kid[off: off + n]
                vt[b, h, :n] = vid[off: off + n]
                off += n
            layer_k_ids.append(kid)
            layer_v_ids.append(vid)
        kt_d = torch.from_numpy(kt).to(dev)
        vt_d = torch.from_numpy(vt).to(dev)
        # values, sequence by sequence (bounded memory), encoded on the device
        outl = None
        if spec.outlier_channels:
            outl = torch.from_numpy(np.stack([rng.choice(hd, spec.outlier_channels, replace=False) for _ in range(H)])).to(dev)
        for b in range(B):
            T = int(lengths[b])
            for kind, pool, table in (("K", k_pool, kt_d), ("V", v_pool, vt_d)):
                x = _gen((H, T, hd), gen, spec.distribution, dev)
                if outl is not None:
                    for h in range(H):
                        x[h, :, outl[h]] *= 16.0
                t_idx = torch.arange(T, device=dev, dtype=torch.int64)
                pages = table[b][:, (t_idx // P)].to(torch.int32)  # [H, T]
                slots = (t_idx % P).to(torch.int32).expand(H, T)
                pool.encode_rows(x.reshape(H * T, hd), pages.reshape(-1), slots.reshape(-1))
                del x
        # token counts: full pages except a partial last page
        for b in range(B):
            n = int(n_pages[b])
            last = int(lengths[b]) - (n - 1) * P
            k_pool.set_tokens(kt[b, :, : n - 1], P)
            v_pool.set_tokens(vt[b, :, : n - 1], P)
            k_pool.set_tokens(kt[b, :, n - 1], last)
            v_pool.set_tokens(vt[b, :, n - 1], last)
        lt = LayerTables(kt_d, vt_d, n_pages.astype(np.int32))
        if spec.recent_window:
            _apply_recent_window(spec, k_pool, v_pool, kt, vt, n_pages, lengths, gen, dev, lt, l)
            lt.k_table = torch.from_numpy(kt).to(dev)
            lt.v_table = torch.from_numpy(vt).to(dev)
        if spec.append:
            tk = k_pool.allocate(*spec.key.fmt, B * H, tokens=0).reshape(B, H)
            tv = v_pool.allocate(*spec.value.fmt, B * H, tokens=0).reshape(B, H)
            seq_pages = n_pages.astype(np.int32).copy()
            for b in range(B):
                kt[b, :, seq_pages[b]] = tk[b]
                vt[b, :, seq_pages[b]] = tv[b]
            seq_pages += 1
            lt.k_table = torch.from_numpy(kt).to(dev)
            lt.v_table = torch.from_numpy(vt).to(dev)
            lt.seq_pages = seq_pages
            lt.tail_k, lt.tail_v = tk, tv
            new_k.append(_gen((B * H, hd), gen, spec.distribution, dev))
            new_v.append(_gen((B * H, hd), gen, spec.distribution, dev))
            # the tail holds the appended token of this step: count it
            k_pool.set_tokens(tk.ravel(), 1)
            v_pool.set_tokens(tv.ravel(), 1)
        tables.append(lt)
        kt_now = lt.k_table.cpu().numpy()
        vt_now = lt.v_table.cpu().numpy()
        kids_tables.append(kt_now)
        vids_tables.append(vt_now)
        kids_by_layer.append(np.concatenate([kt_now[b, :, : lt.seq_pages[b]].ravel() for b in range(B)]))
        vids_by_layer.append(np.concatenate([vt_now[b, :, : lt.seq_pages[b]].ravel() for b in range(B)]))
        queries.append((torch.randn((B, H, Q, hd), generator=gen, device=dev)).to(torch.bfloat16))
    if spec.append:
        attended = lengths + 1
    wl = Workload(spec=spec, seed=seed, lengths=lengths, k_pool=k_pool, v_pool=v_pool, layers=tables, queries=queries,
                  new_k=new_k, new_v=new_v, k_page_ids_by_layer=kids_by_layer, v_page_ids_by_layer=vids_by_layer,
                  attended=attended)
    # per layer: a launch's budget of items cut at 32-token chunks, each
    # stream cut by its pages' costs (an exact recent window reads more
    # bytes per token)
    # (the last pages' token counts: C5's tail holds the one appended token)
    cpp = chunks_per_page(P)

    def _lead(kp, vp, q, km=None, vm=None):
        if pages_per_split is not None or lead_ratio is None or launch_lead_ratio(kp, vp, q, km, vm) is None:
            r = None
        else:
            r = launch_lead_ratio(kp, vp, q, km, vm) if lead_ratio == "auto" else float(lead_ratio)
        wl.lead_ratios.append(r)
        return r

    for l, lt in enumerate(tables):
        cost = None
        if pages_per_split is None:
            cost = page_costs(k_pool, v_pool, kids_tables[l], vids_tables[l], lt.seq_pages)
        last = k_pool.tokens_of(kids_tables[l][np.arange(B), 0, np.asarray(lt.seq_pages) - 1]).astype(np.int32)
        front = _exact_window(k_pool, v_pool, kids_tables[l], vids_tables[l], lt.seq_pages) \
            if (window != "none" and spec.recent_window and pages_per_split is None) else None
        if front is not None:
            # the bulk launch: every page outside the window, at the waves
            # per SIMD of its own formats
            pg = np.arange(kids_tables[l].shape[2])[None, None, :]
            outside = np.broadcast_to((pg < np.asarray(lt.seq_pages)[:, None, None])
                                      & ~((pg >= front[:, 0, None, None]) & (pg < front[:, 1, None, None])),
                                      kids_tables[l].shape)
            km = k_pool.format_mask_of(kids_tables[l][outside])
            vm = v_pool.format_mask_of(vids_tables[l][outside])
            wl.plans.append(make_region_plan(lt.seq_pages, H, front, device=dev, chunks_per_page=cpp, page_cost=cost,
                                             target_items=launch_target_items(k_pool, v_pool, Q, km, vm),
                                             last_page_tokens=last, front_items=front_items,
                                             window_merge=window == "merge",
                                             lead_ratio=_lead(k_pool, v_pool, Q, km, vm)))
        else:
            # (page records will narrow the launch to the formats its tables
            # reference: plan for that instance)
            km = k_pool.format_mask_of(kids_by_layer[l])
            vm = v_pool.format_mask_of(vids_by_layer[l])
            wl.plans.append(make_plan(lt.seq_pages, H, pages_per_split, device=dev, chunks_per_page=cpp,
                                      page_cost=cost, target_items=launch_target_items(k_pool, v_pool, Q, km, vm),
                                      last_page_tokens=last, lead_ratio=_lead(k_pool, v_pool, Q, km, vm)))
    wl.plan = wl.plans[0]
    need = max(workspace_bytes(p, Q, hd) for p in wl.plans)
    wl.workspace = torch.zeros(max(need, 16), dtype=torch.uint8, device=dev)
    wl.outs = [torch.empty((B, H, Q, hd), dtype=torch.float32, device=dev) for _ in range(n_sets)]
    if spec.append:
        wl.tail_k_dev = [torch.from_numpy(t.tail_k.ravel().astype(np.int32)).to(dev) for t in tables]
        wl.tail_v_dev = [torch.from_numpy(t.tail_v.ravel().astype(np.int32)).to(dev) for t in tables]
        wl.slot_dev = torch.zeros(B * H, dtype=torch.int32, device=dev)
    k_pool.device_descs()
    v_pool.device_descs()
    # the descriptors of every item's pages, gathered once: the tables and
    # descriptors stay fixed from here on (the append writes a tail page's
    # codes, not its descriptor)
    wl.records = [gather_records(k_pool, lt.k_table, lt.v_table, lt.seq_pages, wl.plans[l], v_pool=v_pool)
                  for l, lt in enumerate(tables)]
    torch.cuda.synchronize(dev)
    return wl


def _exact_window(k_pool, v_pool, kt: np.ndarray, vt: np.ndarray, seq_pages) -> np.ndarray | None:
    """Per sequence, the page range ``[begin, end)`` of its exact recent
    window: the fp16 (M3) key and value pages, the same for every KV head
    and contiguous.  None when some sequence has none or they do not form
    one such range."""
    out = np.zeros((kt.shape[0], 2), dtype=np.int64)
    for b in range(kt.shape[0]):
        n = int(seq_pages[b])
        exact = (k_pool.formats_of(kt[b, :, :n]) == _lib.FMT_M3_F16) & (v_pool.formats_of(vt[b, :, :n]) == _lib.FMT_M3_F16)
        if not np.all(exact == exact[0]) or not exact[0].any():
            return None
        idx = np.flatnonzero(exact[0])
        if idx[-1] - idx[0] + 1 != idx.size:
            return None
        out[b] = (idx[0], idx[-1] + 1)
    return out


def _apply_recent_window(spec, k_pool, v_pool, kt, vt, n_pages, lengths, gen, dev, lt, layer):
    """Replace the pages that the planner's recent-window rule keeps exact
    (``choose_page_mode``: the page's oldest token is younger than
    ``recent_window``, reference ``planner.py:84-106``) by fp16 (M3) pages
    holding fresh rows."""
    torch = _torch()
    P = spec.page_size
    B, H = kt.shape[:2]
    hd = spec.head_dim
    policy = {kind: make_explicit_policy(kind=kind, policy_id=f"{kind.lower()}_workload", sensitivity_tier="balanced",
                                         candidates=(PageModeSpec(mode=fmt.mode, bits=fmt.bits,
                                                                  quant_scheme=fmt.scheme),),
                                         recent_window=spec.recent_window)
              for kind, fmt in (("K", spec.key), ("V", spec.value))}
    for b in range(B):
        n = int(n_pages[b])
        exact = [p for p in range(n)
                 if all(choose_page_mode(layer, kind, int(lengths[b]) - p * P - 1, None,
                                         layer_policy=policy[kind]).mode == "M3" for kind in ("K", "V"))]
        for p in exact:
            tokens = min(P, int(lengths[b]) - p * P)
            for pool, table in ((k_pool, kt), (v_pool, vt)):
                ids = pool.allocate(_lib.FMT_M3_F16, 0, H, tokens=tokens)
                x = _gen((H * tokens, hd), gen, spec.distribution, dev)
                pages = torch.from_numpy(np.repeat(ids, tokens).astype(np.int32)).to(dev)
                slots = torch.arange(tokens, dtype=torch.int32, device=dev).repeat(H)
                pool.encode_rows(x, pages, slots)
                pool.free(table[b, :, p])
                table[b, :, p] = ids
