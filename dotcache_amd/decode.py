"""Host driver of the fused paged decode kernel (``dc_decode_paged``).

A decode call covers a batch of sequences x KV heads of one layer.  Page
tables are int32 ``[n_seqs, n_kv_heads, table_stride]`` arrays of page ids in
one :class:`~dotcache_amd.page_pool.DevicePagePool`; sequences may have
different page counts (ragged batch) and their pages may sit anywhere in the
arena.  The host planner splits long page lists into work items (split-K):
``dc_plan_decode`` into items of ``pages_per_split`` pages,
``dc_plan_decode_fill`` into a launch's budget of items of near-equal cost,
cut on 32-token chunk boundaries inside pages.  The kernel writes
``(m, l, o)`` partials for split items and the merge pass combines them by
log-sum-exp.  Plans are cached per (page counts, heads, split, costs) so a
steady decode loop uploads nothing.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib
from .page_pool import DevicePagePool, current_stream_ptr, dtype_code

# A work item is one wavefront's share.  Split long page lists so a launch has
# about one item per SIMD (256 CUs x 4): every wavefront then streams several
# pages, which amortises its fixed cost (the page-table and descriptor reads
# before the first load, the query set-up, the final write) and keeps the
# split-K partials a small fraction of the bytes read.
DEFAULT_TARGET_ITEMS = 1024
MIN_PAGES_PER_SPLIT = 2
# The fill planner splits a stream no finer than this many 32-token chunks
# per item.  Only launches with budget to spare reach it (small batches):
# on C2 (8 streams of 64 pages) items of 2 chunks took 6.7 us per layer
# against 8.4 us for 4 chunks (4-page items), with the merge unchanged
# (4.0 us); single chunks gained nothing more once the merge grew.
MIN_CHUNKS_PER_SPLIT = 2
# Planner cost of a page (page_costs): its compressed key and value bytes
# plus this much per 32-token chunk.  Measured on MI355X with one wave per
# SIMD, a 32-token chunk of 4-bit M0 keys and values at head_dim 256 (10 KiB)
# took a wave 2.4 us and one of fp16 keys and values (32 KiB) 5.4 us: about
# 1.0 us plus 7.5 GB/s per wave, and 1.0 us is worth about 8 KiB at that rate.
CHUNK_COST_BYTES = 8192
# Instances built for two waves per SIMD: the first wave placed on a SIMD
# (blocks [0, n_simd) of a launch; block b + n_simd joins block b's SIMD)
# issues first whenever both are ready, so with equal items it finished
# first (C5: 91 against 123 us; C4: 26 against 33 us) and the second one
# then ran alone.  Lead-trail plans (``lead_ratio``) cut each SIMD's share
# into a lead item, placed in the first half of the launch, and a trail
# item this many times smaller in the second.
LEAD_RATIO = 1.6
# A wave alone on its SIMD streams about this fraction of what the SIMD's
# two waves stream together: in those equal-item C4 launches the second wave
# ran alone for the last 7 of 33 us.  Lead-trail plans use it to price a
# SIMD whose two items do not end together (``_pair_time``).
LONE_WAVE_RATE = 0.86


def _torch():
    import torch

    return torch


@dataclass
class DecodePlan:
    items: object          # device uint8 tensor holding dc_work_item[n_items]
    merges: object | None  # device uint8 tensor holding dc_merge_item[n_merges]
    n_items: int
    n_merges: int
    n_partials: int
    pages_per_split: int              # largest item, in (whole or partly covered) pages
    host_items: np.ndarray            # int32 [n_items, 8]: dc_work_item fields
    host_merges: np.ndarray | None = None  # int32 [n_merges, 4]: dc_merge_item fields
    checked: set = None               # (seq_pages, n_kv_heads, table_stride) keys already validated
    chunks_per_page: int = 1          # the page split granularity the items were cut for
    largest_chunks: int = 0           # largest item in 32-token chunks (fill plans)
    # items [0, n_front) run in a launch of their own ahead of the rest
    # (make_region_plan: the pages of a different format mix, such as an
    # exact recent window, kept out of the bulk launch's kernel instance)
    n_front: int = 0
    # region plans with window_merge: per merge item the page range
    # [begin, end) of its stream that the merge itself attends
    # (dc_window_merge; fp16 key and value pages), device int32 [n_merges, 2]
    windows: object | None = None
    host_windows: np.ndarray | None = None

    def check(self, seq_pages: np.ndarray, n_kv_heads: int, table_stride: int, chunks_per_page: int = 1) -> None:
        """Raise ValueError unless every work item and merge item of the plan
        stays inside these shapes: sequence < n_seqs, KV head < n_kv_heads,
        pages within the sequence's count (and so within the page table),
        chunk offsets within a page of ``chunks_per_page`` chunks (and cut
        for that many), partial slots below n_partials, and device buffers
        as long as the counts.  The kernels read items without checking them
        against the tables, so a plan built for other shapes must not reach
        them.  Validated once per shape key."""
        sp = np.asarray(seq_pages, dtype=np.int64)
        key = (sp.tobytes(), int(n_kv_heads), int(table_stride), int(chunks_per_page))
        if self.checked is None:
            self.checked = set()
        if key in self.checked:
            return
        B = sp.size
        it = np.asarray(self.host_items, dtype=np.int64).reshape(-1, 8)
        if it.shape[0] != self.n_items or self.items.numel() < 32 * self.n_items:
            raise ValueError("plan: work item count does not match its device buffer")
        seq, head, pb, pe, part = it[:, 0], it[:, 1], it[:, 2], it[:, 3], it[:, 4]
        if np.any((seq < 0) | (seq >= B)) or np.any((head < 0) | (head >= n_kv_heads)):
            raise ValueError(f"plan: a work item names a sequence or KV head outside [{B}] x [{n_kv_heads}]")
        limit = np.minimum(sp[np.clip(seq, 0, max(B - 1, 0))], int(table_stride))
        if np.any(pb < 0) or np.any(pe < pb) or np.any(pe > limit):
            raise ValueError("plan: a work item's pages lie outside its sequence's page table")
        if np.any(part >= self.n_partials):
            raise ValueError("plan: a work item names a partial slot past n_partials")
        cb, ce = it[:, 5], it[:, 6]
        if np.any(cb != 0) or np.any(ce != 0):
            if int(self.chunks_per_page) != int(chunks_per_page):
                raise ValueError(f"plan: items cut for {self.chunks_per_page} chunks per page, pool pages hold "
                                 f"{chunks_per_page}")
            if (np.any((cb < 0) | (cb >= chunks_per_page)) or np.any((ce < 0) | (ce > chunks_per_page))
                    or np.any((pe - pb == 1) & (ce > 0) & (ce <= cb))):
                raise ValueError("plan: a work item's chunk range lies outside its pages")
        if self.n_merges:
            m = np.asarray(self.host_merges, dtype=np.int64).reshape(-1, 4)
            if m.shape[0] != self.n_merges or self.merges is None or self.merges.numel() < 16 * self.n_merges:
                raise ValueError("plan: merge item count does not match its device buffer")
            if (np.any((m[:, 0] < 0) | (m[:, 0] >= B)) or np.any((m[:, 1] < 0) | (m[:, 1] >= n_kv_heads))
                    or np.any(m[:, 2] < 0) or np.any(m[:, 3] <= 0) or np.any(m[:, 2] + m[:, 3] > self.n_partials)):
                raise ValueError("plan: a merge item lies outside the shapes or the partial slots")
        self.checked.add(key)


_plan_cache: dict = {}


def default_target_items() -> int:
    """Work items one launch should have: one per SIMD of the current device
    (4 per CU), so a one-wavefront-per-SIMD kernel runs every item in a single
    round."""
    try:
        torch = _torch()
        if torch.cuda.is_available():
            return 4 * int(torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count)
    except Exception:
        pass
    return DEFAULT_TARGET_ITEMS


def waves_per_simd(pool: DevicePagePool, v_pool: DevicePagePool | None, n_q: int, k_mask: int | None = None,
                   v_mask: int | None = None) -> int:
    """Work items per SIMD the decode kernel for these pools and ``n_q``
    runs at once (``dc_decode_waves_per_simd``): 1 or 2.  ``k_mask`` /
    ``v_mask``: the formats of the pages the launch reads
    (``format_mask_of``), when narrower than the pools'."""
    vpool = pool if v_pool is None else v_pool
    kp, vp = pool.c_pool(), vpool.c_pool()
    if k_mask:
        kp.format_mask = int(k_mask) & pool.format_mask
    if v_mask:
        vp.format_mask = int(v_mask) & vpool.format_mask
    return int(_lib.lib().dc_decode_waves_per_simd(kp, vp, int(n_q)))


def launch_target_items(pool: DevicePagePool, v_pool: DevicePagePool | None, n_q: int, k_mask: int | None = None,
                        v_mask: int | None = None) -> int:
    """Items that fill one launch round: one per SIMD times the kernel's
    waves per SIMD."""
    return default_target_items() * waves_per_simd(pool, v_pool, n_q, k_mask, v_mask)


def launch_lead_ratio(pool: DevicePagePool, v_pool: DevicePagePool | None, n_q: int, k_mask: int | None = None,
                      v_mask: int | None = None) -> float | None:
    """``LEAD_RATIO`` when the instance for these formats runs two waves per
    SIMD (plan lead-trail items for it), else None."""
    return LEAD_RATIO if waves_per_simd(pool, v_pool, n_q, k_mask, v_mask) == 2 else None


def choose_pages_per_split(seq_pages: np.ndarray, n_kv_heads: int, target_items: int | None = None) -> int:
    """Smallest pages-per-split (at least MIN_PAGES_PER_SPLIT) for which the
    plan has at most ``target_items`` items; the planner then cuts every
    sequence into near-equal items of at most that many pages."""
    sp = np.asarray(seq_pages, dtype=np.int64)
    target = int(target_items) if target_items else default_target_items()
    top = max(int(sp.max()), 1)

    def n_items(per: int) -> int:
        return int(n_kv_heads * np.sum(-(-sp // per)))

    lo, hi = min(MIN_PAGES_PER_SPLIT, top), top
    if n_items(hi) > target:
        return hi  # more sequences x heads than items: one item each
    while lo < hi:
        mid = (lo + hi) // 2
        if n_items(mid) <= target:
            hi = mid
        else:
            lo = mid + 1
    return int(lo)


def chunks_per_page(page_capacity: int) -> int:
    """32-token chunks in a page of this capacity: the finest split a plan
    may cut pages at."""
    return max(1, (int(page_capacity) + 31) // 32)


def page_costs(k_pool: DevicePagePool, v_pool: DevicePagePool, k_table, v_table, seq_pages) -> np.ndarray:
    """float32 ``[n_seqs, n_kv_heads, table_stride]``: each page's decode
    cost for :func:`make_plan`, 0 past a sequence's pages.  ``k_table`` /
    ``v_table``: host int32 page ids.

    Within a stream (one sequence and KV head) a page costs its key and
    value bytes of valid tokens plus ``CHUNK_COST_BYTES`` per started
    32-token chunk, so the item holding an exact recent window gets fewer
    pages.  Each stream's costs are then scaled to sum to its page count:
    between streams the planner balances page counts.  Measured on MI355X,
    a batch whose exact (fp16) key streams got smaller items by their byte
    cost ran slower (C4 shape: 51.5 against 50.7 us per layer): the exact
    streams' waves share HBM with the others, so their items run no longer
    than the rest when all are the same size."""
    kt = np.asarray(k_table, dtype=np.int64)
    vt = np.asarray(v_table, dtype=np.int64)
    if kt.ndim != 3 or vt.shape != kt.shape:
        raise ValueError("page tables must have shape [n_seqs, n_kv_heads, table_stride]")
    sp = np.asarray(seq_pages, dtype=np.int64)
    live = np.arange(kt.shape[2])[None, None, :] < sp[:, None, None]
    kt = np.where(live, kt, 0)
    vt = np.where(live, vt, 0)
    tok = k_pool.tokens_of(kt)
    raw = k_pool.read_bytes_each(kt) + v_pool.read_bytes_each(vt) + CHUNK_COST_BYTES * ((tok + 31) // 32)
    raw = np.where(live, raw, 0).astype(np.float64)
    total = raw.sum(axis=2, keepdims=True)
    scale = np.where(total > 0, sp[:, None, None] / np.maximum(total, 1.0), 0.0)
    cost = np.where(total > 0, raw * scale, live.astype(np.float64))
    return cost.astype(np.float32)


def make_plan(seq_pages, n_kv_heads: int, pages_per_split: int | None = None, *, device="cuda",
              target_items: int | None = None, chunks_per_page: int = 1, page_cost=None,
              last_page_tokens=None, lead_ratio: float | None = None) -> DecodePlan:
    """Work and merge items for a batch with these page counts.  With
    ``pages_per_split`` the near-equal splits of ``dc_plan_decode`` (whole
    pages).  Without it ``dc_plan_decode_fill``: ``target_items`` (default:
    one per SIMD) items of near-equal cost, cut at 32-token chunk
    boundaries when ``chunks_per_page`` > 1 (pass
    :func:`chunks_per_page` of the pool's page capacity), with each page
    costing ``page_cost[b, h, page]`` (float ``[n_seqs, n_kv_heads, >= max
    pages]``; default: the same for every chunk).  No item has fewer than
    ``MIN_CHUNKS_PER_SPLIT`` chunks unless its stream does.
    ``last_page_tokens`` (one per sequence, fill plans only): the tokens in
    each sequence's last page, so the chunks past them are not counted and
    no item falls among them; without it every page counts as full.
    ``DecodePlan.pages_per_split`` is the largest item's page count.
    ``lead_ratio`` (fill plans for an instance at two waves per SIMD): a
    lead-trail plan (:func:`lead_trail_split`) of ``target_items / 2`` SIMD
    shares."""
    torch = _torch()
    sp = np.ascontiguousarray(np.asarray(seq_pages, dtype=np.int32))
    if sp.ndim != 1 or sp.size == 0:
        raise ValueError("seq_pages must be a non-empty 1-D array")
    if np.any(sp <= 0):
        raise ValueError("decode requires at least one page per sequence")
    fill = pages_per_split is None
    pps = 0 if fill else int(pages_per_split)
    target = (int(target_items) if target_items else default_target_items()) if fill else 0
    cpp = int(chunks_per_page) if fill else 1
    if cpp <= 0:
        raise ValueError("chunks_per_page must be positive")
    cost = None
    if fill and page_cost is not None:
        cost = np.ascontiguousarray(np.asarray(page_cost, dtype=np.float32))
        if cost.ndim != 3 or cost.shape[:2] != (sp.size, int(n_kv_heads)) or cost.shape[2] < int(sp.max()):
            raise ValueError("page_cost must have shape [n_seqs, n_kv_heads, >= max pages]")
    last = None
    if fill and last_page_tokens is not None:
        last = np.ascontiguousarray(np.asarray(last_page_tokens, dtype=np.int32))
        if last.shape != sp.shape:
            raise ValueError("last_page_tokens must have one entry per sequence")
        if np.any(last <= 0) or np.any(last > 32 * cpp):
            raise ValueError(f"last_page_tokens must lie in [1, {32 * cpp}]")
    lead = float(lead_ratio) if (fill and lead_ratio) else None
    # the plan depends on the last pages only through their chunk counts, so
    # a decode that appends a token reuses it until a new chunk starts
    key = (sp.tobytes(), int(n_kv_heads), pps, target, cpp, None if cost is None else (cost.shape, cost.tobytes()),
           None if last is None else ((last + 31) // 32).tobytes(), lead, str(device))
    hit = _plan_cache.get(key)
    if hit is not None:
        return hit
    if lead:
        target = max(target // 2, 1)  # SIMD shares, each cut into a lead and a trail item
    L = _lib.lib()
    ni, nm, npart, big = C.c_int32(), C.c_int32(), C.c_int32(), C.c_int32()

    def plan(items_p, max_items, merges_p, max_merges):
        if fill:
            return L.dc_plan_decode_fill(sp.ctypes.data, None if last is None else last.ctypes.data, sp.size,
                                         n_kv_heads, cpp,
                                         None if cost is None else cost.ctypes.data,
                                         0 if cost is None else cost.shape[2], target, MIN_CHUNKS_PER_SPLIT,
                                         items_p, max_items, C.byref(ni), merges_p, max_merges, C.byref(nm),
                                         C.byref(npart), C.byref(big))
        return L.dc_plan_decode(sp.ctypes.data, sp.size, n_kv_heads, pps, items_p, max_items, C.byref(ni), merges_p,
                                max_merges, C.byref(nm), C.byref(npart))

    st = plan(None, 0, None, 0)
    if st not in (_lib.DC_OK, _lib.DC_ESPACE):
        _lib.check(st, "dc_plan_decode")
    items = (_lib.WorkItem * max(ni.value, 1))()
    merges = (_lib.MergeItem * max(nm.value, 1))()
    st = plan(C.addressof(items), ni.value, C.addressof(merges), nm.value)
    _lib.check(st, "dc_plan_decode")
    if fill:
        pps = -(-int(big.value) // cpp)
    host_items = np.frombuffer(bytes(items), dtype=np.int32).reshape(-1, 8)[: ni.value].copy()
    host_merges = np.frombuffer(bytes(merges), dtype=np.int32).reshape(-1, 4)[: nm.value].copy()
    n_part = npart.value
    if lead:
        pairs = []
        if fill:
            host_items, pairs = _pair_short_streams(host_items, sp, int(n_kv_heads), cpp, last, cost, target, lead)
        host_items = lead_trail_split(host_items, lead, cpp, pairs=pairs)
        host_items, host_merges, n_part = _stream_partials(host_items, int(n_kv_heads))
        big.value = int(_item_chunks(host_items, cpp).max())
        pps = -(-int(big.value) // cpp)
    dev_items = torch.from_numpy(host_items.ravel().view(np.uint8).copy()).to(device)
    dev_merges = torch.from_numpy(host_merges.ravel().view(np.uint8).copy()).to(device) if len(host_merges) else None
    plan = DecodePlan(dev_items, dev_merges, len(host_items), len(host_merges), n_part, pps, host_items, host_merges,
                      chunks_per_page=cpp, largest_chunks=int(big.value) if fill else pps)
    if len(_plan_cache) > 256:
        _plan_cache.clear()
    _plan_cache[key] = plan
    return plan


def _item_chunks(items: np.ndarray, cpp: int) -> np.ndarray:
    """32-token chunks of each host work item (``[n, 8]``)."""
    it = np.asarray(items, dtype=np.int64).reshape(-1, 8)
    first = it[:, 2] * cpp + it[:, 5]
    end = np.where(it[:, 6] > 0, (it[:, 3] - 1) * cpp + it[:, 6], it[:, 3] * cpp)
    return end - first


def lead_trail_split(items: np.ndarray, ratio: float, cpp: int, pairs=()) -> np.ndarray:
    """Cut each host work item (one SIMD's share) at a chunk boundary into
    a lead item ``ratio`` times the trail item's chunks and the trail item;
    the leads first, in order, then the unsplit shares, then the trails in
    the leads' order, so trail j follows the launch's n shares at block n +
    j and shares lead j's SIMD.  A share of one chunk stays whole.  (The
    only share of a short stream is cut too, although its stream then needs
    a merge: left whole it ran alone on its SIMD and set the end of the
    launch, C4 39.3 -> 47.0 us.)  ``pairs``: (lead, trail) host items of
    shares made of two whole streams (``_pair_short_streams``), placed after
    the cut shares' leads and trails.  Partial slots are not set."""
    it = np.asarray(items, dtype=np.int64).reshape(-1, 8)
    first = it[:, 2] * cpp + it[:, 5]
    n = _item_chunks(it, cpp)
    cut = first + np.clip(np.rint(n * float(ratio) / (1.0 + float(ratio))).astype(np.int64), 1, np.maximum(n - 1, 1))
    split = n >= 2

    def rng(seq, head, u0, u1):
        return [seq, head, u0 // cpp, -(-u1 // cpp), -1, u0 % cpp, u1 % cpp, 0]

    leads, whole, trails = [], [], []
    for k in range(len(it)):
        seq, head = int(it[k, 0]), int(it[k, 1])
        u0, u1 = int(first[k]), int(first[k] + n[k])
        if split[k]:
            leads.append(rng(seq, head, u0, int(cut[k])))
            trails.append(rng(seq, head, int(cut[k]), u1))
        else:
            whole.append(rng(seq, head, u0, u1))
    leads += [list(map(int, a)) for a, _ in pairs]
    trails += [list(map(int, b)) for _, b in pairs]
    return np.asarray(leads + whole + trails, dtype=np.int32).reshape(-1, 8)


def _pair_time(a: float, b: float, ratio: float) -> float:
    """Time of a SIMD running items of costs a (the older wave, which issues
    first) and b at two waves per SIMD, in units of one cost unit at the
    SIMD's two-wave rate: a share cut at ``ratio`` : 1 takes a + b; an item
    left alone after the other ends runs at ``LONE_WAVE_RATE``."""
    lf = ratio / (1.0 + ratio)  # the lead's part of the SIMD's rate while both run
    if a >= ratio * b:
        return b / (1.0 - lf) + (a - ratio * b) / LONE_WAVE_RATE
    return a / lf + (b - a * (1.0 - lf) / lf) / LONE_WAVE_RATE


def _stream_cost_prefix(sp: np.ndarray, n_kv_heads: int, cpp: int, last, cost):
    """Running costs over each stream's chunks that hold tokens, streams s =
    b * H + h laid end to end: (flat, off, n) with flat[off[s] + u] the cost
    of stream s's chunks [0, u) and n[s] its chunk count.  A page's cost is
    spread over its chunks (1 per chunk without page costs), as
    ``dc_plan_decode_fill`` prices them."""
    parts, off, n = [], [], []
    at = 0
    for b in range(sp.size):
        lc = cpp if last is None else min(cpp, (int(last[b]) + 31) // 32)
        per_page = np.full(int(sp[b]), cpp, dtype=np.int64)
        per_page[-1] = lc
        for h in range(n_kv_heads):
            if cost is None:
                c = np.ones(int(per_page.sum()))
            else:
                c = np.repeat(np.asarray(cost[b, h, : sp[b]], dtype=np.float64) / per_page, per_page)
            parts.append(np.concatenate([[0.0], np.cumsum(c)]))
            off.append(at)
            n.append(c.size)
            at += c.size + 1
    return np.concatenate(parts), np.asarray(off, dtype=np.int64), np.asarray(n, dtype=np.int64)


def _items_cost(items: np.ndarray, prefix, n_kv_heads: int, cpp: int) -> np.ndarray:
    flat, off, _ = prefix
    it = np.asarray(items, dtype=np.int64).reshape(-1, 8)
    first = it[:, 2] * cpp + it[:, 5]
    base = off[it[:, 0] * n_kv_heads + it[:, 1]]
    return flat[base + first + _item_chunks(it, cpp)] - flat[base + first]


def _pair_short_streams(items: np.ndarray, sp: np.ndarray, n_kv_heads: int, cpp: int, last, cost, n_shares: int,
                        ratio: float):
    """A fill plan of ``n_shares`` SIMD shares (``items``, one stream per
    share) gives every stream a whole number of shares, so its largest share
    exceeds the mean by up to a chunk (C4: 28 chunks against a mean of
    25.7), while a short stream's only share holds less.  Two short whole
    streams may share one SIMD instead, the longer as the lead (the older
    wave) and the shorter as the trail, freeing a share for the long
    streams, and the paired streams, each one item, need no merge.  Pairs
    are formed under a bound on their SIMD time (``_pair_time``), found by
    bisection between the mean share and the plain plan's largest, where
    the long streams' largest share meets it.  Returns (items of the other
    streams' fill plan, [(lead, trail) host items]) for the pairing whose
    largest SIMD time is lowest and no higher than the plain plan's, the
    most pairs among equals; else (``items``, []).  (C4: 12 pairs, the
    decode launch 39.4-39.7 against 39.3-39.6 us, the merge 4.6 against 5.1
    us with 24 fewer merge items.)"""
    H = n_kv_heads
    if len(items) < n_shares or not 3 <= sp.size * H < n_shares:  # (more streams than shares: no spare SIMD)
        return items, []
    prefix = _stream_cost_prefix(sp, H, cpp, last, cost)
    flat, off, nch = prefix
    total = flat[off + nch]
    level = float(_items_cost(items, prefix, H, cpp).max())
    mean = float(total.sum()) / n_shares
    short = [int(s) for s in np.argsort(-total, kind="stable") if total[s] < level]
    if len(short) < 2:
        return items, []

    def whole(s):
        b, h = divmod(s, H)
        n = int(nch[s])
        return [b, h, 0, -(-n // cpp), -1, 0, n % cpp, 0]

    def evaluate(bound):
        # longest first, each with the longest partner whose pair time fits:
        # the partners left are kept by ascending cost, all at most the
        # current stream's, over which the pair time only grows
        avail = short[::-1]
        used, pairs = set(), []
        while avail:
            s = avail.pop()
            lo, hi = 0, len(avail)
            while lo < hi:  # first partner whose pair time exceeds the bound
                mid = (lo + hi) // 2
                if _pair_time(total[s], total[avail[mid]], ratio) <= bound:
                    lo = mid + 1
                else:
                    hi = mid
            if lo > 0:
                t = avail.pop(lo - 1)
                used |= {s, t}
                pairs.append((s, t))
        rest = np.asarray([s for s in range(total.size) if s not in used], dtype=np.int64)
        if not pairs:
            return None  # the bound is below every pair
        if rest.size == 0:
            return False  # every stream paired: leave some to the fill planner
        b_, h_ = rest // H, rest % H
        pages = sp[b_].astype(np.int32)
        ulast = (np.full(len(rest), 32 * cpp, np.int32) if last is None else np.asarray(last)[b_]).astype(np.int32)
        ucost = None
        if cost is not None:
            ucost = np.zeros((len(rest), 1, int(pages.max())), dtype=np.float32)
            for k in range(len(rest)):
                ucost[k, 0, : pages[k]] = cost[b_[k], h_[k], : pages[k]]
        it, _ = _fill_units(pages, ulast, ucost, cpp, n_shares - len(pairs), MIN_CHUNKS_PER_SPLIT)
        src = rest[it[:, 0]]
        it[:, 0], it[:, 1] = src // H, src % H
        return (float(_items_cost(it, prefix, H, cpp).max()),
                max(_pair_time(total[s], total[t], ratio) for s, t in pairs), pairs, it)

    best = (level, 0, items, [])
    lo, hi, bound = mean, level, level  # the most pairs first, then four bisection steps
    for _ in range(5):
        r = evaluate(bound)
        if r is None:
            lo = bound
        elif r is False:
            hi = bound
        else:
            longest, pair_max, pairs, it = r
            worst = max(longest, pair_max)
            if (worst, -len(pairs)) < (best[0], -best[1]):
                best = (worst, len(pairs), it, [(whole(s), whole(t)) for s, t in pairs])
            if longest > bound:  # the long streams are still above it: allow more pairs
                lo = bound
            else:
                hi = bound
        bound = 0.5 * (lo + hi)
    return best[2], best[3]


def _stream_partials(items: np.ndarray, n_kv_heads: int, force_merge: bool = False):
    """Partial slots and merge items for host work items in any order:
    every (sequence, KV head) stream's items take consecutive slots and one
    merge item; a stream of one item writes its output directly (unless
    ``force_merge``).  Returns (items, merges [m, 4], n_partials)."""
    items = np.asarray(items, dtype=np.int32).reshape(-1, 8).copy()
    H = int(n_kv_heads)
    stream = items[:, 0].astype(np.int64) * H + items[:, 1]
    merges, n_part = [], 0
    for s_ in np.unique(stream):
        rows = np.flatnonzero(stream == s_)
        if len(rows) == 1 and not force_merge:
            items[rows[0], 4] = -1
            continue
        items[rows, 4] = n_part + np.arange(len(rows), dtype=np.int32)
        merges.append((int(s_) // H, int(s_) % H, n_part, len(rows)))
        n_part += len(rows)
    items[:, 7] = 0
    return items, np.asarray(merges, dtype=np.int32).reshape(-1, 4), n_part


def _fill_units(unit_pages: np.ndarray, unit_last: np.ndarray, unit_cost, cpp: int, target: int,
                min_chunks: int) -> tuple[np.ndarray, int]:
    """``dc_plan_decode_fill`` over independent page runs ("units", each
    planned as a sequence of one KV head): host items ``[n, 8]`` with the
    unit index in the sequence field, and the largest item in chunks."""
    L = _lib.lib()
    ni, nm, npart, big = C.c_int32(), C.c_int32(), C.c_int32(), C.c_int32()
    sp = np.ascontiguousarray(unit_pages, dtype=np.int32)
    last = np.ascontiguousarray(unit_last, dtype=np.int32)
    cost = None if unit_cost is None else np.ascontiguousarray(unit_cost, dtype=np.float32)

    def plan(items_p, max_items, merges_p, max_merges):
        return L.dc_plan_decode_fill(sp.ctypes.data, last.ctypes.data, sp.size, 1, cpp,
                                     None if cost is None else cost.ctypes.data,
                                     0 if cost is None else cost.shape[2], max(int(target), 1), int(min_chunks),
                                     items_p, max_items, C.byref(ni), merges_p, max_merges, C.byref(nm),
                                     C.byref(npart), C.byref(big))

    st = plan(None, 0, None, 0)
    if st not in (_lib.DC_OK, _lib.DC_ESPACE):
        _lib.check(st, "dc_plan_decode_fill")
    items = (_lib.WorkItem * max(ni.value, 1))()
    merges = (_lib.MergeItem * max(nm.value, 1))()
    _lib.check(plan(C.addressof(items), ni.value, C.addressof(merges), nm.value), "dc_plan_decode_fill")
    return np.frombuffer(bytes(items), dtype=np.int32).reshape(-1, 8)[: ni.value].copy(), int(big.value)


def make_region_plan(seq_pages, n_kv_heads: int, front, *, device="cuda", chunks_per_page: int = 1, page_cost=None,
                     last_page_tokens=None, target_items: int | None = None, front_items: int | None = None,
                     front_min_chunks: int = 1, window_merge: bool = False,
                     lead_ratio: float | None = None) -> DecodePlan:
    """A fill plan in two launches: pages ``[front[b, 0], front[b, 1])`` of
    every stream of sequence b (``front``: int ``[n_seqs, 2]``, an empty
    range for none) are cut into ``front_items`` items (default: one per
    32-token chunk) that run first, in a launch of their own; the pages
    before and after that range into ``target_items`` items of near-equal
    cost (as :func:`make_plan`), the second launch.  One merge per stream
    then combines the partials of both.  Each launch takes the kernel
    instance of the page formats its own items read, so a stream's few
    pages of another format (an exact fp16 recent window among 4-bit
    pages) do not hold the bulk launch to the instance that reads both
    (``decode_paged``, with page records).  Arguments otherwise as for
    :func:`make_plan` (fill plans only).

    ``window_merge``: no front launch; the merge of every stream attends its
    front pages itself (``dc_window_merge``: fp16 key and value pages, at
    most 256 tokens in 8 pages per stream), so the plan has one merge item
    per stream and one launch.  ``lead_ratio``: the bulk launch as a
    lead-trail plan (:func:`make_plan`)."""
    torch = _torch()
    sp = np.ascontiguousarray(np.asarray(seq_pages, dtype=np.int32))
    if sp.ndim != 1 or sp.size == 0 or np.any(sp <= 0):
        raise ValueError("seq_pages must be a non-empty 1-D array of positive page counts")
    B, H = sp.size, int(n_kv_heads)
    fr = np.asarray(front, dtype=np.int64).reshape(B, 2)
    if np.any(fr[:, 0] < 0) or np.any(fr[:, 1] < fr[:, 0]) or np.any(fr[:, 1] > sp):
        raise ValueError("front ranges must satisfy 0 <= begin <= end <= seq_pages")
    cpp = max(int(chunks_per_page), 1)
    full = 32 * cpp
    last = np.full(B, full, dtype=np.int32) if last_page_tokens is None else np.asarray(last_page_tokens, np.int32)
    if last.shape != (B,):
        raise ValueError("last_page_tokens must have one entry per sequence")
    cost = None if page_cost is None else np.asarray(page_cost, dtype=np.float32)
    if cost is not None and (cost.ndim != 3 or cost.shape[:2] != (B, H) or cost.shape[2] < int(sp.max())):
        raise ValueError("page_cost must have shape [n_seqs, n_kv_heads, >= max pages]")
    target = int(target_items) if target_items else default_target_items()
    if window_merge:
        wtok = [sum(full if p + 1 < sp[b] else int(last[b]) for p in range(int(fr[b, 0]), int(fr[b, 1])))
                for b in range(B)]
        if np.any(fr[:, 1] - fr[:, 0] > 8) or max(wtok) > 256:
            raise ValueError("window_merge: a window holds at most 256 tokens in at most 8 pages")
        if np.any((fr[:, 0] == 0) & (fr[:, 1] == sp)):
            raise ValueError("window_merge: every stream needs pages outside its window")
    key = ("region", sp.tobytes(), H, fr.tobytes(), cpp, None if cost is None else cost.tobytes(), last.tobytes(),
           target, front_items, int(front_min_chunks), bool(window_merge), lead_ratio, str(device))
    hit = _plan_cache.get(key)
    if hit is not None:
        return hit

    def plan_units(units, n_target, min_chunks):
        """units: (b, h, p0, p1) page runs -> host items with real (seq,
        head, pages), or an empty array."""
        if not units:
            return np.zeros((0, 8), dtype=np.int32), 0
        u = np.asarray(units, dtype=np.int64)
        pages = (u[:, 3] - u[:, 2]).astype(np.int32)
        ulast = np.where(u[:, 3] == sp[u[:, 0]], last[u[:, 0]], full).astype(np.int32)
        ucost = None
        if cost is not None:
            ucost = np.zeros((len(u), 1, int(pages.max())), dtype=np.float32)
            for i, (b, h, p0, p1) in enumerate(u):
                ucost[i, 0, : p1 - p0] = cost[b, h, p0:p1]
        it, big = _fill_units(pages, ulast, ucost, cpp, n_target, min_chunks)
        src = u[it[:, 0]]
        it[:, 0], it[:, 1] = src[:, 0], src[:, 1]
        it[:, 2] += src[:, 2].astype(np.int32)
        it[:, 3] += src[:, 2].astype(np.int32)
        return it, big

    front_units = [(b, h, int(fr[b, 0]), int(fr[b, 1])) for b in range(B) for h in range(H) if fr[b, 1] > fr[b, 0]]
    bulk_units = [(b, h, p0, p1) for b in range(B) for h in range(H)
                  for p0, p1 in ((0, int(fr[b, 0])), (int(fr[b, 1]), int(sp[b]))) if p1 > p0]
    if window_merge:
        front_units = []
    if front_items is None:  # one item per chunk that holds tokens
        front_items = sum((p1 - p0 - 1) * cpp + (min(cpp, (int(last[b]) + 31) // 32) if p1 == sp[b] else cpp)
                          for b, h, p0, p1 in front_units)
    f_it, f_big = plan_units(front_units, int(front_items), int(front_min_chunks))
    b_it, b_big = plan_units(bulk_units, max(target // 2, 1) if lead_ratio else target, MIN_CHUNKS_PER_SPLIT)
    if lead_ratio and len(b_it):
        b_it = lead_trail_split(b_it, float(lead_ratio), cpp)
        b_big = int(_item_chunks(b_it, cpp).max())
    items = np.concatenate([f_it, b_it]) if len(f_it) else b_it
    # partial slots: every stream's items (front and bulk) take consecutive
    # slots, merged by one merge item; a stream of one item writes its output
    # (with window_merge every stream has a merge item: it attends the window)
    items, host_merges, n_part = _stream_partials(items, H, force_merge=window_merge)
    merges = host_merges
    dev_items = torch.from_numpy(items.ravel().view(np.uint8).copy()).to(device)
    dev_merges = torch.from_numpy(host_merges.ravel().view(np.uint8).copy()).to(device) if len(merges) else None
    big = max(f_big, b_big)
    plan = DecodePlan(dev_items, dev_merges, len(items), len(merges), n_part, -(-big // cpp), items, host_merges,
                      chunks_per_page=cpp, largest_chunks=big, n_front=len(f_it))
    if window_merge:
        hw = np.ascontiguousarray(fr[host_merges[:, 0]], dtype=np.int32).reshape(-1, 2)
        plan.host_windows = hw
        plan.windows = torch.from_numpy(hw.ravel().view(np.uint8).copy()).to(device) if len(hw) else None
    if len(_plan_cache) > 256:
        _plan_cache.clear()
    _plan_cache[key] = plan
    return plan


_PATHS = {"auto": 0, "generic": 1, "mfma": 2}


def set_decode_path(path: str) -> None:
    """``"auto"`` (MFMA kernel when the pages fit it), ``"generic"``, or
    ``"mfma"`` (the MFMA kernel only: a decode it does not cover raises
    ValueError)."""
    if path not in _PATHS:
        raise ValueError("decode path must be 'auto', 'generic' or 'mfma'")
    _lib.check(_lib.lib().dc_set_decode_path(_PATHS[path]), "dc_set_decode_path")


def set_mfma_head_block(nqb: int) -> None:
    """Smallest head block of the MFMA kernel: 0 (automatic), 4, 8 or 16.
    With a block of 4 or 8 heads the kernel's 16 MFMA slots carry 4 or 2
    copies of the heads, each on its own key / value group; 16 keeps one
    group per MFMA operand (both layouts give the same results to fp32
    rounding)."""
    if nqb not in (0, 4, 8, 16):
        raise ValueError("MFMA head block must be 0, 4, 8 or 16")
    _lib.check(_lib.lib().dc_set_mfma_head_block(int(nqb)), "dc_set_mfma_head_block")


@dataclass
class PageRecords:
    """The key and value descriptors of every page of a plan's items
    (``dc_gather_page_records``), so the MFMA kernel's waves skip the
    page-table and descriptor reads before their first page loads.  A
    snapshot of the plan, both tables and both pools' descriptors: stale,
    and refused by :func:`decode_paged`, once any of them changes.  It also
    holds the formats of the pages the tables reference (``k_mask`` /
    ``v_mask``, ``dc_pool.format_mask`` bits), which :func:`decode_paged`
    passes in place of the pools' masks: the launcher then picks the kernel
    instance for the formats this launch meets (a layer whose key pages are
    all M0 runs the M0-only instance although the pool also holds fp16
    key pages of other layers)."""

    data: object     # device uint8 tensor: n_items x stride x 16 bytes
    stride: int      # records per item (items with more pages read the tables)
    plan: DecodePlan
    sources: tuple   # (k_table, v_table, key pool, value pool), held so their identities stay unique
    versions: tuple  # the tables' and pools' versions at gather time
    k_mask: int = -1  # formats of the referenced key / value pages (-1: the pools' masks)
    v_mask: int = -1
    # region plans (n_front > 0): k_mask / v_mask cover the bulk items'
    # pages, these the front items'
    front_k_mask: int = -1
    front_v_mask: int = -1
    # plans with merge windows: [n_merges][8] (key, value) descriptor pairs
    # of each window's pages, for dc_window_merge
    windows: object = None

    @staticmethod
    def versions_of(k_table, v_table, pool, vpool) -> tuple:
        return (int(k_table._version), int(v_table._version), int(pool.desc_version), int(vpool.desc_version))

    def fresh_for(self, plan, k_table, v_table, pool, vpool) -> bool:
        src = (k_table, v_table, pool, vpool)
        return (self.plan is plan and all(a is b for a, b in zip(self.sources, src))
                and self.versions == PageRecords.versions_of(*src))


def gather_records(pool: DevicePagePool, k_table, v_table, seq_pages, plan: DecodePlan, *,
                   v_pool: DevicePagePool | None = None, stride: int | None = None) -> PageRecords:
    """Page records of ``plan`` over these tables (one launch of
    ``dc_gather_page_records`` on the current stream): as many records per
    item as its largest item has pages, at most ``stride`` (default and
    limit 64); items with more pages read the tables."""
    torch = _torch()
    vpool = pool if v_pool is None else v_pool
    B, H, stride_t = (int(x) for x in k_table.shape)
    sp = np.asarray(seq_pages, dtype=np.int32)
    plan.check(sp, H, stride_t, chunks_per_page(pool.geometry.page_capacity))
    it = np.asarray(plan.host_items, dtype=np.int64).reshape(-1, 8)
    pages = int(np.max(it[:, 3] - it[:, 2])) if len(it) else 1
    rs = int(min(64 if stride is None else max(1, min(int(stride), 64)), max(1, pages)))
    data = torch.empty(max(plan.n_items, 1) * rs * 16, dtype=torch.uint8, device=k_table.device)
    st = _lib.lib().dc_gather_page_records(pool.c_pool(), vpool.c_pool(), C.c_void_p(k_table.data_ptr()),
                                           C.c_void_p(v_table.data_ptr()), stride_t, C.c_void_p(plan.items.data_ptr()),
                                           plan.n_items, B, H, C.c_void_p(data.data_ptr()), rs,
                                           C.c_void_p(current_stream_ptr()))
    _lib.check(st, "dc_gather_page_records")
    # the formats of every page the plan reads (pages [0, seq_pages[b]) of
    # every row; per launch for region plans)
    kt, vt = k_table.cpu().numpy(), v_table.cpu().numpy()
    win = None
    if plan.host_windows is not None:
        check_windows(pool, vpool, kt, vt, plan)
        k_mask, v_mask = items_format_masks(pool, vpool, kt, vt, it)
        fk = fv = -1
        wr = np.zeros((plan.n_merges, 8, 2), dtype=pool.descs_of([0]).dtype)
        for m, ((seq, head, _, _), (pb, pe)) in enumerate(zip(plan.host_merges, plan.host_windows)):
            wr[m, : pe - pb, 0] = pool.descs_of(kt[seq, head, pb:pe])
            wr[m, : pe - pb, 1] = vpool.descs_of(vt[seq, head, pb:pe])
        win = torch.from_numpy(wr.view(np.uint8).ravel().copy()).to(k_table.device)
    elif plan.n_front:
        (fk, fv), (k_mask, v_mask) = (items_format_masks(pool, vpool, kt, vt, part)
                                      for part in (it[: plan.n_front], it[plan.n_front:]))
    else:
        live = np.broadcast_to(np.arange(stride_t)[None, None, :] < sp[:, None, None], kt.shape)
        k_mask = pool.format_mask_of(kt[live]) & pool.format_mask
        v_mask = vpool.format_mask_of(vt[live]) & vpool.format_mask
        fk = fv = -1
    return PageRecords(data, rs, plan, (k_table, v_table, pool, vpool),
                       PageRecords.versions_of(k_table, v_table, pool, vpool), k_mask, v_mask, fk, fv, win)


def merge_windows(pool: DevicePagePool, vpool: DevicePagePool, kt: np.ndarray, vt: np.ndarray,
                  seq_pages) -> np.ndarray | None:
    """Per sequence, pages ``[begin, end)`` of host tables ``kt`` / ``vt``
    that a window merge can attend: the trailing run of fp16 key and value
    pages (a cache's tail or live block, and young pages the recent window
    kept exact), the same for every KV head, at most 8 pages and 256 tokens
    after at least one other page; ``[end, end)`` for a sequence with none.
    None when some sequence's run does not qualify or none has one, or the
    head_dim is not one ``dc_window_merge`` takes."""
    if pool.geometry.head_dim not in (64, 128, 256):
        return None
    f16 = _lib.FMT_M3_F16
    out = np.zeros((kt.shape[0], 2), dtype=np.int64)
    for b in range(kt.shape[0]):
        n = int(seq_pages[b])
        exact = (pool.formats_of(kt[b, :, :n]) == f16) & (vpool.formats_of(vt[b, :, :n]) == f16)
        if not np.all(exact == exact[0]):
            return None
        run = n - int(np.flatnonzero(~exact[0])[-1]) - 1 if not exact[0].all() else n
        begin = n - run
        if run and (begin == 0 or run > 8 or int(pool.tokens_of(kt[b, :, begin:n]).sum(axis=-1).max()) > 256):
            return None
        out[b] = (begin, n)
    return out if np.any(out[:, 1] > out[:, 0]) else None


def plan_decode(pool: DevicePagePool, vpool: DevicePagePool, kt: np.ndarray, vt: np.ndarray, seq_pages, n_q: int, *,
                device="cuda", last_page_tokens=None) -> tuple[DecodePlan, tuple[int, int]]:
    """The fill plan for a decode over host page tables ``kt`` / ``vt``
    (``[n_seqs, n_kv_heads, stride]``) and the format masks of its decode
    launch, for ``decode_paged(plan=..., page_masks=...)``: a region plan
    with merge windows (:func:`merge_windows`) when the sequences end in
    fp16 pages, so the launch takes the kernel instance of the other pages'
    formats; lead-trail items where that instance runs two waves per SIMD."""
    sp = np.asarray(seq_pages, dtype=np.int64)
    H = kt.shape[1]
    cpp = chunks_per_page(pool.geometry.page_capacity)
    front = merge_windows(pool, vpool, kt, vt, sp)
    pg = np.arange(kt.shape[2])[None, None, :]
    read = pg < sp[:, None, None]
    if front is not None:
        read = read & ~((pg >= front[:, 0, None, None]) & (pg < front[:, 1, None, None]))
    read = np.broadcast_to(read, kt.shape)
    masks = (pool.format_mask_of(kt[read]) & pool.format_mask, vpool.format_mask_of(vt[read]) & vpool.format_mask)
    target = launch_target_items(pool, vpool, n_q, *masks)
    lead = launch_lead_ratio(pool, vpool, n_q, *masks)
    if front is not None:
        plan = make_region_plan(sp, H, front, device=device, chunks_per_page=cpp, target_items=target,
                                last_page_tokens=last_page_tokens, window_merge=True, lead_ratio=lead)
    else:
        plan = make_plan(sp, H, device=device, chunks_per_page=cpp, target_items=target,
                         last_page_tokens=last_page_tokens, lead_ratio=lead)
    return plan, masks


def check_windows(pool: DevicePagePool, vpool: DevicePagePool, kt: np.ndarray, vt: np.ndarray, plan: DecodePlan) -> None:
    """Raise ValueError unless every window of ``plan`` (``window_merge``)
    holds only fp16 (M3 f16) key and value pages of equal token counts, the
    only pages ``dc_window_merge`` reads (it skips others), and at most 8
    pages and 256 tokens (it would attend only the first 256)."""
    for (seq, head, _, _), (pb, pe) in zip(np.asarray(plan.host_merges).reshape(-1, 4),
                                           np.asarray(plan.host_windows).reshape(-1, 2)):
        if pe <= pb:
            continue
        kid, vid = kt[seq, head, pb:pe], vt[seq, head, pb:pe]
        pool.validate_ids(kid)
        vpool.validate_ids(vid)
        if (np.any(pool.formats_of(kid) != _lib.FMT_M3_F16) or np.any(vpool.formats_of(vid) != _lib.FMT_M3_F16)
                or not np.array_equal(pool.tokens_of(kid), vpool.tokens_of(vid))):
            raise ValueError("a merge window holds a page that is not an fp16 (M3) key / value page pair")
        if pe - pb > 8 or int(pool.tokens_of(kid).sum()) > 256:
            raise ValueError("a merge window holds more than 8 pages or 256 tokens")


def items_format_masks(pool: DevicePagePool, vpool: DevicePagePool, kt: np.ndarray, vt: np.ndarray,
                       items: np.ndarray) -> tuple[int, int]:
    """``format_mask`` bits of the key and value pages these host work
    items (``[n, 8]``) read from host tables ``kt`` / ``vt``."""
    used = np.zeros(kt.shape, dtype=bool)
    for seq, head, pb, pe in np.asarray(items, dtype=np.int64).reshape(-1, 8)[:, :4]:
        used[seq, head, pb:pe] = True
    if not used.any():
        return 0, 0
    return pool.format_mask_of(kt[used]) & pool.format_mask, vpool.format_mask_of(vt[used]) & vpool.format_mask


def workspace_bytes(plan: DecodePlan, n_q: int, head_dim: int) -> int:
    return int(_lib.lib().dc_decode_workspace_bytes(plan.n_partials, n_q, head_dim))


def decode_paged(
    pool: DevicePagePool,
    k_table,
    v_table,
    seq_pages,
    queries,
    *,
    query_scale: float = 1.0,
    pages_per_split: int | None = None,
    plan: DecodePlan | None = None,
    out=None,
    workspace=None,
    validate: bool = True,
    v_pool: DevicePagePool | None = None,
    merge: bool = True,
    records: PageRecords | None = None,
    page_masks: tuple[int, int] | None = None,
):
    """Fused decode for ``queries [n_seqs, n_kv_heads, n_q, head_dim]``.

    ``pool`` holds the key pages and, unless ``v_pool`` is given, the value
    pages too (the two pools may differ in group size only).

    Returns ``out`` fp32 ``[n_seqs, n_kv_heads, n_q, head_dim]``.
    ``seq_pages[b]`` is the number of pages of sequence b (the first
    entries of its page-table rows).  ``merge=False`` leaves the split-K
    partials in ``workspace`` for :func:`merge_partials` (sequences that
    were not split are written to ``out`` either way).  ``records``: page
    records of ``plan`` (:func:`gather_records`) over these tables and
    pools; stale records raise ValueError.  A region plan
    (``make_region_plan``) runs as two launches: its front items, then the
    rest and the merges.  ``page_masks`` (without records, plans with no
    front items): the ``format_mask`` bits of the key and value pages the
    work items read, when narrower than the pools' (the launch then takes
    the kernel instance of those formats; ``validate`` checks them).
    """
    torch = _torch()
    vpool = pool if v_pool is None else v_pool
    if (vpool.geometry.head_dim, vpool.geometry.page_capacity) != (pool.geometry.head_dim, pool.geometry.page_capacity):
        raise ValueError("key and value pools must share head_dim and page_capacity")
    if queries.dim() != 4:
        raise ValueError("queries must have shape [n_seqs, n_kv_heads, n_q, head_dim]")
    B, H, Q, hd = (int(x) for x in queries.shape)
    if hd != pool.geometry.head_dim:
        raise ValueError("queries head_dim does not match the pool geometry")
    if tuple(k_table.shape[:2]) != (B, H) or tuple(v_table.shape) != tuple(k_table.shape):
        raise ValueError("page tables must have shape [n_seqs, n_kv_heads, table_stride]")
    if k_table.dtype != torch.int32 or v_table.dtype != torch.int32:
        raise ValueError("page tables must be int32")
    sp = np.asarray(seq_pages, dtype=np.int32)
    if sp.shape != (B,):
        raise ValueError("seq_pages must have one entry per sequence")
    stride = int(k_table.shape[2])
    if np.any(sp > stride):
        raise ValueError("seq_pages exceeds the page-table width")
    if validate:
        kt = k_table.cpu().numpy()
        vt = v_table.cpu().numpy()
        for b in range(B):
            ids_k = kt[b, :, : sp[b]]
            ids_v = vt[b, :, : sp[b]]
            pool.validate_ids(ids_k)
            vpool.validate_ids(ids_v)
            if not np.array_equal(pool.tokens_of(ids_k), vpool.tokens_of(ids_v)):
                raise ValueError("key and value pages must hold the same token counts")
    cpp = chunks_per_page(pool.geometry.page_capacity)
    if plan is None:
        last = None
        if validate:  # the host tables are at hand: cut only chunks that hold tokens
            last = np.asarray([pool.tokens_of(kt[b, 0, sp[b] - 1]) for b in range(B)], dtype=np.int32)
        plan = make_plan(sp, H, pages_per_split, device=queries.device, chunks_per_page=cpp,
                         target_items=launch_target_items(pool, vpool, Q), last_page_tokens=last,
                         lead_ratio=launch_lead_ratio(pool, vpool, Q))
    plan.check(sp, H, stride, cpp)
    if not queries.is_contiguous():
        queries = queries.contiguous()
    if out is None:
        out = torch.empty((B, H, Q, hd), dtype=torch.float32, device=queries.device)
    need = workspace_bytes(plan, Q, hd)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=queries.device)
    if records is not None and not records.fresh_for(plan, k_table, v_table, pool, vpool):
        raise ValueError("page records are stale: gather them again after a change to the plan, the page "
                         "tables or the pools' descriptors")
    stream = C.c_void_p(current_stream_ptr())

    def launch(first: int, count: int, with_merges: bool, masks) -> None:
        """Items [first, first + count) in one launch (and the plan's merges
        after it when ``with_merges``); ``masks``: the formats those items
        read, from the page records, or None for the pools' masks."""
        if count == 0:  # (a region plan whose pages are all in front)
            if with_merges and merge:
                merge_partials(plan, out, workspace)
            return
        kp, vp = pool.c_pool(), vpool.c_pool()
        if masks is not None and masks[0] > 0 and masks[1] > 0:
            # (records checked fresh above: the masks are those of these tables' pages)
            kp.format_mask, vp.format_mask = masks
        m_on = with_merges and merge and plan.merges is not None
        args = (kp, vp, C.c_void_p(k_table.data_ptr()), C.c_void_p(v_table.data_ptr()), stride,
                C.c_void_p(plan.items.data_ptr() + 32 * first), count,
                C.c_void_p(plan.merges.data_ptr() if m_on else 0), plan.n_merges if m_on else 0,
                C.c_void_p(queries.data_ptr()), dtype_code(queries), float(query_scale),
                B, H, Q, C.c_void_p(out.data_ptr()), C.c_void_p(workspace.data_ptr()), int(workspace.numel()))
        if records is None:
            st = _lib.lib().dc_decode_paged(*args, stream)
        else:
            st = _lib.lib().dc_decode_paged_records(
                *args, C.c_void_p(records.data.data_ptr() + 16 * records.stride * first), records.stride, stream)
        _lib.check(st, "dc_decode_paged")

    nf = int(plan.n_front)
    if nf:  # region plan: the front items first, with their own formats
        launch(0, nf, False, None if records is None else (records.front_k_mask, records.front_v_mask))
    windowed = plan.host_windows is not None
    if windowed and validate:
        check_windows(pool, vpool, kt, vt, plan)
    masks = None if records is None else (records.k_mask, records.v_mask)
    if masks is None and page_masks is not None:
        if nf:
            raise ValueError("page_masks apply to plans without front items")
        masks = (int(page_masks[0]) & pool.format_mask, int(page_masks[1]) & vpool.format_mask)
        if validate:
            have = items_format_masks(pool, vpool, kt, vt, np.asarray(plan.host_items)[nf:])
            if (have[0] & ~masks[0]) or (have[1] & ~masks[1]):
                raise ValueError("page_masks leave out formats of pages the plan reads")
    launch(nf, plan.n_items - nf, not windowed, masks)
    if windowed and merge:
        merge_partials(plan, out, workspace, window=(pool, vpool, k_table, v_table, queries, query_scale),
                       records=records)
    return out


def merge_partials(plan: DecodePlan, out, workspace, *, window=None, records: PageRecords | None = None) -> None:
    """The split-K log-sum-exp merge of ``plan`` on its own
    (``dc_lse_merge``): partials in ``workspace`` -> ``out``.  A plan with
    merge windows (``make_region_plan(window_merge=True)``) needs
    ``window = (pool, v_pool, k_table, v_table, queries, query_scale)`` of
    its decode: the merge attends those pages too (``dc_window_merge``),
    reading their descriptors from ``records`` (``gather_records`` of the
    plan over those tables) when given."""
    if plan.n_merges == 0:
        return
    B, H, Q, hd = (int(x) for x in out.shape)
    m = np.asarray(plan.host_merges, dtype=np.int64).reshape(-1, 4)
    if np.any((m[:, 0] < 0) | (m[:, 0] >= B)) or np.any((m[:, 1] < 0) | (m[:, 1] >= H)):
        raise ValueError("plan: a merge item names a sequence or KV head outside the output")
    if plan.host_windows is not None:
        if window is None:
            raise ValueError("this plan's merges attend window pages: pass window=(pool, v_pool, k_table, v_table, "
                             "queries, query_scale)")
        pool, vpool, k_table, v_table, queries, query_scale = window
        vpool = pool if vpool is None else vpool
        if tuple(queries.shape) != (B, H, Q, hd) or not queries.is_contiguous():
            raise ValueError("window merge: queries must be contiguous [n_seqs, n_kv_heads, n_q, head_dim]")
        win = None
        if records is not None:
            if not records.fresh_for(plan, k_table, v_table, pool, vpool):
                raise ValueError("page records are stale: gather them again after a change to the plan, the page "
                                 "tables or the pools' descriptors")
            win = records.windows
        st = _lib.lib().dc_window_merge(pool.c_pool(), vpool.c_pool(), C.c_void_p(k_table.data_ptr()),
                                        C.c_void_p(v_table.data_ptr()), int(k_table.shape[2]),
                                        C.c_void_p(plan.merges.data_ptr()), C.c_void_p(plan.windows.data_ptr()),
                                        plan.n_merges, C.c_void_p(queries.data_ptr()), dtype_code(queries),
                                        float(query_scale), B, H, Q, C.c_void_p(out.data_ptr()),
                                        C.c_void_p(workspace.data_ptr()), int(workspace.numel()),
                                        C.c_void_p(win.data_ptr() if win is not None else 0),
                                        C.c_void_p(current_stream_ptr()))
        _lib.check(st, "dc_window_merge")
        return
    st = _lib.lib().dc_lse_merge(C.c_void_p(plan.merges.data_ptr()), plan.n_merges, C.c_void_p(workspace.data_ptr()),
                                 int(workspace.numel()), B, H, Q, hd, C.c_void_p(out.data_ptr()),
                                 C.c_void_p(current_stream_ptr()))
    _lib.check(st, "dc_lse_merge")
