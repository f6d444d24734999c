"""Decode-attention throughput on compressed KV pages (one MI355X).

A step is one decode step of the whole model: for every layer, one fused
``dc_decode_paged`` launch over the whole batch (plus, for workloads with
append, the encode/append of the new token).  Inputs are resident in HBM
before timing starts.  Prints ONE JSON line on stdout; progress goes to
stderr.

    python bench.py [--steps K] [--warmup W] [--config c3] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0
METRIC = "KV tokens attended/s + HBM GB/s (% of 8 TB/s peak), 7B GQA, 16K ctx, batch 8"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c3", choices=["c1", "c2", "c3", "c4", "c5"])
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--pages-per-split", type=int, default=None)
    ap.add_argument("--no-page-records", action="store_true",
                    help="decode through the page tables instead of page records gathered ahead")
    ap.add_argument("--contiguous-pages", action="store_true",
                    help="keep each sequence's pages in allocation order instead of scattering them over the pool")
    ap.add_argument("--decode-path", default="auto", choices=["auto", "generic", "mfma"],
                    help="auto: the MFMA kernel where the pages fit it; generic: the VALU kernel only; "
                         "mfma: the MFMA kernel only (an error where it does not fit)")
    ap.add_argument("--head-block", type=int, default=0, choices=[0, 4, 8, 16],
                    help="smallest head block of the MFMA kernel (0: automatic; 16: one key / value group "
                         "per MFMA operand)")
    ap.add_argument("--key-bits", type=int, default=None,
                    help="re-code the configuration's M0 key pages at this width (a variant, not the "
                         "configuration's own line)")
    ap.add_argument("--eager", action="store_true",
                    help="launch every kernel from Python each step instead of replaying captured HIP graphs")
    ap.add_argument("--window", default="merge", choices=["merge", "launch", "none"],
                    help="where an exact recent window (c5) is attended: in the split-K merge (default), in a "
                         "decode launch of its own, or in the same decode launch as the 4-bit pages")
    ap.add_argument("--front-items", type=int, default=None,
                    help="items of the exact window's launch (default: one per 32-token chunk)")
    ap.add_argument("--lead-ratio", type=float, default=None,
                    help="lead-trail plans for two-waves-per-SIMD instances with this lead/trail ratio "
                         "(default: the library's; 0: plain plans)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--shortlist-pages", type=int, default=0, metavar="N",
                    help="only time the execution shortlist kernels: relevance of N pages (4-row sketches, "
                         "head_dim 128) and the top-k of one min(N, 2048)-page stream; prints its own JSON line")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--encode-probe", action="store_true",
                    help="only time the bulk page encode (dc_encode_rows_kv) of one C3 layer: the keys of 8 x 16384 "
                         "tokens x 4 KV heads into M3 fp16 pages and the values into M0 symmetric int4 g32 pages; "
                         "prints its own JSON line")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only copy a BYTES-sized device buffer three times and exit: the known-size "
                         "transfer that calibrates the FETCH_SIZE / WRITE_SIZE counters")
    return ap.parse_args()


def profiled_traffic(workload: str, plan: str, pages_per_split: int, decode_path: str, head_block: int,
                     window: str | None = None):
    """HBM bytes per decode launch measured for this workload and plan by
    the FETCH_SIZE / WRITE_SIZE runs summarised under profiles/ (calibrated
    against a copy of known size there), or None if none matches."""
    import re

    for f in sorted((ROOT / "profiles").glob("*.md")):
        for m in re.finditer(r"<!-- traffic (\{.*?\}) -->", f.read_text()):
            rec = json.loads(m.group(1))
            if (rec.get("workload"), rec.get("plan"), rec.get("pages_per_split"), rec.get("decode_path"),
                    rec.get("head_block"), rec.get("window")) == (workload, plan, pages_per_split, decode_path,
                                                                 head_block, window):
                return float(rec["traffic_bytes"])
    return None


def shortlist_probe(n_pages: int, steps: int) -> None:
    """Time dc_page_relevance over n_pages 4-row fp32 sketches (an HBM-bound
    GEMV: 4 x 128 x 4 bytes per page) and dc_select_top_k over one stream of
    min(n_pages, 2048) pages (k = 64), each replayed ``steps`` times between
    events."""
    import ctypes as C

    import torch

    from dotcache_amd import _lib
    from dotcache_amd.page_pool import current_stream_ptr

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(0)
    # the top-k ranks the first n_tk of the relevance scores: never more than exist
    S, hd, k = 4, 128, 64
    n_tk = min(2048, n_pages)
    sk = torch.randn((n_pages, S, hd), device=dev, generator=g)
    lo = torch.randn((n_pages, hd), device=dev, generator=g)
    hi = lo + 1.0
    q = torch.randn(hd, device=dev, generator=g)
    scores = torch.empty(n_pages, device=dev)
    cand = torch.ones(n_tk, dtype=torch.uint8, device=dev)
    sel = torch.empty(n_tk, dtype=torch.uint8, device=dev)
    L = _lib.lib()
    stream = C.c_void_p(current_stream_ptr())

    def relevance():
        _lib.check(L.dc_page_relevance(C.c_void_p(sk.data_ptr()), S, C.c_void_p(lo.data_ptr()), C.c_void_p(hi.data_ptr()),
                                       0, C.c_void_p(q.data_ptr()), hd, n_pages, C.c_void_p(scores.data_ptr()), stream),
                   "dc_page_relevance")

    def topk():
        _lib.check(L.dc_select_top_k(C.c_void_p(scores.data_ptr()), C.c_void_p(cand.data_ptr()), n_tk, k,
                                     C.c_void_p(sel.data_ptr()), stream), "dc_select_top_k")

    out = {}
    for name, fn in (("relevance", relevance), ("top_k", topk)):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            fn()
        b.record()
        torch.cuda.synchronize()
        out[name] = a.elapsed_time(b) * 1e3 / steps
    nbytes = n_pages * S * hd * 4
    print(json.dumps({"metric": "execution shortlist: pages scored/s", "value": n_pages / (out["relevance"] * 1e-6),
                      "unit": "pages/s", "relevance_us": out["relevance"], "relevance_bytes": nbytes,
                      "relevance_hbm_frac": nbytes / (out["relevance"] * 1e-6) / (HBM_PEAK_GBPS * 1e9),
                      "top_k_us": out["top_k"], "top_k_pages": n_tk, "k": k, "steps": steps}), flush=True)


def encode_probe(steps: int) -> None:
    """Bulk encode of one C3 layer in one dc_encode_rows_kv launch: 524,288
    fp32 key rows into M3 fp16 pages and as many value rows into M0 symmetric
    4-bit group-32 pages (head_dim 128, 64-token pages), timed over
    ``steps`` launches between events.  Bytes per row: the 512-byte fp32 row
    read, plus the page bytes written (256 for the key, 64 code bytes and
    8 scale bytes for the value)."""
    import torch

    from dotcache_amd import _lib
    from dotcache_amd.page_pool import DevicePagePool, PoolGeometry

    dev = torch.device("cuda", 0)
    B, H, T, hd, P = 8, 4, 16384, 128, 64
    n = B * H * T
    g = torch.Generator(device=dev).manual_seed(0)
    k = torch.randn((n, hd), device=dev, generator=g)
    v = torch.randn((n, hd), device=dev, generator=g)
    kp = DevicePagePool(PoolGeometry(hd, 32, P), device=dev, reserve_bytes=n // P * 16384 + (1 << 20),
                        reserve_pages=n // P + 16)
    vp = DevicePagePool(PoolGeometry(hd, 32, P), device=dev, reserve_bytes=n // P * 4608 + (1 << 20),
                        reserve_pages=n // P + 16)
    kid = kp.allocate(_lib.FMT_M3_F16, 0, n // P, tokens=P)
    vid = vp.allocate(_lib.FMT_M0_SYMMETRIC, 4, n // P, tokens=P)
    rows = torch.arange(n, device=dev, dtype=torch.int64)
    kpage = torch.from_numpy(kid).to(dev)[rows // P].contiguous()
    vpage = torch.from_numpy(vid).to(dev)[rows // P].contiguous()
    slots = (rows % P).to(torch.int32).contiguous()

    def run():
        kp.encode_rows_with(vp, k, v, kpage, slots, vpage, slots)

    for _ in range(3):
        run()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record()
    for i in range(steps):
        run()
        ev[i + 1].record()
    torch.cuda.synchronize()
    us = np.array([ev[i].elapsed_time(ev[i + 1]) * 1e3 for i in range(steps)])
    nbytes = n * (512 + 256) + n * (512 + 64 + 8)
    mean = float(us.mean())
    print(json.dumps({"metric": "bulk page encode (dc_encode_rows_kv, one C3 layer)", "value": 2 * n / (mean * 1e-6),
                      "unit": "rows/s", "launch_us": mean, "launch_us_median": float(np.median(us)),
                      "rows": 2 * n, "bytes_per_launch": nbytes,
                      "hbm_gbps": nbytes / (mean * 1e-6) / 1e9,
                      "hbm_frac": nbytes / (mean * 1e-6) / (HBM_PEAK_GBPS * 1e9), "steps": steps}), flush=True)


def copy_probe(nbytes: int) -> None:
    import torch

    src = torch.ones(nbytes, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copied {nbytes} bytes x3")


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# token positions of one (sequence, KV head) stream that a CPU sample slice
# covers at most (config 3's whole stream), so that one slice of a 131K-token
# config 5 stream stays a few seconds of oracle time
CPU_SLICE_TOKENS = 16384


def _oracle_worker_init():
    """Imports of an all-cores baseline worker, done before the clock starts."""
    import threadpoolctl  # noqa: F401

    from oracle import dotcache_oracle  # noqa: F401


def _oracle_stream_worker(job):
    """One worker of the all-cores baseline: decode every stream of ``job``
    (oracle pages and queries, every GQA head) with BLAS on one thread,
    starting at wall-clock time ``start_at``; returns (tokens, end time)."""
    from threadpoolctl import threadpool_limits

    from oracle import dotcache_oracle as O

    streams, start_at = job
    while time.time() < start_at:  # every worker starts together
        time.sleep(0.0005)
    tokens = 0
    with threadpool_limits(limits=1):
        for qs, kp, vp in streams:
            for q in qs:
                O.decode_step(q, kp, vp)
            tokens += sum(p.header.token_count for p in kp)
    return tokens, time.time()


def cpu_baseline(wl, budget_s: float, all_cores: bool = True) -> dict:
    """Time the CPU oracle (numpy restatement of the reference cpu_ref path:
    per page score, one global softmax, per page mix, one query head at a
    time) on a bounded sample of the same workload: layer 0's (sequence, KV
    head) streams in order, every GQA query head of each, each stream cut to
    at most CPU_SLICE_TOKENS tokens.  Two slices of the same streams check
    that the cost per token position is linear in the context: first each
    stream cut to half its slice (a third of the budget), then the whole
    slices (the rest).  One (sequence, layer, token) position covers all KV
    heads, so a rate is tokens done / KV heads / seconds; ``value`` is the
    whole-slice rate on one core.  ``all_cores``: the same slices spread over
    one worker process per visible CPU (at most 16, the GPU box's share),
    each on one BLAS thread, timed by the wall clock from a common start."""
    import multiprocessing as mp

    from threadpoolctl import threadpool_limits

    from oracle import dotcache_oracle as O

    spec = wl.spec
    lt = wl.layers[0]
    H, Q, P = spec.n_kv_heads, spec.gqa, spec.page_size
    cap_pages = max(1, -(-CPU_SLICE_TOKENS // P))
    q_all = wl.queries[0].float().cpu().numpy() * wl.query_scale  # [B, H, Q, hd]

    def to_oracle(pool, pid, kind):
        page = pool.download_page(int(pid), kind=kind)
        oh = O.OracleHeader(**page.header.to_dict())
        return O.OraclePage(header=oh, payload=page.payload, scales=page.scales, bias=page.bias,
                            escape_payload=page.escape_payload, escape_scales=page.escape_scales)

    def stream(b, h, fraction):
        n = min(int(lt.seq_pages[b]), cap_pages)
        keep = max(1, int(round(n * fraction)))
        kt = lt.k_table[b].cpu().numpy()
        vt = lt.v_table[b].cpu().numpy()
        kp = [to_oracle(wl.k_pool, kt[h, p], "K") for p in range(keep)]
        vp = [to_oracle(wl.v_pool, vt[h, p], "V") for p in range(keep)]
        return [q_all[b, h, j] for j in range(Q)], kp, vp

    order = [(b, h) for b in range(spec.batch) for h in range(H)]

    def run(fraction: float, budget: float):
        tokens = streams = 0
        dt = 0.0
        for b, h in order:
            qs, kp, vp = stream(b, h, fraction)
            t0 = time.perf_counter()
            for q in qs:
                O.decode_step(q, kp, vp)
            dt += time.perf_counter() - t0
            tokens += sum(p.header.token_count for p in kp)
            streams += 1
            if dt > budget:
                break
        return tokens, streams, dt

    with threadpool_limits(limits=1):
        t_half, s_half, dt_half = run(0.5, budget_s / 3)
        tokens, streams, dt = run(1.0, budget_s * 2 / 3)
    rate = tokens / H / dt
    rate_half = t_half / H / dt_half
    out = {
        "value": rate,
        "unit": "KV tokens/s",
        "cores": 1,
        "kind": "port",
        "cpu_model": cpu_model(),
        "host_cpus": os.cpu_count(),
        "linearity": {"half_context_tokens_per_s": rate_half, "full_context_tokens_per_s": rate,
                      "ratio_full_over_half": rate / rate_half},
        "sample": f"layer 0: {streams} (sequence, KV head) streams of at most {cap_pages * P} tokens x {Q} query "
                  f"heads, {tokens} tokens, {dt:.1f} s of oracle time (page downloads excluded), after {s_half} "
                  f"streams cut to half that ({t_half} tokens, {dt_half:.1f} s) for the linearity check; numpy "
                  f"oracle of reference cpu_ref, one thread (BLAS pinned to 1), on {cpu_model()} "
                  f"({os.cpu_count()} cpus visible)",
    }
    if all_cores:
        workers = max(1, min(os.cpu_count() or 1, 16))
        per = max(1, -(-max(streams, 2) // 2))  # about half the one-core sample per worker
        jobs = []
        for w in range(workers):
            picks = [order[(w * per + i) % len(order)] for i in range(per)]
            jobs.append([stream(b, h, 1.0) for b, h in picks])
        # fresh interpreters (spawn: started as child programs, with no GPU
        # state), their imports done by the initializer before the clock
        ctx = mp.get_context("spawn")
        with ctx.Pool(workers, initializer=_oracle_worker_init) as pool:
            pool.map(abs, range(4 * workers), chunksize=1)
            start_at = time.time() + 2.0  # jobs are pickled and handed out meanwhile
            res = pool.map(_oracle_stream_worker, [(j, start_at) for j in jobs], chunksize=1)
        done = sum(r[0] for r in res)
        wall = max(r[1] for r in res) - start_at  # common start to the last worker's end
        out["all_cores"] = {
            "value": done / H / wall,
            "cores": workers,
            "sample": f"{workers} worker processes x {per} streams each (the one-core slices), {done} tokens, "
                      f"{wall:.1f} s wall from a common start to the last worker's end, one BLAS thread per worker",
        }
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (every box here has one GPU). "
              "The path shards by (sequence, KV head) with no exchange between GPUs.", file=sys.stderr)
        sys.exit(2)
    import torch

    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.shortlist_pages:
        shortlist_probe(args.shortlist_pages, max(args.steps, 1))
        return
    if args.encode_probe:
        encode_probe(max(args.steps, 1))
        return

    from dotcache_amd.decode import set_decode_path, set_mfma_head_block
    from dotcache_amd.workloads import SPECS, build_workload

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    t0 = time.time()
    log(f"building workload {args.config} ...")
    set_decode_path(args.decode_path)
    set_mfma_head_block(args.head_block)
    wl = build_workload(args.config, seed=args.seed, pages_per_split=args.pages_per_split,
                        scatter_pages=not args.contiguous_pages, key_bits=args.key_bits,
                        window=args.window, front_items=args.front_items,
                        lead_ratio="auto" if args.lead_ratio is None else (args.lead_ratio or None))
    spec = wl.spec
    # "fill": per-layer plans of a launch's item budget cut at 32-token chunks
    # by page cost; "pages": --pages-per-split whole-page splits
    plan_kind = "fill" if args.pages_per_split is None else "pages"
    if args.no_page_records:
        wl.records = []
    log(f"built in {time.time() - t0:.1f} s: {wl.plan.n_items} work items/layer, pages/split {wl.plan.pages_per_split}, "
        f"K pool {wl.k_pool.arena.numel() / 1e9:.2f} GB, V pool {wl.v_pool.arena.numel() / 1e9:.2f} GB")

    if not args.eager:
        wl.capture()  # the whole step (every layer's kernels) as one HIP graph
    for _ in range(args.warmup):
        wl.step()
    torch.cuda.synchronize()

    # All events are recorded on torch's current stream, the stream the
    # library's kernels are launched on.  Nothing is recorded between the
    # kernels of a step: an event between two kernels costs more than the
    # gap it measures.
    L = spec.n_layers

    def timed(fn, n):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        for _ in range(n):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b)

    def per_call(fn, n, lead=0):
        """ms of each of n calls, from events recorded between the calls
        (each call is a whole graph replay: never between kernels); `lead`
        untimed calls are queued right before the first event, so the timed
        calls do not start from an idle GPU."""
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
        torch.cuda.synchronize()
        for _ in range(lead):
            fn()
        ev[0].record()
        for i in range(n):
            fn()
            ev[i + 1].record()
        torch.cuda.synchronize()
        return np.array([ev[i].elapsed_time(ev[i + 1]) for i in range(n)])

    # (1) the benchmark proper: exactly K whole steps between two syncs
    ms_step = timed(wl.step, args.steps) / args.steps
    # (1b) the per-step distribution: >= 50 steps, an event between steps
    n_med = max(50, args.steps)
    step_ms = per_call(wl.step, n_med)

    # (2) the dominant kernel alone: the decode launches of a step back to
    # back (partials left in the workspace), then (3) the merges alone; each
    # as a graph of one step's launches (unless --eager), so that a short
    # kernel is not timed at the host's launch rate; medians over >= 50
    # replays, an event between replays
    # (the KV sets are cycled here as in the steps, so every launch reads
    # its pages from HBM)
    R = wl.replicas
    # each kernel-only graph holds at least 28 launches (the layers of `reps`
    # consecutive KV sets), so that a short replay is not timed at the host's
    # graph-launch rate (C1 has one launch per step)
    reps = max(1, -(-28 // L))

    def decode_set(r):
        for k in range(reps):
            for l in wl.replica_layers((r + k) % R):
                wl.decode_kernel(l)

    def merge_set(r):
        for k in range(reps):
            for l in wl.replica_layers((r + k) % R):
                wl.merge_kernel(l)

    if args.eager:
        dec_fns = [lambda r=r: decode_set(r) for r in range(R)]
        merge_fns = [lambda r=r: merge_set(r) for r in range(R)]
    else:
        dec_fns = [wl.capture_fn(lambda r=r: decode_set(r)).replay for r in range(R)]
        merge_fns = [wl.capture_fn(lambda r=r: merge_set(r)).replay for r in range(R)]

    def cycling(fns):
        turn = [0]

        def call():
            fns[turn[0] % len(fns)]()
            turn[0] += 1

        return call

    decode_all, merge_all = cycling(dec_fns), cycling(merge_fns)
    # untimed warm-up replays of the freshly captured graphs (a graph's first
    # replays carry its upload and first-launch costs), and a few more queued
    # right before each timed region: after the host's synchronisation the
    # first replays of a region measured up to 18 % slower (C3: 37.6, 34.6,
    # 34.2 ... down to 31.9 us per launch over the first ten replays)
    for fn in dec_fns + merge_fns:
        for _ in range(max(3, args.warmup)):
            fn()
    torch.cuda.synchronize()
    lead = max(10, args.warmup)
    dec_ms = per_call(decode_all, n_med, lead) / (L * reps)
    merge_ms_all = per_call(merge_all, n_med, lead) / (L * reps)
    # roofline.achieved uses the mean launch time (what a kernel trace's
    # average gives); the median is reported beside it
    launch_ms = float(np.mean(dec_ms))
    merge_ms = float(np.mean(merge_ms_all))

    bytes_step = wl.algorithmic_bytes_per_step()
    pos_step = wl.token_positions_per_step()
    value = pos_step / (ms_step / 1e3)
    ms_step_median = float(np.median(step_ms))
    gbps = bytes_step / (ms_step / 1e3) / 1e9
    # (the decode launches read every page but those the merges attend)
    win_bytes = wl.window_bytes_per_step()
    bytes_launch = (bytes_step - win_bytes) / L
    achieved = bytes_launch / (launch_ms / 1e3) / 1e9
    log(f"{ms_step:.3f} ms/step (median {ms_step_median:.3f} over {n_med}), {value / 1e9:.3f} G tokens/s, "
        f"{gbps:.0f} GB/s over the step; "
        f"decode kernel {launch_ms * 1e3:.1f} us -> {achieved:.0f} GB/s ({achieved / HBM_PEAK_GBPS:.1%} of peak), "
        f"merge {merge_ms * 1e3:.1f} us")

    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU oracle baseline ...")
        cpu = cpu_baseline(wl, args.cpu_seconds)
        log(f"cpu baseline {cpu['value']:.0f} tokens/s ({cpu['sample']})"
            + (f"; all cores {cpu['all_cores']['value']:.0f} tokens/s ({cpu['all_cores']['sample']})" if "all_cores" in cpu else ""))

    fmt = lambda f: f"{f.mode} fp16" if f.mode == "M3" else f"M0 {f.scheme} int{f.bits} g{f.group_size}"
    line = {
        "metric": METRIC,
        "value": value,
        "unit": "KV tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "ms_per_step_median": ms_step_median,
        "ms_per_step_p10_p90": [float(np.percentile(step_ms, 10)), float(np.percentile(step_ms, 90))],
        "median_steps": n_med,
        "value_at_median_step": pos_step / (ms_step_median / 1e3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded; K/V encoded on device into compressed pages)",
        "config": {
            "workload": spec.name,
            "layers": L,
            "kv_sets": wl.replicas,
            "batch": spec.batch,
            "context": int(spec.context) if spec.ragged is None else f"log-uniform {spec.ragged}",
            "q_heads": spec.n_q_heads,
            "kv_heads": spec.n_kv_heads,
            "head_dim": spec.head_dim,
            "page_size": spec.page_size,
            "key_pages": fmt(spec.key) + (f", {spec.key_m3_fraction:.0%} streams M3" if spec.key_m3_fraction else ""),
            "value_pages": fmt(spec.value),
            "append": spec.append,
            "plan": plan_kind,
            "page_records": bool(wl.records),
            "pages_per_split": wl.plan.pages_per_split,
            "decode_launches_per_layer": 2 if wl.plan.n_front else 1,
            "lead_ratio": max((r for r in wl.lead_ratios if r), default=None),
            "window": args.window if spec.recent_window else None,
            "launch": "eager" if args.eager else "hip graph of the whole step",
            "parallelism": "single GPU",
        },
        "hbm_gbps": gbps,
        "hbm_pct_of_peak": 100.0 * gbps / HBM_PEAK_GBPS,
        "bytes_per_step": bytes_step,
        "token_positions_per_step": pos_step,
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBPS,
            "traffic": profiled_traffic(spec.name, plan_kind, wl.plan.pages_per_split, args.decode_path,
                                        args.head_block, args.window if spec.recent_window else None),
            "kernel": ("decode_generic_kernel" if args.decode_path == "generic" else "decode_mfma_kernel")
                      + (" (dc_decode_paged: the exact window's launch, then the rest's; launch_us is both)"
                         if wl.plan.n_front else " (dc_decode_paged, one launch per layer"
                         + ("; the exact window is read by the merge)" if wl.plan.host_windows is not None else ")")),
            "launch_us": launch_ms * 1e3,
            "launch_us_stat": f"mean over {n_med} replays of {L * reps} decode launches ({reps} step(s) of {L}; "
                              "event per replay)",
            "launch_us_median": float(np.median(dec_ms)) * 1e3,
            "launch_us_p10_p90": [float(np.percentile(dec_ms, 10)) * 1e3, float(np.percentile(dec_ms, 90)) * 1e3],
            "frac_at_median_launch": bytes_launch / (float(np.median(dec_ms)) / 1e3) / 1e9 / HBM_PEAK_GBPS,
            "bytes_per_launch": bytes_launch,
            "merge_window_bytes_per_layer": win_bytes / L,
            "merge_us": merge_ms * 1e3,
            "decode_path": args.decode_path,
            "head_block": args.head_block,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
