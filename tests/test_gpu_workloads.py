"""The benchmark workloads end to end: pages encoded on the device into the
pools, one fused ``dc_decode_paged`` launch per layer (plus the per-step
append for config 5), checked against the oracle run on the same pages
downloaded from the device.  Reduced sizes cover every configuration; the
full shapes of configs 2 to 5 are checked on sampled (sequence, KV head)
streams."""
import numpy as np
import pytest

from tests.helpers import workload_oracle

pytestmark = pytest.mark.gpu

TOL = 1e-3  # max-abs error bound on the attention output


def _check(wl, layer, pairs):
    out = wl.outs[layer].cpu().numpy()
    for b, h in pairs:
        want = workload_oracle(wl, layer, b, h)
        err = float(np.max(np.abs(out[b, h] - want)))
        assert err < TOL, f"{wl.spec.name} layer {layer} seq {b} head {h}: max-abs error {err}"


@pytest.mark.parametrize("name,context", [("c1", None), ("c2", 700), ("c3", 1500), ("c4", None), ("c5", 1000)])
def test_workload_step_matches_oracle(name, context):
    import torch

    from dotcache_amd.workloads import build_workload

    print(f"workload {name} context {context}", flush=True)
    batch = {"c1": None, "c4": 2}.get(name, 3)
    wl = build_workload(name, seed=3, layers=2, batch=batch, context=context, pages_per_split=2)
    for _ in range(2):  # twice: a step must leave the pools and workspace ready for the next
        wl.step()
    torch.cuda.synchronize()
    B, H = wl.spec.batch, wl.spec.n_kv_heads
    for layer in range(2):
        _check(wl, layer, [(b, h) for b in range(B) for h in range(H)])


def test_workspace_reused_across_plans():
    """One workspace serves plans with different split counts in turn."""
    import torch

    from dotcache_amd.decode import decode_paged, make_plan
    from dotcache_amd.workloads import build_workload

    wl = build_workload("c3", seed=4, layers=1, batch=3, context=1300)
    lt = wl.layers[0]
    H = wl.spec.n_kv_heads
    ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    outs = []
    for pps in (2, None, 3, 1, 2):
        plan = make_plan(lt.seq_pages, H, pps)
        out = decode_paged(wl.k_pool, lt.k_table, lt.v_table, lt.seq_pages, wl.queries[0],
                           query_scale=wl.query_scale, plan=plan, workspace=ws, validate=True, v_pool=wl.v_pool)
        outs.append(out.cpu().numpy())
    for o in outs[1:]:
        assert np.max(np.abs(o - outs[0])) < 2e-5
    wl.outs[0].copy_(torch.from_numpy(outs[0]))
    _check(wl, 0, [(b, h) for b in range(3) for h in range(H)])


def test_full_size_c4_sampled_streams():
    """Config 4 at its full shape (64 ragged sequences of 256..32768 tokens,
    per-(layer, KV head) key modes, int8 values, one layer): the longest and
    the shortest sequence's streams against the oracle."""
    import torch

    from dotcache_amd.workloads import build_workload

    wl = build_workload("c4", seed=0, layers=1)
    wl.step()
    torch.cuda.synchronize()
    sp = np.asarray(wl.layers[0].seq_pages)
    b_long, b_short = int(np.argmax(sp)), int(np.argmin(sp))
    print(f"c4 full: sequences {b_long} ({sp[b_long]} pages) and {b_short} ({sp[b_short]} pages)", flush=True)
    _check(wl, 0, [(b_long, 0), (b_long, 1), (b_short, 1)])


def test_full_size_c5_sampled_stream():
    """Config 5 at its full shape (4 x 131072 tokens, head_dim 256, the
    appended token and the fp16 recent window, one layer): one stream
    against the oracle."""
    import torch

    from dotcache_amd.workloads import build_workload

    wl = build_workload("c5", seed=0, layers=1)
    wl.step()
    torch.cuda.synchronize()
    _check(wl, 0, [(3, 2)])


def test_full_size_c3_sampled_streams():
    """Config 3 at its full shape (batch 8 x 16384 tokens, hd 128, GQA 7,
    one layer): streams of the first and last sequence against the oracle."""
    import torch

    from dotcache_amd.workloads import build_workload

    wl = build_workload("c3", seed=0, layers=1)
    wl.step()
    torch.cuda.synchronize()
    _check(wl, 0, [(0, 0), (0, 3), (7, 1), (7, 2)])


def test_full_size_c2_streams():
    """Config 2 at its bench shape (batch 1, context 4096, page 64, GQA 4,
    head_dim 64, affine 4-bit keys and values) with the bench's plan (a
    launch's item budget of 2-chunk items) and its page records: every KV
    head of two layers against the oracle."""
    import torch

    from dotcache_amd.workloads import build_workload

    wl = build_workload("c2", seed=0, layers=2)
    assert wl.spec.batch == 1 and int(wl.lengths[0]) == 4096 and wl.spec.head_dim == 64
    plan = wl.plans[0]
    assert wl.records, "the workload gathers page records for its plans"
    # 8 streams of 64 pages (128 chunks) in 512 items of 2 chunks
    assert plan.n_items == 512 and plan.largest_chunks == 2, (plan.n_items, plan.largest_chunks)
    print(f"c2 full: {plan.n_items} items per layer, largest {plan.largest_chunks} chunks", flush=True)
    wl.step()
    torch.cuda.synchronize()
    H = wl.spec.n_kv_heads
    for layer in range(2):
        _check(wl, layer, [(0, h) for h in range(H)])


@pytest.mark.parametrize("name,context", [("c2", 700), ("c5", 1000)])
def test_graph_replays_match_eager_steps(name, context):
    """A captured step graph (append, decode and merge kernels of every
    layer) gives the eager step's outputs bit for bit on every replay, with
    eager launches on the same buffers in between."""
    import torch

    from dotcache_amd.workloads import build_workload

    wl = build_workload(name, seed=6, layers=2, batch=3, context=context, pages_per_split=2)
    wl.step()
    torch.cuda.synchronize()
    want = [o.clone() for o in wl.outs]
    wl.capture()
    for rep in range(3):
        for o in wl.outs:
            o.fill_(float("nan"))
        wl.step()
        torch.cuda.synchronize()
        for l, (o, w) in enumerate(zip(wl.outs, want)):
            assert torch.equal(o, w), f"replay {rep} layer {l} differs from the eager step"
        graph, wl.graph = wl.graph, None
        wl.step()  # eager work between replays
        torch.cuda.synchronize()
        wl.graph = graph


def test_kv_sets_cycle_step_by_step():
    """A workload with two KV sets: consecutive steps attend set 0, then set
    1, each layer of each set matching the oracle; the captured graphs (one
    per set) replay the eager outputs bit for bit, in the same order."""
    import torch

    from dotcache_amd.workloads import build_workload

    wl = build_workload("c2", seed=7, layers=2, batch=1, context=300, pages_per_split=2, replicas=2)
    assert wl.replicas == 2 and len(wl.layers) == 4 and list(wl.replica_layers(1)) == [2, 3]
    wl.step()
    wl.step()
    torch.cuda.synchronize()
    B, H = wl.spec.batch, wl.spec.n_kv_heads
    for layer in range(4):
        _check(wl, layer, [(b, h) for b in range(B) for h in range(H)])
    want = [o.clone() for o in wl.outs]
    wl.capture()
    assert wl.next_replica == 0
    for r in (0, 1, 0):
        for o in wl.outs:
            o.fill_(float("nan"))
        wl.step()
        torch.cuda.synchronize()
        for l in wl.replica_layers(r):
            assert torch.equal(wl.outs[l], want[l]), f"set {r} layer {l} differs from the eager step"


@pytest.mark.parametrize("window", ["merge", "launch"])
def test_c5_window_matches_oracle_and_one_launch(window):
    """Config 5's fill plans keep the exact fp16 window out of the decode
    launch (a region plan): attended by the split-K merge ("merge") or by a
    decode launch of its own ("launch"), so the decode launch runs the
    kernel instance of the 4-bit pages.  Every stream of two layers against
    the oracle, and against the same pages decoded in one launch; then the
    captured step graph against the eager step, bit for bit."""
    import torch

    from dotcache_amd.decode import waves_per_simd
    from dotcache_amd.workloads import build_workload

    kw = dict(seed=5, layers=2, batch=3, context=3000)
    wl = build_workload("c5", window=window, **kw)
    plan = wl.plans[0]
    if window == "merge":
        assert plan.n_front == 0 and plan.host_windows is not None and plan.n_merges == 3 * wl.spec.n_kv_heads
        assert np.all(plan.host_windows[:, 1] > plan.host_windows[:, 0])
    else:
        assert plan.n_front > 0, "the window gets its own launch"
    rec = wl.records[0]
    assert waves_per_simd(wl.k_pool, wl.v_pool, wl.spec.gqa, rec.k_mask, rec.v_mask) == 2
    print(f"c5 window {window}: {plan.n_front} front items of {plan.n_items}", flush=True)
    for _ in range(2):
        wl.step()
    torch.cuda.synchronize()
    B, H = wl.spec.batch, wl.spec.n_kv_heads
    for layer in range(2):
        _check(wl, layer, [(b, h) for b in range(B) for h in range(H)])
    one = build_workload("c5", window="none", **kw)
    assert one.plans[0].n_front == 0 and one.plans[0].host_windows is None
    for _ in range(2):
        one.step()
    torch.cuda.synchronize()
    for layer in range(2):
        err = float((wl.outs[layer] - one.outs[layer]).abs().max())
        assert err < 2e-5, f"layer {layer}: window {window} vs one launch differ by {err}"
    want = [o.clone() for o in wl.outs]
    wl.capture()
    for rep in range(3):
        for o in wl.outs:
            o.fill_(float("nan"))
        wl.step()
        torch.cuda.synchronize()
        for l, (o, w) in enumerate(zip(wl.outs, want)):
            # (each step appends the same token again into slot 0 of the tail)
            assert torch.equal(o, w), f"replay {rep} layer {l} differs from the eager step"
        graph, wl.graph = wl.graph, None
        wl.step()
        torch.cuda.synchronize()
        wl.graph = graph
