"""Work items that start and end inside pages (32-token chunk cuts) on both
decode kernels, against the oracle: cuts from the fill planner with page
costs, and random cuts that put an item inside a single page, on an empty
page, or past a partial page's last valid chunk."""
import numpy as np
import pytest

from oracle import dotcache_oracle as O
from tests.helpers import hard_values, to_product_page

pytestmark = pytest.mark.gpu

KERNEL_TOL = 1e-3  # max-abs error bound on the attention output


@pytest.fixture(autouse=True)
def fresh_pools():
    from dotcache_amd.backends import clear_prepared_pools
    from dotcache_amd.decode import set_decode_path

    clear_prepared_pools()
    set_decode_path("auto")
    yield
    set_decode_path("auto")
    clear_prepared_pools()


def _case(rng, lens, hd, Q, tpp, kfmt, vfmt, vgs, empty_at=None):
    """Pools, tables and queries of a ragged batch (one KV head per
    sequence); ``empty_at = (b, i)`` inserts a page with no tokens at
    position i of sequence b."""
    import torch

    from dotcache_amd.backends import prepare_pages_hip

    kp, vp = [], []
    for n in lens:
        kp.append(O.encode_pages(hard_values(rng, n, hd), tokens_per_page=tpp, head_dim=hd, group_size=32, kind="K",
                                 **kfmt))
        vp.append(O.encode_pages(hard_values(rng, n, hd), tokens_per_page=tpp, head_dim=hd, group_size=vgs, kind="V",
                                 **vfmt))
    if empty_at is not None:
        b, i = empty_at
        kp[b].insert(i, O.encode_page(np.zeros((0, hd), np.float32), head_dim=hd, group_size=32, kind="K", **kfmt))
        vp[b].insert(i, O.encode_page(np.zeros((0, hd), np.float32), head_dim=hd, group_size=vgs, kind="V", **vfmt))
    kprep = prepare_pages_hip([to_product_page(p) for g in kp for p in g])
    vprep = prepare_pages_hip([to_product_page(p) for g in vp for p in g])
    counts = [len(g) for g in kp]
    width = max(counts)
    kt = np.zeros((len(lens), 1, width), np.int32)
    vt = np.zeros((len(lens), 1, width), np.int32)
    off = 0
    for b, n in enumerate(counts):
        kt[b, 0, :n] = [p.page_id for p in kprep[off:off + n]]
        vt[b, 0, :n] = [p.page_id for p in vprep[off:off + n]]
        off += n
    q = torch.from_numpy((rng.normal(size=(len(lens), 1, Q, hd)) / np.sqrt(hd)).astype(np.float32)).cuda()
    return dict(kpool=kprep[0].pool, vpool=vprep[0].pool, kt=torch.from_numpy(kt).cuda(),
                vt=torch.from_numpy(vt).cuda(), counts=np.asarray(counts, np.int32), q=q, keep=(kprep, vprep),
                want=O.decode_grouped(q.cpu().numpy()[:, 0], kp, vp))


def _random_plan(rng, counts, cpp, cuts_per_stream):
    """A plan cutting each stream's chunks [0, pages * cpp) at random
    distinct chunk positions."""
    import torch

    from dotcache_amd.decode import DecodePlan

    items, merges, n_part = [], [], 0
    for b, n in enumerate(counts):
        length = int(n) * cpp
        k = min(cuts_per_stream, length - 1)
        cuts = [0] + sorted(rng.choice(np.arange(1, length), size=k, replace=False).tolist()) + [length]
        first = n_part
        for u0, u1 in zip(cuts[:-1], cuts[1:]):
            part = n_part if len(cuts) > 2 else -1
            items.append([b, 0, u0 // cpp, -(-u1 // cpp), part, u0 % cpp, u1 % cpp, 0])
            if part >= 0:
                n_part += 1
        if len(cuts) > 2:
            merges.append([b, 0, first, len(cuts) - 1])
    it = np.asarray(items, np.int32)
    ms = np.asarray(merges, np.int32).reshape(-1, 4)
    dev_items = torch.from_numpy(it.ravel().view(np.uint8).copy()).cuda()
    dev_merges = torch.from_numpy(ms.ravel().view(np.uint8).copy()).cuda() if len(ms) else None
    return DecodePlan(dev_items, dev_merges, len(it), len(ms), n_part, 0, it, ms, chunks_per_page=cpp)


def _decode(case, plan):
    from dotcache_amd.decode import decode_paged

    out = decode_paged(case["kpool"], case["kt"], case["vt"], case["counts"], case["q"], plan=plan,
                       v_pool=case["vpool"])
    return out.cpu().numpy()[:, 0]


CASES = [
    # keys through LDS (config 3 formats), 64-token pages: two chunks per page
    (dict(mode="M3"), dict(bits=4, scheme="symmetric"), 32, 128, 7, 64),
    # pipelined mixed-format pools (config 4 formats): 16-byte key pieces
    (dict(bits=4), dict(bits=8, scheme="symmetric"), 64, 128, 6, 64),
    # head_dim 256, 128-token pages: four chunks per page (config 5 formats)
    (dict(bits=4), dict(bits=4), 32, 256, 4, 128),
    # 2- and 3-bit codes: the generic kernel only
    (dict(bits=2), dict(bits=3), 32, 64, 3, 96),
]


@pytest.mark.parametrize("path", ["auto", "generic"])
@pytest.mark.parametrize("kfmt,vfmt,vgs,hd,Q,tpp", CASES)
def test_chunk_cut_plans_match_oracle(kfmt, vfmt, vgs, hd, Q, tpp, path):
    """Full pages (the kernel's fast chunk walk) and ragged pages with an
    empty page (its prefix-sum walk), items of more than one 64-page
    metadata batch, planner cuts under random page costs, and random cuts."""
    from dotcache_amd.decode import chunks_per_page, make_plan, set_decode_path

    set_decode_path(path)
    rng = np.random.default_rng(hd + tpp + vgs)
    layouts = {
        "full": dict(lens=[tpp * 9, tpp * 70, tpp * 3, tpp], empty_at=None),
        "ragged": dict(lens=[tpp * 9 - 5, tpp * 70 + 1, 33, 1], empty_at=(1, 66)),
    }
    for name, lay in layouts.items():
        print(f"path {path} hd {hd} tpp {tpp} layout {name}", flush=True)
        case = _case(rng, lay["lens"], hd, Q, tpp, kfmt, vfmt, vgs, lay["empty_at"])
        counts = case["counts"]
        cpp = chunks_per_page(case["kpool"].geometry.page_capacity)  # pools may round the page capacity up
        plans = []
        for target in (5, 9, 23):
            cost = rng.uniform(0.2, 3.0, size=(len(counts), 1, int(counts.max()))).astype(np.float32)
            plans.append((f"fill {target}", make_plan(counts, 1, device="cuda", target_items=target,
                                                      chunks_per_page=cpp, page_cost=cost)))
        for ratio in (1.6, 3.0):  # lead-trail plans (instances at two waves per SIMD)
            plans.append((f"lead-trail {ratio}", make_plan(counts, 1, device="cuda", target_items=18,
                                                           chunks_per_page=cpp, lead_ratio=ratio)))
        for cuts in (1, 3, 12):
            plans.append((f"random {cuts}", _random_plan(rng, counts, cpp, cuts)))
        if cpp > 1:
            cut = np.concatenate([p.host_items[:, 5:7] for _, p in plans])
            assert np.any(cut[:, 0] != 0) and np.any(cut[:, 1] != 0)
        for label, plan in plans:
            err = float(np.max(np.abs(_decode(case, plan) - case["want"])))
            assert err < KERNEL_TOL, f"path {path} layout {name} plan {label}: max-abs error {err}"


def test_single_page_items_and_empty_items():
    """Items inside one page (chunks [1, 3) of a 4-chunk page), items made
    only of a partial page's missing chunks (they write an empty partial),
    and whole-page items in one plan, on the MFMA kernel."""
    import torch

    from dotcache_amd.decode import DecodePlan, set_decode_path

    set_decode_path("mfma")
    rng = np.random.default_rng(77)
    hd, Q, tpp, cpp = 256, 4, 128, 4
    case = _case(rng, [tpp * 3 + 20, tpp * 2], hd, Q, tpp, dict(bits=4), dict(bits=4), 32)
    # sequence 0: 4 pages, the last with 20 tokens (one valid chunk of four)
    items = [
        [0, 0, 0, 1, 0, 0, 1, 0],    # page 0, chunk 0
        [0, 0, 0, 1, 1, 1, 3, 0],    # page 0, chunks 1-2
        [0, 0, 0, 2, 2, 3, 2, 0],    # page 0 chunk 3 to page 1 chunk 1
        [0, 0, 1, 4, 3, 2, 1, 0],    # page 1 chunk 2 to page 3 chunk 0 (its only valid chunk)
        [0, 0, 3, 4, 4, 1, 0, 0],    # page 3 chunks 1-3: no valid tokens, an empty partial
        [1, 0, 0, 2, -1, 0, 0, 0],   # sequence 1 whole
    ]
    it = np.asarray(items, np.int32)
    ms = np.asarray([[0, 0, 0, 5]], np.int32)
    plan = DecodePlan(torch.from_numpy(it.ravel().view(np.uint8).copy()).cuda(),
                      torch.from_numpy(ms.ravel().view(np.uint8).copy()).cuda(), len(it), 1, 5, 0, it, ms,
                      chunks_per_page=cpp)
    err = float(np.max(np.abs(_decode(case, plan) - case["want"])))
    assert err < KERNEL_TOL, f"max-abs error {err}"


@pytest.mark.parametrize("records", [False, True])
def test_first_chunk_cases_on_the_dma_key_instance(records):
    """The config 3 instance (M3 keys by DMA, pipelined) issues an item's
    first chunk before its batch layout when the item's first page holds
    it.  Items here start inside a page (chunk 1 of 2), end inside one,
    start on a partial page's missing chunk (no valid tokens: an empty
    partial) or on an empty page, beside a whole-sequence item; through
    the tables and through page records."""
    import torch

    from dotcache_amd.decode import DecodePlan, decode_paged, gather_records, set_decode_path

    set_decode_path("mfma")
    rng = np.random.default_rng(91)
    hd, Q, tpp, cpp = 128, 7, 64, 2
    # sequence 0: 4 pages, the last with 20 tokens (chunk 1 of it empty);
    # sequence 1: an empty page, then 2 full pages
    case = _case(rng, [tpp * 3 + 20, tpp * 2], hd, Q, tpp, dict(mode="M3"), dict(bits=4, scheme="symmetric"), 32,
                 empty_at=(1, 0))
    items = [
        [0, 0, 0, 1, 0, 0, 1, 0],    # page 0, chunk 0
        [0, 0, 0, 1, 1, 1, 0, 0],    # page 0, chunk 1
        [0, 0, 1, 3, 2, 0, 1, 0],    # page 1 to page 2 chunk 0
        [0, 0, 2, 4, 3, 1, 1, 0],    # page 2 chunk 1 to page 3 chunk 0 (its only valid chunk)
        [0, 0, 3, 4, 4, 1, 0, 0],    # page 3 chunk 1: no valid tokens, an empty partial
        [1, 0, 0, 3, -1, 0, 0, 0],   # sequence 1 whole, starting on its empty page
    ]
    it = np.asarray(items, np.int32)
    ms = np.asarray([[0, 0, 0, 5]], np.int32)
    plan = DecodePlan(torch.from_numpy(it.ravel().view(np.uint8).copy()).cuda(),
                      torch.from_numpy(ms.ravel().view(np.uint8).copy()).cuda(), len(it), 1, 5, 0, it, ms,
                      chunks_per_page=cpp)
    args = (case["kpool"], case["kt"], case["vt"], case["counts"])
    rec = gather_records(*args, plan, v_pool=case["vpool"]) if records else None
    got = decode_paged(*args, case["q"], plan=plan, v_pool=case["vpool"], records=rec).cpu().numpy()[:, 0]
    err = float(np.max(np.abs(got - case["want"])))
    assert err < KERNEL_TOL, f"records {records}: max-abs error {err}"


@pytest.mark.parametrize("kfmt,vfmt,vgs,hd,Q,tpp", CASES[:3])
def test_page_records_give_the_same_outputs(kfmt, vfmt, vgs, hd, Q, tpp):
    """Decode with page records (every item's descriptors gathered ahead)
    equals the decode through the tables bit for bit, with records covering
    every item or only the items of at most 3 pages; records go stale when
    a table or a pool's descriptors change."""
    import torch

    from dotcache_amd.decode import chunks_per_page, decode_paged, gather_records, make_plan

    rng = np.random.default_rng(500 + hd)
    case = _case(rng, [tpp * 9 - 5, tpp * 70 + 1, 33, 1], hd, Q, tpp, kfmt, vfmt, vgs, empty_at=(1, 66))
    counts = case["counts"]
    cpp = chunks_per_page(case["kpool"].geometry.page_capacity)
    args = (case["kpool"], case["kt"], case["vt"], counts)
    for plan in (make_plan(counts, 1, device="cuda", target_items=23, chunks_per_page=cpp),
                 make_plan(counts, 1, 3, device="cuda")):
        want = decode_paged(*args, case["q"], plan=plan, v_pool=case["vpool"]).clone()
        for stride in (None, 3):
            rec = gather_records(*args, plan, v_pool=case["vpool"], stride=stride)
            got = decode_paged(*args, case["q"], plan=plan, v_pool=case["vpool"], records=rec)
            assert torch.equal(got, want), f"stride {stride}: max diff {(got - want).abs().max().item()}"
            assert np.max(np.abs(got.cpu().numpy()[:, 0] - case["want"])) < KERNEL_TOL
    # stale: another plan, a table written in place, a pool's descriptors changed
    rec = gather_records(*args, plan, v_pool=case["vpool"])
    other = make_plan(counts, 1, 2, device="cuda")
    with pytest.raises(ValueError):
        decode_paged(*args, case["q"], plan=other, v_pool=case["vpool"], records=rec)
    case["kt"][0, 0, 0] = case["kt"][0, 0, 0]
    with pytest.raises(ValueError):
        decode_paged(*args, case["q"], plan=plan, v_pool=case["vpool"], records=rec)
    rec = gather_records(*args, plan, v_pool=case["vpool"])
    pid = int(case["kt"][2, 0, 0].item())
    case["kpool"].set_tokens([pid], case["kpool"].tokens_of([pid]))
    with pytest.raises(ValueError):
        decode_paged(*args, case["q"], plan=plan, v_pool=case["vpool"], records=rec)


def test_page_records_narrow_the_format_mask():
    """Page records carry the formats of the pages their tables reference.
    A batch whose key pages are all M0, in a pool that also holds fp16 key
    pages of another batch, then runs the M0-only kernel instance: within
    1e-4 of the mixed-format instance (which it gets without records; two
    instances need not round alike) and within the bound of the oracle; the
    other batch keeps the fp16 bit."""
    from dotcache_amd import _lib
    from dotcache_amd.decode import chunks_per_page, decode_paged, gather_records, make_plan

    rng = np.random.default_rng(808)
    vfmt = dict(bits=8, scheme="symmetric")
    m0 = _case(rng, [64 * 9 - 5, 64 * 30 + 1, 33], 128, 6, 64, dict(bits=4), vfmt, 64)
    m3 = _case(rng, [64 * 5, 70], 128, 6, 64, dict(mode="M3"), vfmt, 64)
    pool = m0["kpool"]
    assert m3["kpool"] is pool and m3["vpool"] is m0["vpool"], "both batches share the pools"
    m3_bit = _lib.format_bit(_lib.FMT_M3_F16, 0)
    assert pool.format_mask & m3_bit
    cpp = chunks_per_page(pool.geometry.page_capacity)
    for case, has_m3 in ((m0, False), (m3, True)):
        counts = case["counts"]
        args = (pool, case["kt"], case["vt"], counts)
        plan = make_plan(counts, 1, device="cuda", target_items=11, chunks_per_page=cpp)
        rec = gather_records(*args, plan, v_pool=case["vpool"])
        assert rec.k_mask != 0 and (rec.k_mask & ~pool.format_mask) == 0
        assert bool(rec.k_mask & m3_bit) == has_m3
        assert rec.v_mask == case["vpool"].format_mask
        want = decode_paged(*args, case["q"], plan=plan, v_pool=case["vpool"]).clone()
        got = decode_paged(*args, case["q"], plan=plan, v_pool=case["vpool"], records=rec)
        diff = float((got - want).abs().max().item())
        assert diff < 1e-4, f"fp16 keys {has_m3}: records against tables, max diff {diff}"
        err = float(np.max(np.abs(got.cpu().numpy()[:, 0] - case["want"])))
        assert err < KERNEL_TOL, f"fp16 keys {has_m3}: max-abs error {err}"
