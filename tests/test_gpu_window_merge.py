"""The split-K merge that also attends a stream's fp16 pages
(``dc_window_merge``, region plans with ``window_merge=True``), against the
oracle: windows of one or two pages (the second partly filled) with 4-bit
pages before and after them, a stream with no window, every head_dim the
merge takes, and fp32 / fp16 / bf16 queries."""
import numpy as np
import pytest

from oracle import dotcache_oracle as O
from tests.helpers import hard_values, to_product_page

pytestmark = pytest.mark.gpu

TOL = 1e-3  # max-abs error bound on the attention output


@pytest.fixture(autouse=True)
def fresh_pools():
    from dotcache_amd.backends import clear_prepared_pools

    clear_prepared_pools()
    yield
    clear_prepared_pools()


def _stream(rng, hd, tpp, n_before, win_tokens, n_after_tokens, kind, group):
    """Pages of one stream: n_before full 4-bit pages, fp16 pages holding
    win_tokens tokens, then 4-bit pages of n_after_tokens tokens."""
    kw = dict(head_dim=hd, group_size=group, kind=kind)
    m0 = dict(bits=4, scheme="affine" if kind == "K" else "symmetric")
    pages = []
    if n_before:
        pages += O.encode_pages(hard_values(rng, n_before * tpp, hd), tokens_per_page=tpp, **kw, **m0)
    if win_tokens:
        pages += O.encode_pages(rng.normal(size=(win_tokens, hd)).astype(np.float32) * 3, tokens_per_page=tpp,
                                mode="M3", **kw)
    if n_after_tokens:
        pages += O.encode_pages(hard_values(rng, n_after_tokens, hd), tokens_per_page=tpp, **kw, **m0)
    return pages


@pytest.mark.parametrize("hd,qdtype", [(256, "bfloat16"), (128, "float16"), (64, "float32"), (256, "float32")])
def test_window_merge_matches_oracle(hd, qdtype):
    import torch

    from dotcache_amd.backends import prepare_pages_hip
    from dotcache_amd.decode import decode_paged, gather_records, make_region_plan

    rng = np.random.default_rng(hd + len(qdtype))
    tpp, H, Q = 128, 2, 4
    # (pages before, window tokens, tokens after): a one-page window, a
    # window of a full and a partial page, one with no window
    layout = [(5, 128, 1), (3, 200, 70), (4, 0, 90)]
    kp, vp, front = [], [], []
    for b, (nb, wt, na) in enumerate(layout):
        for h in range(H):
            kp.append(_stream(rng, hd, tpp, nb, wt, na, "K", 32))
            vp.append(_stream(rng, hd, tpp, nb, wt, na, "V", 32))
        front.append((nb, nb + (-(-wt // tpp))))
    kprep = prepare_pages_hip([to_product_page(p) for g in kp for p in g])
    vprep = prepare_pages_hip([to_product_page(p) for g in vp for p in g])
    counts = [len(kp[b * H]) for b in range(len(layout))]
    width = max(counts)
    kt = np.zeros((len(layout), H, width), np.int32)
    vt = np.zeros((len(layout), H, width), np.int32)
    off = 0
    for s, g in enumerate(kp):
        n = len(g)
        kt[s // H, s % H, :n] = [p.page_id for p in kprep[off:off + n]]
        vt[s // H, s % H, :n] = [p.page_id for p in vprep[off:off + n]]
        off += n
    q32 = (rng.normal(size=(len(layout), H, Q, hd)) / np.sqrt(hd)).astype(np.float32)
    q = torch.from_numpy(q32).cuda().to(getattr(torch, qdtype))
    want = O.decode_grouped(q.float().cpu().numpy().reshape(-1, Q, hd), kp, vp).reshape(len(layout), H, Q, hd)
    pool, vpool = kprep[0].pool, vprep[0].pool
    ktd, vtd = torch.from_numpy(kt).cuda(), torch.from_numpy(vt).cuda()
    last = np.asarray([pool.tokens_of(kt[b, 0, counts[b] - 1]) for b in range(len(layout))], np.int32)
    plan = make_region_plan(counts, H, np.asarray(front), device="cuda", chunks_per_page=4, last_page_tokens=last,
                            target_items=24, window_merge=True)
    assert plan.n_front == 0 and plan.n_merges == len(layout) * H
    ws = torch.zeros(1 << 22, dtype=torch.uint8, device="cuda")
    out = decode_paged(pool, ktd, vtd, counts, q, plan=plan, workspace=ws, v_pool=vpool, validate=True)
    err = float(np.max(np.abs(out.cpu().numpy() - want)))
    assert err < TOL, f"hd {hd} {qdtype}: window merge vs oracle {err}"
    rec = gather_records(pool, ktd, vtd, counts, plan, v_pool=vpool)
    out2 = decode_paged(pool, ktd, vtd, counts, q, plan=plan, workspace=ws, v_pool=vpool, validate=False, records=rec)
    assert torch.equal(out, out2), "page records change the result"


def test_window_merge_rejects_non_fp16_windows():
    """A window naming a 4-bit page is refused on the host."""
    import torch

    from dotcache_amd.backends import prepare_pages_hip
    from dotcache_amd.decode import decode_paged, make_region_plan

    rng = np.random.default_rng(0)
    hd, tpp = 128, 128
    kp = _stream(rng, hd, tpp, 3, 0, 10, "K", 32)
    vp = _stream(rng, hd, tpp, 3, 0, 10, "V", 32)
    kprep = prepare_pages_hip([to_product_page(p) for p in kp])
    vprep = prepare_pages_hip([to_product_page(p) for p in vp])
    kt = torch.tensor([[[p.page_id for p in kprep]]], dtype=torch.int32).cuda()
    vt = torch.tensor([[[p.page_id for p in vprep]]], dtype=torch.int32).cuda()
    q = torch.zeros((1, 1, 2, hd), dtype=torch.float32).cuda()
    plan = make_region_plan([4], 1, np.array([[1, 2]]), device="cuda", chunks_per_page=4, window_merge=True,
                            last_page_tokens=np.array([10], np.int32))
    with pytest.raises(ValueError, match="fp16"):
        decode_paged(kprep[0].pool, kt, vt, [4], q, plan=plan, v_pool=vprep[0].pool, validate=True)


def test_window_bound_holds_on_every_head():
    """merge_windows bounds a window's tokens on every KV head: here head
    0's fp16 run holds 120 tokens and head 1's 276, past the 256 a window
    merge attends, so plan_decode takes a plan without windows, and the
    decode still matches the oracle."""
    import torch

    from dotcache_amd.backends import prepare_pages_hip
    from dotcache_amd.decode import decode_paged, merge_windows, plan_decode

    rng = np.random.default_rng(7)
    hd, Q = 128, 3
    kw = dict(head_dim=hd, group_size=32)

    def head_pages(kind, win):  # one full 4-bit page, then fp16 pages of these token counts
        m0 = dict(bits=4, scheme="affine" if kind == "K" else "symmetric")
        pages = O.encode_pages(hard_values(rng, 256, hd), tokens_per_page=256, kind=kind, **kw, **m0)
        for t in win:
            pages += O.encode_pages(rng.normal(size=(t, hd)).astype(np.float32), tokens_per_page=t, mode="M3",
                                    kind=kind, **kw)
        return pages

    kp = [head_pages("K", (100, 20)), head_pages("K", (256, 20))]
    vp = [head_pages("V", (100, 20)), head_pages("V", (256, 20))]
    kprep = prepare_pages_hip([to_product_page(p) for g in kp for p in g])
    vprep = prepare_pages_hip([to_product_page(p) for g in vp for p in g])
    pool, vpool = kprep[0].pool, vprep[0].pool
    kt = np.asarray([p.page_id for p in kprep], np.int32).reshape(1, 2, 3)
    vt = np.asarray([p.page_id for p in vprep], np.int32).reshape(1, 2, 3)
    assert merge_windows(pool, vpool, kt, vt, [3]) is None
    plan, masks = plan_decode(pool, vpool, kt, vt, [3], Q, device="cuda", last_page_tokens=np.array([20], np.int32))
    assert plan.host_windows is None
    q32 = (rng.normal(size=(1, 2, Q, hd)) / np.sqrt(hd)).astype(np.float32)
    want = O.decode_grouped(q32.reshape(-1, Q, hd), kp, vp).reshape(1, 2, Q, hd)
    out = decode_paged(pool, torch.from_numpy(kt).cuda(), torch.from_numpy(vt).cuda(), [3], torch.from_numpy(q32).cuda(),
                       plan=plan, v_pool=vpool, page_masks=masks)
    err = float(np.max(np.abs(out.cpu().numpy() - want)))
    assert err < TOL, f"decode vs oracle {err}"
