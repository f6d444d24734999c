"""The allocation-free decode entry point (dc_decode_paged_noalloc) against
dc_decode_paged with a caller workspace: identical outputs on two calls in a
row (the second smaller, so stale partials of the first would show), called
through the C ABI; and its size limit."""
import ctypes as C

import numpy as np
import pytest

from oracle import dotcache_oracle as O
from tests.helpers import hard_values, to_product_page

pytestmark = pytest.mark.gpu


def _case(rng, lens, hd, Q, kfmt, vfmt):
    """Pools, tables, plan and queries of a ragged batch (one KV head per
    sequence), built through the backend's page preparation."""
    import torch

    from dotcache_amd.backends import prepare_pages_hip

    kp, vp = [], []
    for n in lens:
        kp.append(O.encode_pages(hard_values(rng, n, hd), tokens_per_page=64, head_dim=hd, group_size=32, kind="K",
                                 **kfmt))
        vp.append(O.encode_pages(hard_values(rng, n, hd), tokens_per_page=64, head_dim=hd, group_size=32, kind="V",
                                 **vfmt))
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


def _noalloc(case, plan, out):
    from dotcache_amd import _lib
    from dotcache_amd.page_pool import current_stream_ptr

    B, H, Q, hd = (int(x) for x in case["q"].shape)
    return _lib.lib().dc_decode_paged_noalloc(
        case["kpool"].c_pool(), case["vpool"].c_pool(), C.c_void_p(case["kt"].data_ptr()),
        C.c_void_p(case["vt"].data_ptr()), int(case["kt"].shape[2]), C.c_void_p(plan.items.data_ptr()), plan.n_items,
        C.c_void_p(plan.merges.data_ptr() if plan.merges is not None else 0), plan.n_merges, plan.n_partials,
        C.c_void_p(case["q"].data_ptr()), _lib.DT_F32, 1.0, B, H, Q, C.c_void_p(out.data_ptr()),
        C.c_void_p(current_stream_ptr()))


@pytest.mark.parametrize("kfmt,vfmt,hd,Q", [
    (dict(mode="M3"), dict(bits=4, scheme="symmetric"), 128, 7),  # the C3 formats (MFMA kernel)
    (dict(bits=2), dict(bits=3), 64, 3),                           # generic kernel
])
def test_noalloc_matches_workspace_decode_twice(kfmt, vfmt, hd, Q):
    import torch

    from dotcache_amd import _lib
    from dotcache_amd.backends import clear_prepared_pools
    from dotcache_amd.decode import chunks_per_page, decode_paged, make_plan

    clear_prepared_pools()
    rng = np.random.default_rng(hd + Q)
    for lens in ([64 * 9 + 17, 30, 64 * 4, 1000], [64 * 3 + 5, 64]):  # the second call is smaller
        case = _case(rng, lens, hd, Q, kfmt, vfmt)
        cpp = chunks_per_page(case["kpool"].geometry.page_capacity)
        plans = {
            "2 pages per split": make_plan(case["counts"], 1, 2, device="cuda"),
            # items cut at 32-token chunks inside pages
            "fill": make_plan(case["counts"], 1, device="cuda", target_items=7, chunks_per_page=cpp),
        }
        for name, plan in plans.items():
            assert plan.n_merges > 0
            ref = decode_paged(case["kpool"], case["kt"], case["vt"], case["counts"], case["q"], plan=plan,
                               v_pool=case["vpool"])
            out = torch.full_like(ref, float("nan"))
            _lib.check(_noalloc(case, plan, out), "dc_decode_paged_noalloc")
            torch.cuda.synchronize()
            assert torch.equal(out, ref), f"lens {lens} plan {name}: max diff {(out - ref).abs().max().item()}"
            assert np.max(np.abs(out.cpu().numpy()[:, 0] - case["want"])) < 3e-4
    clear_prepared_pools()


def test_noalloc_rejects_partials_beyond_its_scratch():
    from dotcache_amd import _lib

    L = _lib.lib()
    cap = int(L.dc_decode_noalloc_scratch_bytes())
    assert cap == 32 << 20
    geo = _lib.geometry(256, 32, 64)
    pool = _lib.Pool(None, 0, None, 0, geo, 0)
    per_partial = 16 * (256 + 2) * 4
    too_many = cap // per_partial + 1
    st = L.dc_decode_paged_noalloc(pool, pool, None, None, 1, None, 0, None, 0, too_many, None, _lib.DT_F32, 1.0,
                                   1, 1, 16, None, None)
    assert st == _lib.DC_ESPACE
    assert b"static scratch" in L.dc_last_error()
    # the largest count that fits passes the size check (nothing to run: no items)
    assert L.dc_decode_paged_noalloc(pool, pool, None, None, 1, None, 0, None, 0, too_many - 1, None, _lib.DT_F32,
                                     1.0, 1, 1, 16, None, None) == _lib.DC_OK
