"""GPU read-path parity against the oracle: score_page / mix_page /
decode_step through the backend surface, and the fused paged decode
(GQA, split-K, ragged batches, mixed per-page formats)."""
import numpy as np
import pytest

from oracle import dotcache_oracle as O
from tests.helpers import hard_values, to_product_page

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def fresh_pools():
    """Every test prepares into fresh pools, so the formats one test puts in a
    pool never change which decode kernel another test gets."""
    from dotcache_amd.backends import clear_prepared_pools
    from dotcache_amd.decode import set_decode_path, set_mfma_head_block

    clear_prepared_pools()
    set_decode_path("auto")
    set_mfma_head_block(0)
    yield
    set_decode_path("auto")
    set_mfma_head_block(0)
    clear_prepared_pools()


FORMATS = [
    dict(mode="M0", scheme="affine", bits=4),
    dict(mode="M0", scheme="symmetric", bits=4),
    dict(mode="M0", scheme="symmetric", bits=8),
    dict(mode="M0", scheme="affine", bits=2),
    dict(mode="M0", scheme="affine", bits=3),
    dict(mode="M3", scheme="affine", bits=4),
    dict(mode="M3", scheme="affine", bits=4, escape_dtype="int8"),
]


def _pages(x, tpp, hd, gs, kind, fmt):
    return O.encode_pages(x, tokens_per_page=tpp, head_dim=hd, group_size=gs, kind=kind, **fmt)


@pytest.mark.parametrize("fmt", FORMATS, ids=lambda f: "-".join(str(v) for v in f.values()))
def test_score_and_mix_page_match_oracle(fmt):
    from dotcache_amd import attention_runtime as rt

    rng = np.random.default_rng(901)
    hd, gs = 128, 32
    k = hard_values(rng, 64, hd)
    q = rng.normal(size=hd).astype(np.float32)
    page = O.encode_page(k, head_dim=hd, group_size=gs, kind="K", **fmt)
    got = rt.score_page(q, to_product_page(page), backend="hip_mi355x")
    np.testing.assert_allclose(got, O.score_page_ref(q, page), atol=1e-4, rtol=1e-4)
    w = O.softmax(rng.normal(size=64).astype(np.float32))
    acc = rng.normal(size=hd).astype(np.float32)
    got_mix = rt.mix_page(w, to_product_page(page), out_acc=acc, backend="hip_mi355x")
    np.testing.assert_allclose(got_mix, acc + O.mix_page_ref(w, page), atol=1e-4, rtol=1e-4)


def test_decode_step_matches_cpu_reference():
    """Reference tests/test_torch_cuda_backend.py:53-79 shape: hd 128, 160 tokens."""
    from dotcache_amd import attention_runtime as rt

    rng = np.random.default_rng(902)
    hd = 128
    keys = rng.normal(size=(160, hd)).astype(np.float32)
    values = rng.normal(size=(160, hd)).astype(np.float32)
    q = rng.normal(size=hd).astype(np.float32)
    kp = _pages(keys, 64, hd, 32, "K", dict(bits=4))
    vp = _pages(values, 64, hd, 32, "V", dict(bits=4))
    want = O.decode_step(q, kp, vp)
    got = rt.decode_step(q, [to_product_page(p) for p in kp], [to_product_page(p) for p in vp], backend="hip_mi355x")
    np.testing.assert_allclose(got[0], want[0], atol=1e-4, rtol=1e-4)
    np.testing.assert_allclose(got[1], want[1], atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(got[2], want[2], atol=1e-4, rtol=1e-4)


def test_score_pages_splits_per_page():
    from dotcache_amd.backends import score_pages_hip

    rng = np.random.default_rng(903)
    keys = rng.normal(size=(150, 64)).astype(np.float32)
    q = rng.normal(size=64).astype(np.float32)
    kp = _pages(keys, 64, 64, 32, "K", dict(bits=4))
    got = score_pages_hip(q, [to_product_page(p) for p in kp])
    assert [g.shape[0] for g in got] == [64, 64, 22]
    for g, p in zip(got, kp):
        np.testing.assert_allclose(g, O.score_page_ref(q, p), atol=1e-4, rtol=1e-4)


def _grouped_case(rng, hd, gs, Q, n_tokens, kfmt, vfmt, tpp=64):
    G = len(n_tokens)
    qs = rng.normal(size=(G, Q, hd)).astype(np.float32)
    kpg, vpg = [], []
    for n in n_tokens:
        kpg.append(_pages(hard_values(rng, n, hd), tpp, hd, gs, "K", kfmt))
        vpg.append(_pages(hard_values(rng, n, hd), tpp, hd, gs, "V", vfmt))
    return qs, kpg, vpg


@pytest.mark.parametrize("kfmt,vfmt,hd,gs,Q", [
    (dict(mode="M3"), dict(bits=4, scheme="symmetric"), 128, 32, 7),           # C3 formats
    (dict(bits=4), dict(bits=4), 64, 32, 4),                                    # C2 formats
    (dict(bits=4), dict(bits=8, scheme="symmetric"), 128, 64, 6),               # C4 V format (g64)
    (dict(bits=4), dict(bits=4), 256, 32, 4),                                   # C5 formats
    (dict(bits=2), dict(bits=3), 128, 32, 3),
    (dict(mode="M3", escape_dtype="int8"), dict(mode="M3", escape_dtype="float32"), 64, 32, 16),
])
def test_fused_output_only_matches_oracle(kfmt, vfmt, hd, gs, Q):
    from dotcache_amd.backends import decode_grouped_multiquery_step_prepared_hip_tensor_output_only as fused

    rng = np.random.default_rng(hd + Q)
    qs, kpg, vpg = _grouped_case(rng, hd, gs, Q, [1000, 64, 130], kfmt, vfmt)
    qs = qs / np.sqrt(hd)
    want = O.decode_grouped(qs, kpg, vpg)
    kp = [[to_product_page(p) for p in g] for g in kpg]
    vp = [[to_product_page(p) for p in g] for g in vpg]
    for pps in (None, 1, 3):
        got = fused(list(qs), kp, vp, pages_per_split=pps).cpu().numpy()
        np.testing.assert_allclose(got, want, atol=1e-3, rtol=0)
        assert np.max(np.abs(got - want)) < 2e-4


@pytest.mark.parametrize("kbits", [4, 8])
def test_fused_mixed_key_formats_per_page(kbits):
    """Selective key precision: M3 and M0 key pages interleaved in one list,
    on the MFMA kernel."""
    from dotcache_amd.backends import decode_grouped_multiquery_step_prepared_hip_tensor_output_only as fused
    from dotcache_amd.decode import set_decode_path

    set_decode_path("mfma")
    rng = np.random.default_rng(77 + kbits)
    hd, n = 128, 640
    keys = hard_values(rng, n, hd)
    vals = hard_values(rng, n, hd)
    kp = []
    for i, s in enumerate(range(0, n, 64)):
        fmt = dict(mode="M3") if i % 3 == 1 else dict(bits=kbits, scheme="affine" if i % 2 else "symmetric")
        kp.append(O.encode_page(keys[s:s + 64], head_dim=hd, group_size=32, kind="K", token_start=s, **fmt))
    vp = _pages(vals, 64, hd, 64, "V", dict(bits=8, scheme="symmetric"))  # V group 64, K group 32 (config 4)
    q = (rng.normal(size=(1, 6, hd)) / np.sqrt(hd)).astype(np.float32)
    want = O.decode_grouped(q, [kp], [vp])
    got = fused(list(q), [[to_product_page(p) for p in kp]], [[to_product_page(p) for p in vp]]).cpu().numpy()
    np.testing.assert_allclose(got, want, atol=2e-4, rtol=0)


@pytest.mark.parametrize("hd", [64, 128, 256])
@pytest.mark.parametrize("kbits", [4, 8])
def test_fused_mixed_key_and_value_formats_every_head_dim(hd, kbits):
    """M3 and M0 pages interleaved in both the key and the value lists, at
    every head_dim the MFMA kernel takes, with a partial last page: the M3
    key and value rows reach LDS by DMA in their slot swizzle (3 bits at
    head_dim 64, 4 above) and the rows past the page's tokens must not
    contribute.  Compared at the kernels' tolerance, with automatic head
    blocks and with blocks of 16."""
    from dotcache_amd.backends import decode_grouped_multiquery_step_prepared_hip_tensor_output_only as fused
    from dotcache_amd.decode import set_decode_path, set_mfma_head_block

    set_decode_path("mfma")
    rng = np.random.default_rng(900 + hd + kbits)
    tpp, n, Q = 64, 9 * 64 - 23, 4
    keys = hard_values(rng, n, hd)
    vals = hard_values(rng, n, hd)
    kp, vp = [], []
    for i, s in enumerate(range(0, n, tpp)):
        kf = dict(mode="M3") if i % 3 == 2 else dict(bits=kbits, scheme="affine" if i % 2 else "symmetric")
        vf = dict(mode="M3") if i % 4 in (1, 3) or s + tpp >= n else dict(bits=4, scheme="affine")
        kp.append(O.encode_page(keys[s:s + tpp], head_dim=hd, group_size=32, kind="K", token_start=s, **kf))
        vp.append(O.encode_page(vals[s:s + tpp], head_dim=hd, group_size=32, kind="V", token_start=s, **vf))
    q = (rng.normal(size=(1, Q, hd)) / np.sqrt(hd)).astype(np.float32)
    want = O.decode_grouped(q, [kp], [vp])
    args = (list(q), [[to_product_page(p) for p in kp]], [[to_product_page(p) for p in vp]])
    for nqb in (0, 16):
        set_mfma_head_block(nqb)
        for pps in (None, 2):
            got = fused(*args, pages_per_split=pps).cpu().numpy()
            err = np.max(np.abs(got - want))
            assert err < KERNEL_TOL, f"head block {nqb} pps {pps}: max-abs error {err}"


def test_four_and_eight_bit_keys_in_one_pool_take_the_generic_kernel():
    """The MFMA kernel takes one key code width per launch: a pool holding
    both runs on the generic kernel under "auto", and path "mfma" refuses it."""
    from dotcache_amd.backends import decode_grouped_multiquery_step_prepared_hip_tensor_output_only as fused
    from dotcache_amd.decode import set_decode_path

    rng = np.random.default_rng(48)
    hd, n = 128, 320
    keys = hard_values(rng, n, hd)
    kp = [O.encode_page(keys[s:s + 64], head_dim=hd, group_size=32, kind="K", token_start=s, bits=4 if i % 2 else 8)
          for i, s in enumerate(range(0, n, 64))]
    vp = _pages(hard_values(rng, n, hd), 64, hd, 32, "V", dict(bits=4))
    q = (rng.normal(size=(1, 4, hd)) / np.sqrt(hd)).astype(np.float32)
    want = O.decode_grouped(q, [kp], [vp])
    args = (list(q), [[to_product_page(p) for p in kp]], [[to_product_page(p) for p in vp]])
    got = fused(*args).cpu().numpy()
    assert np.max(np.abs(got - want)) < KERNEL_TOL
    set_decode_path("mfma")
    with pytest.raises(ValueError, match="MFMA kernel does not cover"):
        fused(*args)


FAST_CASES = [
    # (key format, value format, head_dim, value group, n_q, page tokens): every BASELINE shape
    (dict(mode="M3"), dict(bits=4, scheme="symmetric"), 128, 32, 7, 64),          # config 3
    (dict(bits=4), dict(bits=4), 64, 32, 4, 64),                                   # config 2
    (dict(bits=4, scheme="symmetric"), dict(bits=4, scheme="symmetric"), 64, 32, 1, 64),  # config 1
    (dict(bits=4), dict(bits=8, scheme="symmetric"), 128, 64, 6, 64),              # config 4
    (dict(bits=4), dict(bits=4), 256, 32, 4, 128),                                 # config 5
    (dict(mode="M3"), dict(mode="M3"), 128, 32, 8, 64),
    (dict(bits=4, scheme="symmetric"), dict(bits=8), 128, 32, 5, 96),
    # 8-bit keys: specialised instances at head_dim 128, group 32 values
    (dict(bits=8), dict(bits=4), 128, 32, 6, 64),
    (dict(bits=8), dict(bits=8), 128, 32, 8, 64),
    # head blocks of 4 with a dead head in every copy
    (dict(bits=4), dict(bits=4), 128, 32, 3, 64),
    (dict(bits=8), dict(bits=4), 128, 32, 2, 64),
    # and the general instances (symmetric keys, other shapes)
    (dict(bits=8, scheme="symmetric"), dict(bits=8, scheme="symmetric"), 128, 32, 4, 64),
    (dict(bits=8), dict(bits=8, scheme="symmetric"), 128, 64, 6, 64),
    (dict(bits=8), dict(bits=4, scheme="symmetric"), 64, 32, 3, 64),
    (dict(bits=8, scheme="symmetric"), dict(bits=4), 256, 32, 4, 128),
    # capacity 256 at head_dim 256: 8-bit key codes (or value codes) fill
    # 64 KiB, so the scales sit at byte 65536 of the blob
    (dict(bits=8), dict(bits=4), 256, 32, 4, 256),
    (dict(bits=4), dict(bits=8, scheme="symmetric"), 256, 64, 4, 256),
    (dict(bits=8), dict(bits=8), 256, 32, 3, 256),
]


# The contract is max-abs error <= 1e-3 against the reference; the kernel
# tests hold a tighter canary bound.  The outputs here reach |o| ~ 36 (the x16
# outlier channels), so 3e-4 is ~1e-5 relative: fp32 accumulation-order noise
# (the oracle's own fp32 result is 7.7e-5 from float64 on the same pages).
KERNEL_TOL = 3e-4


@pytest.mark.parametrize("path", ["mfma", "mfma16", "generic"])
@pytest.mark.parametrize("kfmt,vfmt,hd,vgs,Q,tpp", FAST_CASES)
def test_fused_kernels_match_oracle(kfmt, vfmt, hd, vgs, Q, tpp, path):
    """The MFMA kernel and the generic kernel on the same pages, with ragged
    groups, partial last pages, outlier channels and split-K.  Path "mfma"
    raises if the MFMA kernel does not take the call, so every case here is
    shown to run on it; "mfma16" is the MFMA kernel with one key / value
    group per MFMA operand (head block 16) where "mfma" may use blocks of 4
    or 8 heads."""
    from dotcache_amd.backends import decode_grouped_multiquery_step_prepared_hip_tensor_output_only as fused
    from dotcache_amd.decode import set_decode_path, set_mfma_head_block

    set_decode_path("mfma" if path == "mfma16" else path)
    set_mfma_head_block(16 if path == "mfma16" else 0)
    rng = np.random.default_rng(hd * 7 + Q + tpp)
    lens = [tpp * 5 + 17, 1, tpp - 3, 3 * tpp]
    G = len(lens)
    qs = (rng.normal(size=(G, Q, hd)) / np.sqrt(hd)).astype(np.float32)
    kpg = [_pages(hard_values(rng, n, hd), tpp, hd, 32, "K", kfmt) for n in lens]
    vpg = [_pages(hard_values(rng, n, hd), tpp, hd, vgs, "V", vfmt) for n in lens]
    want = O.decode_grouped(qs, kpg, vpg)
    kp = [[to_product_page(p) for p in g] for g in kpg]
    vp = [[to_product_page(p) for p in g] for g in vpg]
    for pps in (None, 2):
        got = fused(list(qs), kp, vp, pages_per_split=pps).cpu().numpy()
        err = np.max(np.abs(got - want))
        assert err < KERNEL_TOL, f"path {path} pps {pps}: max-abs error {err}"


def test_fused_decode_peaked_attention_and_small_values():
    """Sharp softmax (a few tokens dominate) and tiny value scales: the fp16
    high/residual split of weight x scale must keep the error below 1e-3."""
    from dotcache_amd.backends import decode_grouped_multiquery_step_prepared_hip_tensor_output_only as fused

    rng = np.random.default_rng(5)
    hd, n, Q = 128, 2000, 7
    k = rng.normal(size=(n, hd)).astype(np.float32)
    v = (rng.normal(size=(n, hd)) * 1e-3).astype(np.float32)
    v[::97] *= 5e4  # a few large rows
    q = rng.normal(size=(1, Q, hd)).astype(np.float32) * 0.6  # logits spread ~ +-20
    kp = _pages(k, 64, hd, 32, "K", dict(mode="M3"))
    vp = _pages(v, 64, hd, 32, "V", dict(bits=4, scheme="symmetric"))
    want = O.decode_grouped(q, [kp], [vp])
    got = fused(list(q), [[to_product_page(p) for p in kp]], [[to_product_page(p) for p in vp]]).cpu().numpy()
    assert np.max(np.abs(got - want)) < 1e-3


# Merge layouts: (counts, begins or None for in order, unused slots): ragged
# counts with spare slots, counts that need several passes of a block's
# rows, equal counts, counts whose total divides evenly among the merges
# without being equal, and merges whose partial ranges are not in merge
# order.
MERGE_LAYOUTS = {
    "ragged": ([5, 1, 40, 3], None, 2),
    "long": ([70, 1, 150, 3], None, 1),  # passes of 2 and 4 slots per row, several of 4
    "uniform": ([6, 6, 6, 6], None, 0),
    "divisible": ([5, 1, 10, 8], None, 0),
    "permuted": ([6, 6, 6, 6], [6, 0, 18, 12], 0),
}


@pytest.mark.parametrize("layout", list(MERGE_LAYOUTS))
@pytest.mark.parametrize("hd", [128, 30])
def test_lse_merge_matches_float64(hd, layout):
    """dc_lse_merge on hand-made partials (m, l, o), log2 domain: ragged
    counts, empty partials (m = -inf) and a merge whose partials are all
    empty.  head_dim 30 takes the one-channel-per-thread path."""
    import ctypes as C

    import torch

    from dotcache_amd import _lib
    from dotcache_amd.page_pool import current_stream_ptr

    rng = np.random.default_rng(hd)
    B, H, Q = 2, 2, 3
    counts, begins, spare = MERGE_LAYOUTS[layout]  # (seq, kv_head) in row-major order
    n_part = sum(counts) + spare
    part_o = rng.normal(size=(n_part, Q, hd)).astype(np.float32)
    m = (rng.normal(size=(n_part, Q)) * 8).astype(np.float32)
    l = rng.uniform(0.5, 40.0, size=(n_part, Q)).astype(np.float32)
    m[2, 1] = -np.inf                       # an empty partial
    l[2, 1] = 0.0
    begins = np.cumsum([0] + counts[:-1]) if begins is None else np.array(begins)
    m[begins[3]:begins[3] + 3] = -np.inf    # merge 3: every partial empty
    l[begins[3]:begins[3] + 3] = 0.0
    ml = np.stack([m, l], axis=-1)
    ws = torch.from_numpy(np.concatenate([part_o.ravel(), ml.ravel()]).astype(np.float32)).cuda()
    items = np.array([[i // H, i % H, begins[i], counts[i]] for i in range(len(counts))], np.int32)
    merges = torch.from_numpy(items.ravel().view(np.uint8).copy()).cuda()
    out = torch.full((B, H, Q, hd), 7.0, dtype=torch.float32, device="cuda")
    st = _lib.lib().dc_lse_merge(C.c_void_p(merges.data_ptr()), len(counts), C.c_void_p(ws.data_ptr()),
                                 ws.numel() * 4, B, H, Q, hd, C.c_void_p(out.data_ptr()),
                                 C.c_void_p(current_stream_ptr()))
    _lib.check(st, "dc_lse_merge")
    got = out.cpu().numpy()
    for i, (b, c) in enumerate(zip(begins, counts)):
        s, h = divmod(i, H)
        mm = m[b:b + c].astype(np.float64)
        M = np.max(mm, axis=0)
        w = np.where(np.isneginf(mm), 0.0, np.exp2(mm - np.where(np.isneginf(M), 0.0, M)))
        L = np.sum(w * l[b:b + c], axis=0)
        want = np.einsum("sq,sqd->qd", w, part_o[b:b + c].astype(np.float64)) / np.maximum(L, 1e-30)[:, None]
        np.testing.assert_allclose(got[s, h], want, atol=2e-5, rtol=2e-5)


@pytest.mark.parametrize("path", ["mfma", "generic"])
@pytest.mark.parametrize("kfmt,vfmt,vgs", [
    (dict(mode="M3"), dict(bits=4, scheme="symmetric"), 32),   # config 3 formats (keys through LDS)
    (dict(bits=4), dict(bits=8, scheme="symmetric"), 64),      # config 4 formats
])
def test_items_longer_than_one_metadata_batch(kfmt, vfmt, vgs, path):
    """Items of more than 64 pages: the kernels read page metadata 64 pages
    at a time, so these items walk a second batch.  One sequence also has
    an empty page (0 tokens) in the middle of its list."""
    from dotcache_amd.backends import decode_grouped_multiquery_step_prepared_hip_tensor_output_only as fused
    from dotcache_amd.decode import set_decode_path

    set_decode_path(path)
    rng = np.random.default_rng(130 + vgs)
    hd, Q, tpp = 128, 7, 64
    lens = [130 * tpp - 9, 70 * tpp]
    qs = (rng.normal(size=(len(lens), Q, hd)) / np.sqrt(hd)).astype(np.float32)
    kpg = [_pages(hard_values(rng, n, hd), tpp, hd, 32, "K", kfmt) for n in lens]
    vpg = [_pages(hard_values(rng, n, hd), tpp, hd, vgs, "V", vfmt) for n in lens]
    # an empty page inside sequence 1: the same page with no tokens
    empty_k = O.encode_page(np.zeros((0, hd), np.float32), head_dim=hd, group_size=32, kind="K", **kfmt)
    empty_v = O.encode_page(np.zeros((0, hd), np.float32), head_dim=hd, group_size=vgs, kind="V", **vfmt)
    kpg[1].insert(40, empty_k)
    vpg[1].insert(40, empty_v)
    want = O.decode_grouped(qs, kpg, vpg)
    kp = [[to_product_page(p) for p in g] for g in kpg]
    vp = [[to_product_page(p) for p in g] for g in vpg]
    for pps in (100, 71):  # one item of 100 / 71 pages per sequence, plus a remainder
        got = fused(list(qs), kp, vp, pages_per_split=pps).cpu().numpy()
        err = np.max(np.abs(got - want))
        assert err < KERNEL_TOL, f"path {path} pps {pps}: max-abs error {err}"


@pytest.mark.parametrize("tpp", [128, 64])
def test_fused_long_context_window_pools(tpp):
    """The C5 pool shape on the MFMA kernel: head_dim 256, M0 affine 4-bit
    keys and values with the newest pages exact (M3 fp16 keys and values in
    the same pools), GQA 4, ragged sequences, split-K; run under path "mfma"
    (the instance where two wavefronts share each work item)."""
    from dotcache_amd.backends import decode_grouped_multiquery_step_prepared_hip_tensor_output_only as fused
    from dotcache_amd.decode import set_decode_path

    set_decode_path("mfma")
    rng = np.random.default_rng(256 + tpp)
    hd, Q = 256, 4
    lens = [tpp * 5 + 17, 1, tpp - 3, 3 * tpp, 2 * tpp + 1]
    qs = (rng.normal(size=(len(lens), Q, hd)) / np.sqrt(hd)).astype(np.float32)
    kpg, vpg = [], []
    for n in lens:
        pages_k, pages_v = [], []
        k = rng.standard_t(4, size=(n, hd)).astype(np.float32)
        v = rng.standard_t(4, size=(n, hd)).astype(np.float32)
        n_pages = -(-n // tpp)
        for i, s in enumerate(range(0, n, tpp)):
            fmt = dict(mode="M3") if i >= n_pages - 1 and n_pages > 1 else dict(bits=4)  # the newest page exact
            pages_k.append(O.encode_page(k[s:s + tpp], head_dim=hd, group_size=32, kind="K", token_start=s, **fmt))
            pages_v.append(O.encode_page(v[s:s + tpp], head_dim=hd, group_size=32, kind="V", token_start=s, **fmt))
        kpg.append(pages_k)
        vpg.append(pages_v)
    want = O.decode_grouped(qs, kpg, vpg)
    kp = [[to_product_page(p) for p in g] for g in kpg]
    vp = [[to_product_page(p) for p in g] for g in vpg]
    for pps in (None, 1, 2):
        got = fused(list(qs), kp, vp, pages_per_split=pps).cpu().numpy()
        err = np.max(np.abs(got - want))
        assert err < KERNEL_TOL, f"pps {pps}: max-abs error {err}"
