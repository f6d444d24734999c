"""The block-table cache (vLLM block ids -> device pages) against the oracle:
the reference's adapter tests (``tests/test_vllm_adapter.py:89-218``) on the
device cache, plus batched decode through block tables with ragged
context lengths and scattered block ids."""
import numpy as np
import pytest

from oracle import dotcache_oracle as O
from tests.helpers import hard_values

pytestmark = pytest.mark.gpu


def _block_pages(blocks, cfg, kind, head, live=0):
    """Oracle pages of one head's ``[n, bs, hd]`` blocks, the last one live
    with ``live`` tokens when 0 < live < bs (reference test helper
    ``_encode_blocks_for_head``)."""
    P = cfg.tokens_per_page
    n = blocks.shape[0]
    fin = n if live in (0, P) else n - 1
    bits = cfg.bits_k if kind == "K" else cfg.bits_v
    pages = [O.encode_page(blocks[i], head_dim=cfg.head_dim, group_size=cfg.group_size, kind=kind, bits=bits,
                           mode=cfg.resolve_page_mode(kind=kind, layer_id=0, kv_head_id=head), token_start=i * P,
                           kv_head_id=head) for i in range(fin)]
    if fin < n:
        pages.append(O.encode_page(blocks[fin, :live], head_dim=cfg.head_dim, group_size=cfg.group_size, kind=kind,
                                   mode="M3", token_start=fin * P, kv_head_id=head))
    return pages


def _cache(cfg, Hq=4, H=2, L=1):
    from dotcache_amd.block_cache import DeviceVllmPagedKVCache

    return DeviceVllmPagedKVCache(config=cfg, num_hidden_layers=L, num_attention_heads=Hq, num_key_value_heads=H,
                                  block_size=cfg.tokens_per_page)


def _cfg(**kw):
    from dotcache_amd.config import DotCacheConfig

    return DotCacheConfig(**{**dict(head_dim=32, group_size=32, bits_k=4, bits_v=4, tokens_per_page=4), **kw})


def test_block_table_mapping_tracks_stable_block_ownership():
    cfg = _cfg()
    rng = np.random.default_rng(1201)
    cache = _cache(cfg)
    kb = rng.normal(size=(2, 2, 4, 32)).astype(np.float32)
    vb = rng.normal(size=(2, 2, 4, 32)).astype(np.float32)
    cache.sync_layer_blocks(0, kb, vb, block_ids=[11, 42])
    ke, ve = cache.block_entry(0, 1, 42, "K"), cache.block_entry(0, 1, 42, "V")
    assert ke.finalized and ve.finalized
    assert ke.token_start == 4 and ke.token_count == 4
    assert ke.page.header.layer_id == 0 and ke.page.header.kv_head_id == 1
    assert ke.page.header.kind == "K" and ve.page.header.kind == "V"
    want = _block_pages(kb[1], cfg, "K", 1)[1]
    np.testing.assert_array_equal(ke.page.payload, want.payload)
    np.testing.assert_array_equal(ke.page.scales, want.scales)
    np.testing.assert_array_equal(ke.page.bias, want.bias)
    assert [e.key.block_id for e in cache.block_entries_for_layer(0, kind="K")] == [11, 42, 11, 42]


@pytest.mark.parametrize("live", [0, 2])
def test_synced_blocks_decode_matches_oracle(live):
    """Finalised blocks, and a live partial block that stays an exact M3 page."""
    cfg = _cfg()
    rng = np.random.default_rng(1202 + live)
    cache = _cache(cfg)
    kb = rng.normal(size=(2, 2, 4, 32)).astype(np.float32)
    vb = rng.normal(size=(2, 2, 4, 32)).astype(np.float32)
    q = rng.normal(size=(4, 32)).astype(np.float32)
    cache.sync_layer_blocks(0, kb, vb, block_ids=[5, 9], live_block_token_count=live)
    if live:
        e = cache.block_entry(0, 0, 9, "K")
        assert not e.finalized and e.token_count == live and e.page.header.mode_default == "M3"
    got = cache.decode_layer(0, q, [0, 0, 1, 1])
    for h in range(2):
        want = O.decode_grouped(q[2 * h: 2 * h + 2][None], [_block_pages(kb[h], cfg, "K", h, live)],
                                [_block_pages(vb[h], cfg, "V", h, live)])[0]
        np.testing.assert_allclose(got[2 * h: 2 * h + 2], want, atol=2e-5, rtol=0)


def test_append_tokens_fills_and_finalises_blocks():
    """Ten tokens appended in block-sized chunks: blocks 0 and 1 finalised,
    block 2 live with two tokens; decode after each stage."""
    import torch

    cfg = _cfg()
    rng = np.random.default_rng(1204)
    cache = _cache(cfg)
    k = rng.normal(size=(10, 2, 32)).astype(np.float32)
    v = rng.normal(size=(10, 2, 32)).astype(np.float32)
    cache.append_tokens_torch(0, torch.from_numpy(k[:6]), torch.from_numpy(v[:6]), torch.arange(6))
    cache.append_step(0, k[6:10].transpose(1, 0, 2), v[6:10].transpose(1, 0, 2), 6)
    assert [cache.block_entry(0, 0, b, "K").finalized for b in range(3)] == [True, True, False]
    assert cache.block_entry(0, 1, 2, "V").token_count == 2
    with pytest.raises(ValueError):
        cache.append_step(0, k[:1].transpose(1, 0, 2), v[:1].transpose(1, 0, 2), 3)  # not the cached length
    q = rng.normal(size=(4, 32)).astype(np.float32)
    got = cache.decode_layer(0, q)
    for h in range(2):
        blocks_k = np.concatenate([k[:, h], np.zeros((2, 32), np.float32)]).reshape(3, 4, 32)
        blocks_v = np.concatenate([v[:, h], np.zeros((2, 32), np.float32)]).reshape(3, 4, 32)
        want = O.decode_grouped(q[2 * h: 2 * h + 2][None], [_block_pages(blocks_k, cfg, "K", h, 2)],
                                [_block_pages(blocks_v, cfg, "V", h, 2)])[0]
        np.testing.assert_allclose(got[2 * h: 2 * h + 2], want, atol=2e-5, rtol=0)


def test_decode_block_tables_batches_ragged_sequences():
    """Three sequences of 64-token blocks (the MFMA kernel) written through
    slot mappings into scattered block ids, decoded in one launch."""
    import torch

    cfg = _cfg(head_dim=128, tokens_per_page=64, key_mode_overrides=("layer:0:kv:1=M3",))
    H, Hq, P = 2, 14, 64
    cache = _cache(cfg, Hq=Hq, H=H)
    rng = np.random.default_rng(9)
    lens = [150, 64, 7]
    tables = [[17, 3, 40], [8], [25]]
    rows = []
    for b, (n, blocks) in enumerate(zip(lens, tables)):
        k = hard_values(rng, n * H, 128).reshape(n, H, 128)
        v = hard_values(rng, n * H, 128).reshape(n, H, 128)
        slots = np.array([blocks[t // P] * P + t % P for t in range(n)])
        half = n // 2  # two writes per sequence: a run may end mid-block
        cache.write_slots(0, k[:half], v[:half], slots[:half])
        cache.write_slots(0, torch.from_numpy(k[half:]), torch.from_numpy(v[half:]), torch.from_numpy(slots[half:]))
        rows.append((k, v))
    bt = np.full((3, 4), -1, dtype=np.int32)
    for b, blocks in enumerate(tables):
        bt[b, : len(blocks)] = blocks
    q = (rng.normal(size=(3, Hq, 128)) / np.sqrt(128)).astype(np.float32)
    got = cache.decode_block_tables(0, torch.from_numpy(q), torch.from_numpy(bt), lens).cpu().numpy()
    G = Hq // H
    for b, (k, v) in enumerate(rows):
        for h in range(H):
            kp = O.encode_pages(k[:, h], tokens_per_page=P, head_dim=128, group_size=32, kind="K",
                                mode=cfg.resolve_page_mode(kind="K", layer_id=0, kv_head_id=h))
            vp = O.encode_pages(v[:, h], tokens_per_page=P, head_dim=128, group_size=32, kind="V")
            n = k.shape[0]
            if n % P:  # the live block is an exact page
                kp[-1] = O.encode_page(k[(n // P) * P:, h], head_dim=128, group_size=32, kind="K", mode="M3")
                vp[-1] = O.encode_page(v[(n // P) * P:, h], head_dim=128, group_size=32, kind="V", mode="M3")
            want = O.decode_grouped(q[b, h * G:(h + 1) * G][None], [kp], [vp])[0]
            err = np.max(np.abs(got[b, h * G:(h + 1) * G] - want))
            assert err < 3e-4, f"sequence {b} head {h}: max-abs error {err}"
    # sequences 0 and 1 alone: sequence 0's live block is attended by the
    # split-K merge (a window), and the result is the same
    from dotcache_amd.decode import merge_windows

    kt = cache._map["K"][0][bt[:2].clip(0)].transpose(0, 2, 1)
    vt = cache._map["V"][0][bt[:2].clip(0)].transpose(0, 2, 1)
    front = merge_windows(cache.k_pool, cache.v_pool, kt, vt, np.array([3, 1]))
    assert front is not None and front.tolist() == [[2, 3], [1, 1]]
    got2 = cache.decode_block_tables(0, torch.from_numpy(q[:2]), torch.from_numpy(bt[:2]), lens[:2]).cpu().numpy()
    assert np.max(np.abs(got2 - got[:2])) < 2e-5
    with pytest.raises(ValueError):
        cache.decode_block_tables(0, torch.from_numpy(q), torch.from_numpy(bt), [150, 64, 8])  # block 25 holds 7
