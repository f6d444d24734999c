"""The device KV cache lifecycle (prefill ingest, per-token append into the
tail, page finalise, decode) against the oracle: decode outputs within the
kernel tolerance, finalised pages bit-identical to the oracle's encode of
the same fp32 rows, with the mode and header the reference's cache chooses
(reference ``model_kv_cache.py:3609-4134``; page modes by
``choose_page_mode`` under overrides, ``:3164-3185`` and ``:789-810``)."""
import numpy as np
import pytest

from oracle import dotcache_oracle as O
from oracle import policy_oracle as PO
from tests.helpers import hard_values, pool_page_to_oracle

pytestmark = pytest.mark.gpu

KERNEL_TOL = 3e-4  # as in test_gpu_attention.py; the contract is 1e-3


def _oracle_stream_pages(rows, cfg, kind, layer, head, page_context=None):
    """The reference's pages of one stream of ``rows [T, hd]`` cached from
    token 0: full page i in the mode the reference's cache gives it when it
    is encoded in a context of ``page_context[i]`` tokens (the policy oracle
    restating ``choose_page_mode``; the configured mode without overrides),
    the partial tail as an M3 page."""
    P = cfg.tokens_per_page
    T = rows.shape[0]
    full = (T // P) * P
    pages = []
    for i, s in enumerate(range(0, full, P)):
        ctx = T if page_context is None else page_context[i]
        chosen = PO.select_page_mode(cfg, rows[s:s + P], kind, layer, head, token_start=s, sequence_length=ctx)
        if chosen is None:
            mode = cfg.resolve_page_mode(kind=kind, layer_id=layer, kv_head_id=head)
            sp = PO.encode_spec(cfg, kind, None)
            sp["mode"] = mode
        else:
            sp = PO.encode_spec(cfg, kind, chosen)
        pages.append(O.encode_page(rows[s:s + P], head_dim=cfg.head_dim, group_size=cfg.group_size, kind=kind,
                                   bits=sp["bits"], mode=sp["mode"], scheme=sp["scheme"],
                                   escape_dtype=sp["escape_dtype"], layer_id=layer, kv_head_id=head, token_start=s,
                                   policy_id=sp["policy_id"], sensitivity_tier=sp["sensitivity_tier"],
                                   fallback_reason=sp["fallback_reason"], age_bucket=sp["age_bucket"]))
    if T > full:
        pages.append(O.encode_page(rows[full:], head_dim=cfg.head_dim, group_size=cfg.group_size, kind=kind, mode="M3",
                                   token_start=full))
    return pages


def _check_decode(cache, keys, values, T, cfg, rng, q_map=None, page_context=None):
    import torch

    L, B, H = keys.shape[:3]
    Hq = cache.num_attention_heads
    qmap = np.arange(Hq) // (Hq // H) if q_map is None else np.asarray(q_map)
    for layer in range(L):
        q = (rng.normal(size=(B, Hq, cfg.head_dim)) / np.sqrt(cfg.head_dim)).astype(np.float32)
        got = cache.decode_layer(layer, torch.from_numpy(q), q_map).cpu().numpy()
        for b in range(B):
            for h in range(H):
                kp = _oracle_stream_pages(keys[layer, b, h, :T], cfg, "K", layer, h, page_context)
                vp = _oracle_stream_pages(values[layer, b, h, :T], cfg, "V", layer, h, page_context)
                heads = np.flatnonzero(qmap == h)
                want = O.decode_grouped(q[b, heads][None], [kp], [vp])[0]
                err = np.max(np.abs(got[b, heads] - want))
                assert err < KERNEL_TOL, f"layer {layer} seq {b} head {h} after {T} tokens: max-abs error {err}"


CASES = {
    # a mode override on one stream: the reference's choose_page_mode path
    # for every K page (one-mode override policy there, the exact tier
    # elsewhere), header policy fields included
    "mode_override": dict(quant_scheme_v="symmetric", key_mode_overrides=("layer:1:kv:1=M3",)),
    # a strict key tier: keys younger than the 128-token recent window become
    # M3 fp16 (prefill page 1 and every appended page at 64-token pages, every
    # page at 16); balanced values fall back to 4-bit on these outlier rows
    # (m0_stats+m1_stats), with page statistics computed on the device
    "recent_window": dict(key_policy_tier="strict", value_policy_tier="balanced"),
}


def _finalise_contexts(P, T0, steps, T1):
    """Context length at which each full page of the run is encoded: the
    prefill length for prefill pages, ``t + n`` of the append step that
    completes the page (reference model_kv_cache.py:3887-3892)."""
    ctx = [T0] * (T0 // P)
    for t, n in steps:
        for k in range(len(ctx), T1 // P):
            if t <= k * P + P - 1 < t + n:
                ctx.append(t + n)
    return ctx


@pytest.mark.parametrize("case", sorted(CASES))
@pytest.mark.parametrize("page_tokens", [64, 16])
def test_prefill_append_decode_matches_oracle(page_tokens, case):
    """Prefill of two full pages and a partial tail, then appends one token
    at a time and three at once, across two page finalisations; decode at
    each stage.  page_tokens 64 runs the MFMA kernel, 16 the generic one."""
    import torch

    from dotcache_amd.config import DotCacheConfig
    from dotcache_amd.kv_cache import DevicePagedKVCache

    P = page_tokens
    cfg = DotCacheConfig(head_dim=64, group_size=32, tokens_per_page=P, **CASES[case])
    L, B, H, Hq = 2, 2, 2, 4
    rng = np.random.default_rng(P)
    T0, T1 = 2 * P + 5, 4 * P + 2
    keys = np.stack([hard_values(rng, T1, 64) for _ in range(L * B * H)]).reshape(L, B, H, T1, 64)
    values = np.stack([hard_values(rng, T1, 64) for _ in range(L * B * H)]).reshape(L, B, H, T1, 64)
    cache = DevicePagedKVCache(cfg, num_hidden_layers=L, num_attention_heads=Hq, num_key_value_heads=H, batch_size=B)
    for layer in range(L):
        cache.ingest_prefill_cache(layer, torch.from_numpy(keys[layer, :, :, :T0]), values[layer, :, :, :T0])
    steps = []
    t = T0
    while t < T1:
        n = 3 if t == T0 + 4 else 1
        steps.append((t, n))
        t += n
    ctx = _finalise_contexts(P, T0, steps, T1)
    _check_decode(cache, keys, values, T0, cfg, rng, page_context=ctx)
    # the fp16 tail (5 tokens) was attended by the split-K merge, and the
    # decode launch read only the other pages (with 16-token pages under the
    # recent window every page is exact: one launch reads them all)
    from dotcache_amd.decode import merge_windows

    k_table, _, seq_pages, _ = cache._layer_tables(0)
    front = merge_windows(cache.k_pool, cache.v_pool, *cache._host_tables[0], seq_pages)
    if case == "mode_override" or P == 64:
        assert front is not None and np.all(front[:, 1] == seq_pages) and np.all(front[:, 0] >= 1)
    else:
        assert front is None
    for t, n in steps:
        for layer in range(L):
            cache.append_step(layer, keys[layer, :, :, t:t + n], torch.from_numpy(values[layer, :, :, t:t + n]), t)
        if t + n in (3 * P - 1, 3 * P, 3 * P + 1, T1):
            _check_decode(cache, keys, values, t + n, cfg, rng, page_context=ctx)
    assert cache.sequence_length(0) == T1
    # finalised pages: the reference's mode and header, and bytes identical
    # to the oracle's encode of the same fp32 rows
    modes = set()
    for layer in range(L):
        for b in range(B):
            for h in range(H):
                for kind, src in (("K", keys), ("V", values)):
                    want = _oracle_stream_pages(src[layer, b, h, :T1], cfg, kind, layer, h, ctx)
                    ids = cache.page_ids(layer, b, h, kind)
                    assert len(ids) == T1 // P
                    pool = cache.k_pool if kind == "K" else cache.v_pool
                    for i, (pid, wp) in enumerate(zip(ids, want)):
                        got = cache.page(layer, b, h, i, kind)
                        assert got.header.to_dict() == wp.header.to_dict(), f"{kind} page {i} of ({layer}, {b}, {h})"
                        modes.add((kind, wp.header.mode_default, wp.header.fallback_reason))
                        gp = pool_page_to_oracle(pool, pid, kind)
                        for f in ("payload", "scales", "bias", "escape_payload"):
                            a, e = getattr(gp, f), getattr(wp, f)
                            assert (a is None) == (e is None), f
                            if a is not None:
                                np.testing.assert_array_equal(a, e, err_msg=f"{kind} page {pid} {f}")
    if case == "recent_window":
        # the young key pages flipped to M3 by the recent window
        assert ("K", "M3", "recent_window") in modes
        if P == 64:  # page 0 of the prefill is older than the window
            assert ("K", "M0", "") in modes and ("V", "M0", "m0_stats+m1_stats") in modes
    else:
        assert ("K", "M3", "") in modes and ("K", "M0", "") in modes


def test_decode_with_a_permuted_head_map():
    import torch

    from dotcache_amd.config import DotCacheConfig
    from dotcache_amd.kv_cache import DevicePagedKVCache

    cfg = DotCacheConfig(head_dim=128, group_size=32, tokens_per_page=64)
    L, B, H, Hq, T = 1, 1, 2, 6, 150
    rng = np.random.default_rng(3)
    keys = hard_values(rng, H * T, 128).reshape(L, B, H, T, 128)
    values = hard_values(rng, H * T, 128).reshape(L, B, H, T, 128)
    cache = DevicePagedKVCache(cfg, num_hidden_layers=L, num_attention_heads=Hq, num_key_value_heads=H, batch_size=B)
    cache.ingest_prefill_cache(0, torch.from_numpy(keys[0, 0]), torch.from_numpy(values[0, 0]))
    _check_decode(cache, keys, values, T, cfg, rng, q_map=[1, 0, 0, 1, 1, 0])
    with pytest.raises(ValueError):
        cache.decode_layer(0, torch.zeros(1, Hq, 128), [0, 0, 0, 0, 1, 1])
