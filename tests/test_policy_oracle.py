"""The page-mode choice: the policy oracle pinned by the reference's known
answers, and the product's host policy code checked against the oracle.

Known answers restated from reference ``tests/test_planner.py:12-133`` and
``tests/test_model_kv_cache.py:261-296``; the rest are worked by hand from
``planner.py:75-147`` / ``:199-342`` and ``config.py:546-614``."""
from types import SimpleNamespace

import numpy as np
import pytest

from oracle import policy_oracle as P


def _cfg(**kw):
    base = dict(head_dim=32, group_size=32, bits_k=4, bits_v=4, default_mode_k="M0", default_mode_v="M0",
                quant_scheme_k="affine", quant_scheme_v="affine", recent_window=128, escape_dtype="float16",
                recent_page_escape_dtype="float16", key_mode_overrides=(), value_mode_overrides=(),
                key_policy_tier="exact", value_policy_tier="exact", key_layer_sensitivity=(),
                value_layer_sensitivity=(), key_policy_overrides=(), value_policy_overrides=(),
                prefer_m4_project_k=False)
    base.update(kw)
    return SimpleNamespace(**base)


# ---- the oracle against the reference's known answers ----------------------

def test_observe_page_known_answer():
    st = P.observe_page(np.asarray([[0.0, 1.0], [2.0, -3.0]], np.float32))
    assert st["token_count"] == 2 and st["abs_max"] == 3.0
    # by hand: squares 0, 1, 4, 9 -> mean 3.5; channel ranges 2 and 4 -> 3
    assert st["rms"] == pytest.approx(np.sqrt(3.5), rel=1e-12)
    assert st["channel_range_mean"] == 3.0
    assert st["outlier_fraction"] == 0.0  # cutoff max(3 rms, 6) = 6
    x = np.zeros((4, 4), np.float32)
    x[0, 0] = 7.0  # rms = 7/4, cutoff 6: one entry of 16
    assert P.observe_page(x)["outlier_fraction"] == 1 / 16


def test_recent_pages_escape():
    pol = P.make_tier_candidates("K", "balanced", 4, "affine", "M0", 128, "float16")
    m = P.choose_page_mode("K", 12, P.observe_page(np.ones((4, 8), np.float32)), pol)
    assert (m["mode"], m["fallback_reason"], m["age_bucket"]) == ("M3", "recent_window", "recent")
    pol = P.make_tier_candidates("V", "balanced", 4, "affine", "M0", 128, "int8")
    m = P.choose_page_mode("V", 12, P.observe_page(np.ones((4, 8), np.float32)), pol)
    assert (m["mode"], m["escape_dtype"]) == ("M3", "int8")
    # the recent window is strict: age 127 is recent, 128 is aged
    assert P.choose_page_mode("K", 127, None, P.make_tier_candidates("K", "strict", 4, "affine", "M0", 128))["mode"] == "M3"
    assert P.choose_page_mode("K", 128, None, P.make_tier_candidates("K", "strict", 4, "affine", "M0", 128))["mode"] == "M0"


def test_balanced_and_aggressive_candidates():
    pol = P.make_tier_candidates("K", "balanced", 4, "affine", "M0", 0)
    m = P.choose_page_mode("K", 256, P.observe_page(np.full((8, 32), 0.05, np.float32)), pol)
    assert (m["mode"], m["bits"], m["sensitivity_tier"]) == ("M0", 2, "balanced")
    pol = P.make_tier_candidates("V", "balanced", 4, "affine", "M0", 0)
    m = P.choose_page_mode("V", 256, P.observe_page(np.full((8, 32), 0.3, np.float32)), pol)
    assert (m["mode"], m["bits"], m["quant_scheme"]) == ("M0", 3, "affine")
    pol = P.make_tier_candidates("V", "aggressive", 4, "affine", "M0", 0)
    vals = np.linspace(-8.5, 8.5, num=8 * 32, dtype=np.float32).reshape(8, 32)
    m = P.choose_page_mode("V", 256, P.observe_page(vals), pol)
    assert (m["mode"], m["bits"]) == ("M0", 3) and "m0_stats" in m["fallback_reason"]
    pol = P.make_tier_candidates("K", "strict", 4, "affine", "M0", 0)
    m = P.choose_page_mode("K", 256, P.observe_page(np.ones((8, 32), np.float32)), pol)
    assert (m["mode"], m["bits"]) == ("M0", 4)


def test_deterministic_fallback():
    pol = dict(policy_id="test", sensitivity_tier="balanced", kind="V", recent_window=0, recent_candidate=None,
               outlier=0.0, abs_max=1.0, channel_range=0.1,
               candidates=[P.spec("M0", 2, "affine"), P.spec("M1", 4, "lut"), P.spec("M0", 4, "affine")])
    vals = np.linspace(-10.0, 10.0, num=8 * 32, dtype=np.float32).reshape(8, 32)
    m = P.choose_page_mode("V", 256, P.observe_page(vals), pol)
    assert (m["mode"], m["bits"]) == ("M0", 4)
    assert m["fallback_reason"] == "m0_stats+m1_stats"  # by hand: both cheaper candidates fail


def test_layer_policies_known_answers():
    cfg = _cfg(key_policy_tier="balanced", value_policy_tier="strict", key_layer_sensitivity=("layer:1=aggressive",),
               value_policy_overrides=("layer:0=M3/affine/4/int8,M1/lut/4,M0/affine/4",),
               recent_page_escape_dtype="int8")
    assert P.resolve_layer_policy(cfg, "K", 0, 0)["sensitivity_tier"] == "balanced"
    assert P.resolve_layer_policy(cfg, "K", 1, 0)["sensitivity_tier"] == "aggressive"
    v0 = P.resolve_layer_policy(cfg, "V", 0, 0)
    assert len(v0["candidates"]) == 3 and v0["candidates"][0]["mode"] == "M3"
    assert v0["candidates"][0]["escape_dtype"] == "int8" and v0["recent_candidate"]["escape_dtype"] == "int8"
    cfg = _cfg(key_policy_tier="strict", value_policy_tier="balanced")
    assert [f"{c['mode']}:{c['bits']}" for c in P.resolve_layer_policy(cfg, "V", 0, 0)["candidates"]] == [
        "M0:3", "M1:4", "M0:4"]


def test_mode_override_policy_by_hand():
    """A mode override gives a one-mode explicit policy with no recent
    window; streams without one keep the exact tier, which has none either
    (reference planner.py:268, config.py:567-582)."""
    cfg = _cfg(key_mode_overrides=("layer:1:kv:1=M3",))
    over = P.select_page_mode(cfg, np.ones((4, 32), np.float32), "K", 1, 1, token_start=0, sequence_length=4)
    assert over == P.spec("M3", 4, "affine", None, "k_mode_override_layer_1", "exact", "", "aged")
    plain = P.select_page_mode(cfg, np.ones((4, 32), np.float32), "K", 1, 0, token_start=0, sequence_length=4)
    assert plain == P.spec("M0", 4, "affine", None, "k_exact", "exact", "", "aged")
    assert P.select_page_mode(cfg, np.ones((4, 32), np.float32), "V", 1, 0, 0, 4) is None  # no value overrides


# ---- the product's policy code against the oracle ---------------------------

def _product_cfg(**kw):
    from dotcache_amd.config import DotCacheConfig

    return DotCacheConfig(head_dim=32, group_size=32, **kw)


def _as_dict(s):
    return dict(mode=s.mode, bits=s.bits, quant_scheme=s.quant_scheme, escape_dtype=s.escape_dtype,
                policy_id=s.policy_id, sensitivity_tier=s.sensitivity_tier, fallback_reason=s.fallback_reason,
                age_bucket=s.age_bucket)


CONFIGS = [
    dict(),
    dict(key_mode_overrides=("layer:0=M3", "layer:1:kv:1=M3")),
    dict(key_policy_tier="strict", value_policy_tier="balanced"),
    dict(key_policy_tier="balanced", value_policy_tier="aggressive", recent_page_escape_dtype="int8"),
    dict(key_layer_sensitivity=("layer:1=aggressive",), value_policy_overrides=("layer:0=M1/lut/4,M0/affine/4",)),
    dict(key_policy_overrides=("layer:1=M0/affine/2,M3/affine/4/float32",), bits_k=2, recent_window=64),
    dict(value_mode_overrides=("layer:1=M3",), quant_scheme_v="symmetric", prefer_m4_project_k=True,
         key_policy_tier="aggressive"),
]


@pytest.mark.parametrize("ci", range(len(CONFIGS)))
def test_product_policy_matches_oracle(ci):
    from dotcache_amd.config import observe_page

    kw = CONFIGS[ci]
    cfg = _product_cfg(**kw)
    ocfg = _cfg(**kw)
    rng = np.random.default_rng(ci)
    pages = [rng.normal(size=(16, 32)).astype(np.float32) * s for s in (0.05, 0.3, 1.0, 3.0)]
    pages.append(np.linspace(-8.5, 8.5, num=16 * 32, dtype=np.float32).reshape(16, 32))
    for kind in ("K", "V"):
        for layer in (0, 1):
            for head in (0, 1):
                for x in pages:
                    ps, po = observe_page(x), P.observe_page(x)
                    assert (ps.rms, ps.abs_max, ps.outlier_fraction, ps.channel_range_mean) == (
                        po["rms"], po["abs_max"], po["outlier_fraction"], po["channel_range_mean"])
                    for start, seq_len in ((0, 16), (0, 400), (256, 400), (300, 400)):
                        want = P.select_page_mode(ocfg, x, kind, layer, head, start, seq_len)
                        got = cfg.select_page_mode(kind=kind, layer_id=layer, kv_head_id=head, token_start=start,
                                                   sequence_length=seq_len, stats=lambda: observe_page(x))
                        assert (None if got is None else _as_dict(got)) == want, (kind, layer, head, start)
