"""CPU oracle of the page-mode choice (Selective Key Precision policies).

TEST INFRASTRUCTURE ONLY.  Nothing in the product package (``dotcache_amd``)
may import, call or link this module.

It restates, step by step, how the reference decides the mode of a full
page when a kind has mode or policy overrides:

  * page statistics             reference ``dotcache/planner.py:46-70`` (observe_page)
  * tier policies               reference ``dotcache/planner.py:199-272`` (make_tier_candidates)
  * explicit policies           reference ``dotcache/planner.py:275-300`` (make_explicit_policy)
  * candidate admission         reference ``dotcache/planner.py:303-342`` (_candidate_is_allowed)
  * the choice                  reference ``dotcache/planner.py:75-147`` (choose_page_mode)
  * the layer policy            reference ``dotcache/config.py:546-614`` (resolve_layer_policy)
  * the per-page call           reference ``dotcache/model_kv_cache.py:3164-3185`` (_select_page_mode,
                                token_age = sequence_length - token_start - 1) and ``:789-810``

Specs are plain dicts with the keys of the reference's ``PageModeSpec``
(mode, bits, quant_scheme, escape_dtype, policy_id, sensitivity_tier,
fallback_reason, age_bucket).  Pinned in ``tests/test_policy_oracle.py`` by
the reference's known answers (``tests/test_planner.py:12-133``,
``tests/test_model_kv_cache.py:261-296``) and by hand-worked cases.
"""
from __future__ import annotations

import numpy as np


def spec(mode, bits, quant_scheme, escape_dtype=None, policy_id="exact_baseline", sensitivity_tier="exact",
         fallback_reason="", age_bucket="aged"):
    return dict(mode=mode, bits=int(bits), quant_scheme=quant_scheme, escape_dtype=escape_dtype, policy_id=policy_id,
                sensitivity_tier=sensitivity_tier, fallback_reason=fallback_reason, age_bucket=age_bucket)


def parse_token(token):
    """``MODE/SCHEME/BITS[/ESCAPE]`` (reference ``planner.py:178-197``)."""
    parts = [p.strip() for p in token.split("/") if p.strip()]
    return spec(parts[0].upper(), int(parts[2]), parts[1].lower(), parts[3].lower() if len(parts) == 4 else None)


def observe_page(values):
    """Reference ``planner.py:46-70``."""
    x = np.asarray(values, dtype=np.float32)
    if x.shape[0] == 0:
        return dict(token_count=0, rms=0.0, abs_max=0.0, outlier_fraction=0.0, channel_range_mean=0.0)
    a = np.abs(x, dtype=np.float32)
    rms = float(np.sqrt(np.mean(np.square(x, dtype=np.float32), dtype=np.float64)))
    cutoff = max(3.0 * max(rms, 1e-6), 6.0)
    return dict(
        token_count=int(x.shape[0]),
        rms=rms,
        abs_max=float(np.max(a)),
        outlier_fraction=float(np.mean(a >= cutoff, dtype=np.float64)),
        channel_range_mean=float(np.mean(np.max(x, axis=0) - np.min(x, axis=0), dtype=np.float64)),
    )


def make_tier_candidates(kind, tier, default_bits, default_scheme, default_mode, recent_window,
                         recent_escape_dtype="float16", prefer_project=False):
    """Reference ``planner.py:199-272``."""
    def c(mode, scheme, bits):
        return spec(mode, bits, scheme, sensitivity_tier=tier)

    if tier == "exact":
        cands = [c(default_mode, default_scheme, default_bits)]
        th = (0.0, float("inf"), float("inf"))
    elif kind == "K":
        proj = c("M4", "project", 4) if prefer_project else c("M2", "sketch", 4)
        if tier == "strict":
            cands, th = [c("M0", "affine", 4)], (0.02, 4.5, 3.0)
        elif tier == "aggressive":
            cands, th = [c("M0", "affine", 2), proj, c("M0", "affine", 4)], (0.10, 8.0, 5.5)
        else:
            cands, th = [c("M0", "affine", 2), proj, c("M0", "affine", 4)], (0.05, 6.0, 4.0)
    else:
        if tier == "strict":
            cands, th = [c("M1", "lut", 4), c("M0", "affine", 4)], (0.02, 4.5, 3.0)
        elif tier == "aggressive":
            cands = [c("M0", "affine", 2), c("M0", "affine", 3), c("M1", "lut", 4), c("M0", "affine", 4)]
            th = (0.10, 8.0, 5.5)
        else:
            cands, th = [c("M0", "affine", 3), c("M1", "lut", 4), c("M0", "affine", 4)], (0.05, 6.0, 4.0)
    return dict(policy_id=f"{kind.lower()}_{tier}", sensitivity_tier=tier, kind=kind, candidates=cands,
                recent_candidate=spec("M3", default_bits, "affine", recent_escape_dtype, sensitivity_tier=tier),
                recent_window=0 if tier == "exact" else recent_window,
                outlier=th[0], abs_max=th[1], channel_range=th[2])


def make_explicit_policy(kind, policy_id, tier, candidates, recent_window, recent_escape_dtype="float16"):
    """Reference ``planner.py:275-300``."""
    recent = None
    for cand in candidates:
        if cand["mode"] == "M3":
            recent = cand
            break
    if recent is None:
        recent = spec("M3", 4, "affine", recent_escape_dtype, sensitivity_tier=tier)
    return dict(policy_id=policy_id, sensitivity_tier=tier, kind=kind, candidates=list(candidates),
                recent_candidate=recent, recent_window=recent_window, outlier=0.05, abs_max=6.0, channel_range=4.0)


def candidate_is_allowed(cand, kind, stats, pol):
    """Reference ``planner.py:303-342``."""
    if stats is None or (cand["mode"] == "M0" and cand["bits"] >= 4):
        return True
    if cand["mode"] == "M3":
        return True
    if cand["mode"] in ("M2", "M4"):
        if kind != "K":
            return False
        return stats["outlier_fraction"] <= pol["outlier"] and stats["channel_range_mean"] <= pol["channel_range"]
    if cand["mode"] == "M1":
        if kind != "V":
            return False
        return stats["outlier_fraction"] <= pol["outlier"] and stats["channel_range_mean"] <= pol["channel_range"]
    if cand["mode"] == "T3":
        return False
    if cand["mode"] == "M0" and cand["bits"] <= 2:
        return stats["outlier_fraction"] <= pol["outlier"] and stats["abs_max"] <= pol["abs_max"]
    if cand["mode"] == "M0" and cand["bits"] == 3:
        return stats["outlier_fraction"] <= pol["outlier"] * 1.25 and stats["abs_max"] <= pol["abs_max"] * 1.2
    return True


def choose_page_mode(kind, token_age, stats, pol):
    """Reference ``planner.py:75-147``."""
    def out(c, reason, bucket):
        return spec(c["mode"], c["bits"], c["quant_scheme"], c["escape_dtype"], pol["policy_id"],
                    pol["sensitivity_tier"], reason, bucket)

    if token_age < pol["recent_window"]:
        if pol["recent_candidate"] is not None:
            return out(pol["recent_candidate"], "recent_window", "recent")
        last = pol["candidates"][-1] if pol["candidates"] else None
        return out(spec("M3", last["bits"] if last else 4, last["quant_scheme"] if last else "affine"),
                   "recent_window", "recent")
    if not pol["candidates"]:
        return out(spec("M0", 4, "affine"), "no_candidates", "aged")
    failures = []
    for index, cand in enumerate(pol["candidates"]):
        if candidate_is_allowed(cand, kind, stats, pol):
            return out(cand, "" if index == 0 else ("+".join(failures) or "fallback"), "aged")
        failures.append(f"{cand['mode'].lower()}_stats")
    return out(pol["candidates"][-1], "+".join(failures) if failures else "threshold_fallback", "aged")


def _override_mode(overrides, default_mode, layer_id, kv_head_id):
    """Reference ``config.py:390-414``: the last matching entry wins."""
    mode = default_mode
    for entry in overrides:
        target, value = entry.split("=", 1)
        parts = target.strip().split(":")
        if int(parts[1]) != int(layer_id):
            continue
        if len(parts) == 4 and int(parts[3]) != int(kv_head_id):
            continue
        mode = value.strip()
    return mode


def resolve_layer_policy(cfg, kind, layer_id, kv_head_id):
    """Reference ``config.py:546-614``.  ``cfg`` is any object with the
    reference's config field names."""
    k = kind == "K"
    default_mode = cfg.default_mode_k if k else cfg.default_mode_v
    default_bits = cfg.bits_k if k else cfg.bits_v
    default_scheme = cfg.quant_scheme_k if k else cfg.quant_scheme_v
    tier = cfg.key_policy_tier if k else cfg.value_policy_tier
    layer_tiers = cfg.key_layer_sensitivity if k else cfg.value_layer_sensitivity
    explicit = cfg.key_policy_overrides if k else cfg.value_policy_overrides
    overrides = cfg.key_mode_overrides if k else cfg.value_mode_overrides
    mode = _override_mode(overrides, default_mode, layer_id, kv_head_id)
    if mode != default_mode:
        scheme = {"M1": "lut", "M2": "sketch", "M4": "project", "T3": "turbo3"}.get(mode, default_scheme)
        return make_explicit_policy(kind, f"{kind.lower()}_mode_override_layer_{int(layer_id)}", "exact",
                                    [spec(mode, default_bits, scheme)], 0, cfg.recent_page_escape_dtype)
    for entry in explicit:
        target, raw = entry.split("=", 1)
        if int(target.split(":")[1]) == int(layer_id):
            cands = [parse_token(t) for t in raw.split(",") if t.strip()]
            return make_explicit_policy(kind, f"{kind.lower()}_policy_override_layer_{int(layer_id)}", "balanced",
                                        cands, cfg.recent_window, cfg.recent_page_escape_dtype)
    for entry in layer_tiers:
        target, value = entry.split("=", 1)
        if int(target.split(":")[1]) == int(layer_id):
            tier = value.strip()
    return make_tier_candidates(kind, tier, default_bits, default_scheme, default_mode, cfg.recent_window,
                                cfg.recent_page_escape_dtype, bool(getattr(cfg, "prefer_m4_project_k", False)) and k)


def has_overrides(cfg, kind):
    """Reference ``config.py:369-388`` for one kind."""
    k = kind == "K"
    modes = cfg.key_mode_overrides if k else cfg.value_mode_overrides
    tiers = cfg.key_layer_sensitivity if k else cfg.value_layer_sensitivity
    explicit = cfg.key_policy_overrides if k else cfg.value_policy_overrides
    tier = cfg.key_policy_tier if k else cfg.value_policy_tier
    return bool(modes) or bool(tiers) or bool(explicit) or tier != "exact"


def select_page_mode(cfg, values, kind, layer_id, kv_head_id, token_start, sequence_length):
    """Reference ``model_kv_cache.py:3164-3185``: None without overrides."""
    if not has_overrides(cfg, kind):
        return None
    pol = resolve_layer_policy(cfg, kind, layer_id, kv_head_id)
    age = max(0, int(sequence_length) - int(token_start) - 1)
    return choose_page_mode(kind, age, observe_page(values), pol)


def encode_spec(cfg, kind, chosen):
    """(mode, bits, scheme, escape_dtype, header policy fields) that the
    reference's ``encode_page`` uses for a page encoded with ``page_mode =
    chosen`` (or with the config's default mode when ``chosen`` is None):
    reference ``encode.py:144-155``, ``:180-190``."""
    k = kind == "K"
    if chosen is None:
        return dict(mode=cfg.default_mode_k if k else cfg.default_mode_v, bits=cfg.bits_k if k else cfg.bits_v,
                    scheme=cfg.quant_scheme_k if k else cfg.quant_scheme_v, escape_dtype=cfg.escape_dtype,
                    policy_id="exact_baseline", sensitivity_tier="exact", fallback_reason="", age_bucket="aged")
    return dict(mode=chosen["mode"], bits=chosen["bits"], scheme=chosen["quant_scheme"],
                escape_dtype=chosen["escape_dtype"] or cfg.escape_dtype, policy_id=chosen["policy_id"],
                sensitivity_tier=chosen["sensitivity_tier"], fallback_reason=chosen["fallback_reason"],
                age_bucket=chosen["age_bucket"])
