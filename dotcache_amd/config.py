"""Page-format configuration: the slice of reference ``DotCacheConfig`` that
decides how pages are encoded, plus per-page mode specs.

Mirrors reference ``dotcache/config.py:96-414`` for the fields that shape a
page (head_dim, group_size, bits, tokens_per_page, layouts, default modes,
schemes, escape dtypes, recent window) and the Selective Key Precision
sensitivity map (``key_mode_overrides`` / ``value_mode_overrides``,
``layer:<id>[:kv:<id>]=<MODE>``, reference ``config.py:15-28``, ``:390-414``),
``PageModeSpec`` / ``parse_page_mode_token`` (reference
``dotcache/planner.py:22-32``, ``:178-197``), and the per-page mode choice
that applies whenever a stream has mode or policy overrides: the layer
policies (sensitivity tiers, explicit candidate lists, mode overrides;
reference ``config.py:546-614``, ``planner.py:199-290``), page statistics
(``planner.py:46-70``) and ``choose_page_mode`` with its recent window
(``planner.py:75-147``, ``:292-342``).  The reference's ``execution_*``
shortlist knobs and M1/M2/M4/T3 codec knobs are not part of this backend; a
policy that picks one of those modes for a page is rejected where the page
is encoded.
"""
from __future__ import annotations

from dataclasses import dataclass
from math import ceil

import numpy as np

_KEY_MODES = ("M0", "M1", "M2", "M3", "M4", "T3")
_VALUE_MODES = ("M0", "M1", "M3", "T3")


@dataclass(frozen=True, slots=True)
class PageModeSpec:
    """Reference ``planner.py:22-32``."""

    mode: str
    bits: int
    quant_scheme: str
    escape_dtype: str | None = None
    policy_id: str = "exact_baseline"
    sensitivity_tier: str = "exact"
    fallback_reason: str = ""
    age_bucket: str = "aged"


def parse_page_mode_token(token: str) -> PageModeSpec:
    """``MODE/SCHEME/BITS[/ESCAPE_DTYPE]`` -- reference ``planner.py:178-197``."""
    parts = [p.strip() for p in token.split("/") if p.strip()]
    if len(parts) not in (3, 4):
        raise ValueError("page mode tokens must use MODE/SCHEME/BITS[/ESCAPE_DTYPE], for example M0/affine/4 or M3/affine/4/int8")
    mode = parts[0].upper()
    if mode not in _KEY_MODES:
        raise ValueError(f"unsupported page mode: {parts[0]}")
    scheme = parts[1].lower()
    if scheme not in ("affine", "symmetric", "lut", "sketch", "project", "turbo3"):
        raise ValueError(f"unsupported quant scheme: {parts[1]}")
    bits = int(parts[2])
    escape = None
    if len(parts) == 4:
        escape = parts[3].lower()
        if escape not in ("float16", "float32", "int8"):
            raise ValueError(f"unsupported escape dtype: {parts[3]}")
        if mode != "M3":
            raise ValueError("escape dtype qualifiers are only supported for M3 page modes")
    return PageModeSpec(mode=mode, bits=bits, quant_scheme=scheme, escape_dtype=escape)


_TIERS = ("exact", "strict", "balanced", "aggressive")


@dataclass(frozen=True, slots=True)
class PageStats:
    """Reference ``planner.py:13-19``."""

    token_count: int
    rms: float
    abs_max: float
    outlier_fraction: float
    channel_range_mean: float


@dataclass(frozen=True, slots=True)
class LayerPolicy:
    """Candidate modes of one (kind, layer, KV head) stream, best first, and
    the recent window that keeps young pages exact -- reference
    ``planner.py:35-44``."""

    policy_id: str
    sensitivity_tier: str
    kind: str
    candidates: tuple[PageModeSpec, ...]
    recent_candidate: PageModeSpec | None = None
    recent_window: int = 128
    outlier_fraction_threshold: float = 0.05
    abs_max_threshold: float = 6.0
    channel_range_threshold: float = 4.0


def observe_page(rows) -> PageStats:
    """Statistics of one page's fp32 rows ``[T, head_dim]`` (numpy, or a
    torch tensor on any device) -- reference ``planner.py:46-70``: rms from
    fp32 squares averaged in fp64, abs max, the fraction of entries at or
    above max(3 rms, 6), and the mean over channels of (max - min)."""
    if not isinstance(rows, np.ndarray) and hasattr(rows, "detach"):
        t = rows.detach().float()
        if t.dim() != 2:
            raise ValueError("tensor_slice must have shape [token_count, head_dim]")
        if t.shape[0] == 0:
            return PageStats(0, 0.0, 0.0, 0.0, 0.0)
        a = t.abs()
        rms = float((t * t).double().mean().sqrt())
        cutoff = max(3.0 * max(rms, 1e-6), 6.0)
        frac = float((a >= cutoff).double().mean())
        crange = float((t.amax(dim=0) - t.amin(dim=0)).double().mean())
        return PageStats(int(t.shape[0]), rms, float(a.max()), frac, crange)
    x = np.asarray(rows, dtype=np.float32)
    if x.ndim != 2:
        raise ValueError("tensor_slice must have shape [token_count, head_dim]")
    if x.shape[0] == 0:
        return PageStats(0, 0.0, 0.0, 0.0, 0.0)
    a = np.abs(x)
    rms = float(np.sqrt(np.mean(np.square(x), dtype=np.float64)))
    cutoff = max(3.0 * max(rms, 1e-6), 6.0)
    frac = float(np.mean(a >= cutoff, dtype=np.float64))
    crange = float(np.mean(x.max(axis=0) - x.min(axis=0), dtype=np.float64))
    return PageStats(int(x.shape[0]), rms, float(a.max()), frac, crange)


# Candidate lists and stat thresholds (outlier fraction, abs max, channel
# range) of the non-exact tiers, best candidate first -- the policy table of
# reference planner.py:214-259.  "P4" stands for the key projection mode,
# M4/project when the config prefers it and M2/sketch otherwise.
_TIER_TABLE = {
    ("K", "strict"): (("M0/affine/4",), (0.02, 4.5, 3.0)),
    ("K", "balanced"): (("M0/affine/2", "P4", "M0/affine/4"), (0.05, 6.0, 4.0)),
    ("K", "aggressive"): (("M0/affine/2", "P4", "M0/affine/4"), (0.10, 8.0, 5.5)),
    ("V", "strict"): (("M1/lut/4", "M0/affine/4"), (0.02, 4.5, 3.0)),
    ("V", "balanced"): (("M0/affine/3", "M1/lut/4", "M0/affine/4"), (0.05, 6.0, 4.0)),
    ("V", "aggressive"): (("M0/affine/2", "M0/affine/3", "M1/lut/4", "M0/affine/4"), (0.10, 8.0, 5.5)),
}


def make_tier_candidates(*, kind: str, sensitivity_tier: str, default_bits: int, default_quant_scheme: str,
                         default_mode: str, recent_window: int, recent_escape_dtype: str = "float16",
                         prefer_project_key_mode: bool = False) -> LayerPolicy:
    """The policy of a sensitivity tier -- reference ``planner.py:199-272``.
    The exact tier keeps the configured mode and has no recent window."""
    def spec(mode: str, scheme: str, bits: int) -> PageModeSpec:
        return PageModeSpec(mode=mode, bits=int(bits), quant_scheme=scheme, sensitivity_tier=sensitivity_tier)

    if sensitivity_tier == "exact":
        mode = default_mode if default_mode in _KEY_MODES else "M0"
        scheme = default_quant_scheme if default_quant_scheme in (
            "affine", "symmetric", "lut", "sketch", "project", "turbo3") else "affine"
        candidates = (spec(mode, scheme, default_bits),)
        thresholds = (0.0, float("inf"), float("inf"))
    else:
        tokens, thresholds = _TIER_TABLE[(kind, sensitivity_tier)]
        project = "M4/project/4" if prefer_project_key_mode else "M2/sketch/4"
        parsed = [parse_page_mode_token(project if t == "P4" else t) for t in tokens]
        candidates = tuple(spec(c.mode, c.quant_scheme, c.bits) for c in parsed)
    return LayerPolicy(
        policy_id=f"{kind.lower()}_{sensitivity_tier}", sensitivity_tier=sensitivity_tier, kind=kind,
        candidates=candidates,
        recent_candidate=PageModeSpec(mode="M3", bits=int(default_bits), quant_scheme="affine",
                                      escape_dtype=recent_escape_dtype, sensitivity_tier=sensitivity_tier),
        recent_window=0 if sensitivity_tier == "exact" else int(recent_window),
        outlier_fraction_threshold=float(thresholds[0]), abs_max_threshold=float(thresholds[1]),
        channel_range_threshold=float(thresholds[2]),
    )


def make_explicit_policy(*, kind: str, policy_id: str, sensitivity_tier: str, candidates, recent_window: int,
                         recent_escape_dtype: str = "float16") -> LayerPolicy:
    """A policy from an explicit candidate list -- reference
    ``planner.py:275-300``: its first M3 candidate (or an M3 page of the
    recent escape dtype) serves the recent window; default thresholds."""
    candidates = tuple(candidates)
    if not candidates:
        raise ValueError("explicit policies must provide at least one candidate")
    recent = next((c for c in candidates if c.mode == "M3"), None)
    if recent is None:
        recent = PageModeSpec(mode="M3", bits=4, quant_scheme="affine", escape_dtype=recent_escape_dtype,
                              sensitivity_tier=sensitivity_tier)
    return LayerPolicy(policy_id=policy_id, sensitivity_tier=sensitivity_tier, kind=kind, candidates=candidates,
                       recent_candidate=recent, recent_window=int(recent_window))


def candidate_needs_stats(candidate: PageModeSpec) -> bool:
    """Whether admitting ``candidate`` depends on the page statistics (M0
    below 4 bits and the M1 / M2 / M4 codecs do; 4/8-bit M0 and M3 never)."""
    return not (candidate.mode == "M3" or (candidate.mode == "M0" and candidate.bits >= 4))


def candidate_is_allowed(candidate: PageModeSpec, *, kind: str, stats: PageStats | None, policy: LayerPolicy) -> bool:
    """Reference ``planner.py:303-342``."""
    if stats is None or not candidate_needs_stats(candidate):
        return True
    quiet = stats.outlier_fraction <= policy.outlier_fraction_threshold
    if candidate.mode in ("M2", "M4"):
        return kind == "K" and quiet and stats.channel_range_mean <= policy.channel_range_threshold
    if candidate.mode == "M1":
        return kind == "V" and quiet and stats.channel_range_mean <= policy.channel_range_threshold
    if candidate.mode == "T3":
        return False
    if candidate.mode == "M0" and candidate.bits <= 2:
        return quiet and stats.abs_max <= policy.abs_max_threshold
    if candidate.mode == "M0" and candidate.bits == 3:
        return (stats.outlier_fraction <= policy.outlier_fraction_threshold * 1.25
                and stats.abs_max <= policy.abs_max_threshold * 1.2)
    return True


def choose_page_mode(layer: int, kind: str, token_age: int, page_stats, *, layer_policy: LayerPolicy) -> PageModeSpec:
    """The page's mode under its stream's policy -- reference
    ``planner.py:75-147``.  A page younger than the recent window takes the
    policy's recent candidate (M3).  Otherwise the first candidate the
    statistics admit, with the failed candidates named in
    ``fallback_reason``; the last candidate when none is admitted.

    ``page_stats`` is a :class:`PageStats`, ``None`` (admit everything), or a
    zero-argument callable returning the statistics, called only when a
    candidate needs them (the device caches compute them on demand)."""
    del layer
    pol = layer_policy

    def tagged(c: PageModeSpec, reason: str, bucket: str) -> PageModeSpec:
        return PageModeSpec(mode=c.mode, bits=c.bits, quant_scheme=c.quant_scheme, escape_dtype=c.escape_dtype,
                            policy_id=pol.policy_id, sensitivity_tier=pol.sensitivity_tier,
                            fallback_reason=reason, age_bucket=bucket)

    if token_age < int(pol.recent_window):
        if pol.recent_candidate is not None:
            return tagged(pol.recent_candidate, "recent_window", "recent")
        last = pol.candidates[-1] if pol.candidates else None
        return tagged(PageModeSpec(mode="M3", bits=last.bits if last else 4,
                                   quant_scheme=last.quant_scheme if last else "affine"), "recent_window", "recent")
    if not pol.candidates:
        return tagged(PageModeSpec(mode="M0", bits=4, quant_scheme="affine"), "no_candidates", "aged")
    stats = page_stats
    failed: list[str] = []
    for i, cand in enumerate(pol.candidates):
        if callable(stats) and candidate_needs_stats(cand):
            stats = stats()
        if candidate_is_allowed(cand, kind=kind, stats=stats if not callable(stats) else None, policy=pol):
            return tagged(cand, "" if i == 0 else ("+".join(failed) or "fallback"), "aged")
        failed.append(f"{cand.mode.lower()}_stats")
    return tagged(pol.candidates[-1], "+".join(failed) if failed else "threshold_fallback", "aged")


def _parse_layer_value(spec: str, field_name: str, allowed: tuple[str, ...]) -> tuple[int, str]:
    """``layer:<id>=<value>`` -- reference ``config.py:31-47``."""
    if "=" not in spec:
        raise ValueError(f"{field_name} entries must use layer:<id>=<value>")
    target, value = spec.split("=", 1)
    parts = target.strip().split(":")
    if len(parts) != 2 or parts[0] != "layer":
        raise ValueError(f"{field_name} entries must use layer:<id>=<value>")
    value = value.strip()
    if value not in allowed:
        raise ValueError(f"{field_name} values must be one of {', '.join(allowed)}")
    return int(parts[1]), value


def _parse_layer_candidates(spec: str, field_name: str) -> tuple[int, tuple[PageModeSpec, ...]]:
    """``layer:<id>=MODE/SCHEME/BITS[,...]`` -- reference ``config.py:50-64``."""
    usage = f"{field_name} entries must use layer:<id>=MODE/SCHEME/BITS[,MODE/SCHEME/BITS...]"
    if "=" not in spec:
        raise ValueError(usage)
    target, raw = spec.split("=", 1)
    parts = target.strip().split(":")
    if len(parts) != 2 or parts[0] != "layer":
        raise ValueError(usage)
    cands = tuple(parse_page_mode_token(t.strip()) for t in raw.split(",") if t.strip())
    if not cands:
        raise ValueError(f"{field_name} entries must include at least one candidate")
    return int(parts[1]), cands


def _parse_override(spec: str, allowed: tuple[str, ...], field_name: str) -> tuple[int, int | None, str]:
    """``layer:<id>[:kv:<id>]=<mode>`` -- reference ``config.py:15-28``."""
    if "=" not in spec:
        raise ValueError(f"{field_name} entries must use layer:<id>=<mode> or layer:<id>:kv:<id>=<mode>")
    target, mode = spec.split("=", 1)
    mode = mode.strip()
    if mode not in allowed:
        raise ValueError(f"{field_name} mode must be one of {', '.join(allowed)}")
    parts = target.strip().split(":")
    if len(parts) == 2 and parts[0] == "layer":
        return int(parts[1]), None, mode
    if len(parts) == 4 and parts[0] == "layer" and parts[2] == "kv":
        return int(parts[1]), int(parts[3]), mode
    raise ValueError(f"{field_name} entries must use layer:<id>=<mode> or layer:<id>:kv:<id>=<mode>")


@dataclass(frozen=True, slots=True)
class DotCacheConfig:
    head_dim: int
    group_size: int = 32
    bits_k: int = 4
    bits_v: int = 4
    tokens_per_page: int = 64
    recent_window: int = 128
    payload_layout_k: str = "group_major"
    payload_layout_v: str = "group_major"
    default_mode_k: str = "M0"
    default_mode_v: str = "M0"
    quant_scheme_k: str = "affine"
    quant_scheme_v: str = "affine"
    escape_dtype: str = "float16"
    recent_page_escape_dtype: str = "float16"
    key_mode_overrides: tuple[str, ...] = ()
    value_mode_overrides: tuple[str, ...] = ()
    prefer_m4_project_k: bool = False
    key_policy_tier: str = "exact"
    value_policy_tier: str = "exact"
    key_layer_sensitivity: tuple[str, ...] = ()
    value_layer_sensitivity: tuple[str, ...] = ()
    key_policy_overrides: tuple[str, ...] = ()
    value_policy_overrides: tuple[str, ...] = ()

    def __post_init__(self) -> None:
        # same checks and messages as reference config.py:186-359 for these fields
        if self.head_dim <= 0:
            raise ValueError("head_dim must be positive")
        if self.group_size <= 0:
            raise ValueError("group_size must be positive")
        if self.bits_k not in (2, 3, 4):
            raise ValueError("bits_k must be 2, 3, or 4 for the current runtime")
        if self.bits_v not in (2, 3, 4):
            raise ValueError("bits_v must be 2, 3, or 4 for the current runtime")
        if self.tokens_per_page <= 0:
            raise ValueError("tokens_per_page must be positive")
        for name in ("payload_layout_k", "payload_layout_v"):
            if getattr(self, name) not in ("group_major", "token_major"):
                raise ValueError(f"{name} must be group_major or token_major")
        if self.default_mode_k not in _KEY_MODES:
            raise ValueError("default_mode_k must be M0, M1, M2, M3, M4, or T3")
        if self.default_mode_v not in _VALUE_MODES:
            raise ValueError("default_mode_v must be M0, M1, M3, or T3")
        if self.quant_scheme_k not in ("affine", "symmetric", "lut", "sketch", "project", "turbo3"):
            raise ValueError("quant_scheme_k must be affine, symmetric, lut, sketch, project, or turbo3")
        if self.quant_scheme_v not in ("affine", "symmetric", "lut", "turbo3"):
            raise ValueError("quant_scheme_v must be affine, symmetric, lut, or turbo3")
        for name in ("escape_dtype", "recent_page_escape_dtype"):
            if getattr(self, name) not in ("float16", "float32", "int8"):
                raise ValueError(f"{name} must be float16, float32, or int8")
        for spec in self.key_mode_overrides:
            _parse_override(spec, _KEY_MODES, "key_mode_overrides")
        for spec in self.value_mode_overrides:
            _parse_override(spec, _VALUE_MODES, "value_mode_overrides")
        for name in ("key_policy_tier", "value_policy_tier"):
            if getattr(self, name) not in _TIERS:
                raise ValueError(f"{name} must be exact, strict, balanced, or aggressive")
        for name in ("key_layer_sensitivity", "value_layer_sensitivity"):
            for spec in getattr(self, name):
                _parse_layer_value(spec, name, _TIERS[1:])
        for name in ("key_policy_overrides", "value_policy_overrides"):
            for spec in getattr(self, name):
                _parse_layer_candidates(spec, name)

    @property
    def num_groups(self) -> int:
        return ceil(self.head_dim / self.group_size)

    @property
    def padded_head_dim(self) -> int:
        return self.num_groups * self.group_size

    def has_mode_overrides(self, *, kind: str | None = None) -> bool:
        """Reference ``config.py:369-374``."""
        k, v = bool(self.key_mode_overrides), bool(self.value_mode_overrides)
        return k if kind == "K" else v if kind == "V" else (k or v)

    def has_policy_overrides(self, *, kind: str | None = None) -> bool:
        """Reference ``config.py:376-388``."""
        k = bool(self.key_layer_sensitivity or self.key_policy_overrides or self.key_policy_tier != "exact")
        v = bool(self.value_layer_sensitivity or self.value_policy_overrides or self.value_policy_tier != "exact")
        return k if kind == "K" else v if kind == "V" else (k or v)

    def chooses_page_modes(self, kind: str) -> bool:
        """Whether pages of ``kind`` take their mode from
        :func:`choose_page_mode` (any mode or policy override of that kind)
        rather than from :meth:`resolve_page_mode` -- the condition of
        reference ``model_kv_cache.py:3164-3174`` and ``:789-810``."""
        return self.has_policy_overrides(kind=kind) or self.has_mode_overrides(kind=kind)

    def resolve_layer_policy(self, *, kind: str, layer_id: int, kv_head_id: int) -> LayerPolicy:
        """Reference ``config.py:546-614``: a mode override gives a one-mode
        explicit policy without a recent window; an explicit candidate list
        for the layer comes next; otherwise the layer's sensitivity tier (the
        kind's default tier unless a layer entry names another)."""
        if kind == "K":
            dmode, dbits, dscheme, tier = self.default_mode_k, self.bits_k, self.quant_scheme_k, self.key_policy_tier
            layer_tiers, explicit = self.key_layer_sensitivity, self.key_policy_overrides
        elif kind == "V":
            dmode, dbits, dscheme, tier = self.default_mode_v, self.bits_v, self.quant_scheme_v, self.value_policy_tier
            layer_tiers, explicit = self.value_layer_sensitivity, self.value_policy_overrides
        else:
            raise ValueError("kind must be K or V")
        field = "key" if kind == "K" else "value"
        mode = self.resolve_page_mode(kind=kind, layer_id=layer_id, kv_head_id=kv_head_id)
        if mode != dmode:
            scheme = {"M1": "lut", "M2": "sketch", "M4": "project", "T3": "turbo3"}.get(mode, dscheme)
            return make_explicit_policy(kind=kind, policy_id=f"{kind.lower()}_mode_override_layer_{int(layer_id)}",
                                        sensitivity_tier="exact",
                                        candidates=(PageModeSpec(mode=mode, bits=dbits, quant_scheme=scheme),),
                                        recent_escape_dtype=self.recent_page_escape_dtype, recent_window=0)
        for spec in explicit:
            lid, cands = _parse_layer_candidates(spec, f"{field}_policy_overrides")
            if lid == int(layer_id):
                return make_explicit_policy(kind=kind, policy_id=f"{kind.lower()}_policy_override_layer_{int(layer_id)}",
                                            sensitivity_tier="balanced", candidates=cands,
                                            recent_escape_dtype=self.recent_page_escape_dtype,
                                            recent_window=self.recent_window)
        for spec in layer_tiers:
            lid, value = _parse_layer_value(spec, f"{field}_layer_sensitivity", _TIERS[1:])
            if lid == int(layer_id):
                tier = value
        return make_tier_candidates(kind=kind, sensitivity_tier=tier, default_bits=dbits, default_quant_scheme=dscheme,
                                    default_mode=dmode, recent_escape_dtype=self.recent_page_escape_dtype,
                                    recent_window=self.recent_window,
                                    prefer_project_key_mode=self.prefer_m4_project_k if kind == "K" else False)

    def select_page_mode(self, *, kind: str, layer_id: int, kv_head_id: int, token_start: int,
                         sequence_length: int, stats=None) -> PageModeSpec | None:
        """The mode spec of a page of ``kind`` whose first token is
        ``token_start`` in a context of ``sequence_length`` tokens, or
        ``None`` when the kind has no overrides (the page then takes
        :meth:`resolve_page_mode`) -- reference
        ``model_kv_cache.py:3164-3185``.  ``stats``: as for
        :func:`choose_page_mode`."""
        if not self.chooses_page_modes(kind):
            return None
        policy = self.resolve_layer_policy(kind=kind, layer_id=layer_id, kv_head_id=kv_head_id)
        age = max(0, int(sequence_length) - int(token_start) - 1)
        return choose_page_mode(int(layer_id), kind, age, stats, layer_policy=policy)

    def resolve_page_mode(self, *, kind: str, layer_id: int, kv_head_id: int) -> str:
        """Last matching override wins -- reference ``config.py:390-414``."""
        if kind == "K":
            resolved, specs, allowed, name = self.default_mode_k, self.key_mode_overrides, _KEY_MODES, "key_mode_overrides"
        elif kind == "V":
            resolved, specs, allowed, name = self.default_mode_v, self.value_mode_overrides, _VALUE_MODES, "value_mode_overrides"
        else:
            raise ValueError("kind must be K or V")
        for spec in specs:
            lid, hid, mode = _parse_override(spec, allowed, name)
            if lid != int(layer_id):
                continue
            if hid is not None and hid != int(kv_head_id):
                continue
            resolved = mode
        return resolved


def recent_window_page_mode(token_age: int, recent_window: int, aged: PageModeSpec) -> PageModeSpec:
    """Pages younger than the recent window are kept exact (M3), the rest use
    the aged spec -- reference ``planner.py:84-106`` with no explicit recent
    candidate."""
    if token_age < int(recent_window):
        return PageModeSpec(
            mode="M3", bits=aged.bits, quant_scheme=aged.quant_scheme, escape_dtype=None,
            policy_id=aged.policy_id, sensitivity_tier=aged.sensitivity_tier,
            fallback_reason="recent_window", age_bucket="recent",
        )
    return aged
