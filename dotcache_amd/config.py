"""Page-format configuration: the slice of reference ``DotCacheConfig`` that
decides how pages are encoded, plus per-page mode specs.

Mirrors reference ``dotcache/config.py:96-414`` for the fields that shape a
page (head_dim, group_size, bits, tokens_per_page, layouts, default modes,
schemes, escape dtypes, recent window) and the Selective Key Precision
sensitivity map (``key_mode_overrides`` / ``value_mode_overrides``,
``layer:<id>[:kv:<id>]=<MODE>``, reference ``config.py:15-28``, ``:390-414``),
and ``PageModeSpec`` / ``parse_page_mode_token`` / the recent-window rule of
reference ``dotcache/planner.py:22-106``, ``:178-197``.  The reference's
``execution_*`` shortlist knobs, M1/M2/M4/T3 knobs and tier policies are not
part of this backend.
"""
from __future__ import annotations

from dataclasses import dataclass
from math import ceil

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

    @property
    def num_groups(self) -> int:
        return ceil(self.head_dim / self.group_size)

    @property
    def padded_head_dim(self) -> int:
        return self.num_groups * self.group_size

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
