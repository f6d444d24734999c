"""Page metadata and host page container.

Same contract as reference ``dotcache/types.py:15-112``: the 20-field
:class:`PageHeader` serialised as sorted-key JSON, and :class:`EncodedPage`
holding host numpy arrays -- payload ``[G, T, W]`` uint32 (group_major),
scales / bias ``[T, G]`` fp16, escape rows ``[T, head_dim]`` -- with the same
byte accounting.  ``EncodedPage`` also carries the optional runtime
shortlist metadata of the raw rows (fp16 mean, chunk-mean sketch, min, max;
reference ``dotcache/encode.py:64-75``): ``encode.encode_page`` builds it by
default, as the reference does, and pages read back from a device pool have
none.
"""
from __future__ import annotations

import json
from dataclasses import asdict, dataclass
from typing import Literal

import numpy as np

Kind = Literal["K", "V"]
Layout = Literal["group_major", "token_major"]
Mode = Literal["M0", "M1", "M2", "M3", "M4", "T3"]
QuantScheme = Literal["affine", "symmetric", "lut", "sketch", "project", "turbo3"]


@dataclass(slots=True)
class PageHeader:
    layer_id: int
    kv_head_id: int
    kind: Kind
    token_start: int
    token_count: int
    head_dim: int
    padded_head_dim: int
    group_size: int
    num_groups: int
    bits: int
    words_per_group: int
    mode_default: Mode
    layout: Layout
    quant_scheme: QuantScheme
    policy_id: str = "exact_baseline"
    sensitivity_tier: str = "exact"
    fallback_reason: str = ""
    age_bucket: str = "aged"
    escape_dtype: str = "float16"
    project_basis: str = "hadamard"

    def to_dict(self) -> dict[str, int | str]:
        return asdict(self)

    @classmethod
    def from_dict(cls, data: dict[str, int | str]) -> "PageHeader":
        return cls(**data)

    def to_json(self) -> str:
        return json.dumps(self.to_dict(), sort_keys=True)

    @classmethod
    def from_json(cls, payload: str) -> "PageHeader":
        return cls.from_dict(json.loads(payload))


@dataclass(slots=True)
class EncodedPage:
    header: PageHeader
    payload: np.ndarray | None = None
    scales: np.ndarray | None = None
    bias: np.ndarray | None = None
    escape_payload: np.ndarray | None = None
    escape_scales: np.ndarray | None = None
    # shortlist metadata of the raw rows (fp16), as the reference encoder
    # stores it (encode.py:64-75); None where the page was built without it
    runtime_page_mean: np.ndarray | None = None
    runtime_page_sketch: np.ndarray | None = None
    runtime_page_min: np.ndarray | None = None
    runtime_page_max: np.ndarray | None = None
    requested_mode: str | None = None
    full_page_decode_calls: int = 0
    decode_group_calls: int = 0

    @property
    def payload_nbytes(self) -> int:
        total = 0
        if self.payload is not None:
            total += int(self.payload.nbytes)
        if self.escape_payload is not None:
            total += int(self.escape_payload.nbytes)
        return total

    @property
    def metadata_nbytes(self) -> int:
        total = len(self.header.to_json().encode("utf-8"))
        for arr in (self.scales, self.bias, self.escape_scales):
            if arr is not None:
                total += int(arr.nbytes)
        return total

    @property
    def total_nbytes(self) -> int:
        return self.payload_nbytes + self.metadata_nbytes

    @property
    def device_nbytes(self) -> int:
        """Bytes a device reader fetches: codes or escape rows plus fp16
        scales / biases (no JSON header)."""
        total = self.payload_nbytes
        for arr in (self.scales, self.bias, self.escape_scales):
            if arr is not None:
                total += int(arr.nbytes)
        return total


def serialize_header(header: PageHeader) -> bytes:
    """Reference ``dotcache/page_format.py:11-12``."""
    return header.to_json().encode("utf-8")


def deserialize_header(payload: bytes) -> PageHeader:
    """Reference ``dotcache/page_format.py:15-16``."""
    return PageHeader.from_json(payload.decode("utf-8"))


def words_per_group(group_size: int, bits: int) -> int:
    """Reference ``dotcache/packing.py:6-11``."""
    if group_size <= 0:
        raise ValueError("group_size must be positive")
    if bits <= 0 or bits > 16:
        raise ValueError("bits must be between 1 and 16")
    return (group_size * bits + 31) // 32
