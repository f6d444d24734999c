"""CPU oracle for the compressed-page decode-attention path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package (``dotcache_amd``)
may import, call or link this module.  It is the checker used by ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``.

It restates, in plain numpy, the reference algorithm for this path:

  * symbol packing              reference ``dotcache/packing.py:6-81``
  * group-major payload layout  reference ``dotcache/page_format.py:19-33``
  * M0 affine / symmetric quantisation
                                reference ``dotcache/modes/m0_affine.py:15-90``
  * M3 escape storage           reference ``dotcache/modes/m3_escape.py:10-37``
  * ``encode_page`` (M0 and M3 branches, header fields, fp16 metadata)
                                reference ``dotcache/encode.py:122-219``, ``:399-445``
  * streaming score / mix       reference ``dotcache/attention_reference.py:16-194``
  * explicit dequantised baseline (the oracle's own oracle)
                                reference ``dotcache/attention_reference.py:197-220``,
                                ``dotcache/decode_reference.py:16-88``
  * ``decode_step`` over a page list (concatenate logits, one global softmax,
    per-page mix)               reference ``dotcache/attention_runtime.py:260-315``
  * per-query multi-query decode reference ``dotcache/attention_runtime.py:203-257``
  * GQA head mapping            reference ``dotcache/model_kv_cache.py:85-95``

How each function is pinned (checked by something other than a retyping of
its own formula) is recorded in ``tests/test_oracle.py``: the reference's own
known-answer tests restated (``tests/test_pack_unpack.py``,
``test_m0_quant.py``, ``test_page_format.py``, ``test_score_reference.py``,
``test_mix_reference.py``, ``test_attention_vs_dense.py``,
``test_escape_mode.py``, ``test_model_kv_cache.py:45-47`` of the reference),
hand-derived quantisation vectors (ties, constant groups, clipping), brute
force against the dense dequantised baseline, and softmax / attention
invariants.  Functions without such a check are marked "parity unpinned" in
their docstring; at present there are none on the path.

numpy >= 2 scalar promotion rules (NEP 50) matter here: Python scalars such
as ``eps`` and ``qmax`` stay weak and the arithmetic is IEEE fp32, exactly as
in the reference running on numpy 2.x.
"""
from __future__ import annotations

import json
from dataclasses import asdict, dataclass, field
from math import ceil
from typing import Sequence

import numpy as np

__all__ = [
    "words_per_group",
    "pack_bits",
    "unpack_bits",
    "quantize_tensor",
    "dequantize_group",
    "dequantize_groups",
    "encode_escape_storage",
    "decode_escape_payload",
    "OracleHeader",
    "OraclePage",
    "encode_page",
    "encode_pages",
    "softmax",
    "score_page_ref",
    "mix_page_ref",
    "decode_page",
    "explicit_dequantized_score",
    "explicit_dequantized_mix",
    "decode_step",
    "decode_multi_query_step",
    "decode_grouped",
    "default_q_head_to_kv_head",
    "page_device_nbytes",
]


# --------------------------------------------------------------------------
# packing (reference dotcache/packing.py)
# --------------------------------------------------------------------------

def words_per_group(group_size: int, bits: int) -> int:
    """``ceil(group_size * bits / 32)`` -- reference ``packing.py:6-11``."""
    if group_size <= 0:
        raise ValueError("group_size must be positive")
    if bits <= 0 or bits > 16:
        raise ValueError("bits must be between 1 and 16")
    return (group_size * bits + 31) // 32


def pack_bits(codes: np.ndarray, bits: int) -> np.ndarray:
    """Little-endian symbol packing into uint32 words.

    Symbol ``k`` of the last axis occupies bits ``[k*bits, (k+1)*bits)`` of the
    concatenated word stream; symbols that straddle a word boundary spill
    their high bits into the low bits of the next word.  Reference
    ``packing.py:14-48``.  Written here as one generic loop over symbols (the
    reference has a vectorised divisor-bits branch that produces the same
    words).
    """
    values = np.asarray(codes, dtype=np.uint32)
    if values.ndim == 0:
        raise ValueError("codes must have at least one dimension")
    mask = (1 << bits) - 1
    if np.any(values > mask):
        raise ValueError("codes contain values that do not fit in the requested bit width")
    n = values.shape[-1]
    nwords = words_per_group(n, bits)
    flat = values.reshape(-1, n).astype(np.uint64)
    out = np.zeros((flat.shape[0], nwords), dtype=np.uint64)
    for k in range(n):
        bit = k * bits
        word, off = divmod(bit, 32)
        shifted = flat[:, k] << np.uint64(off)
        out[:, word] |= shifted & np.uint64(0xFFFFFFFF)
        if off + bits > 32:
            out[:, word + 1] |= shifted >> np.uint64(32)
    return out.astype(np.uint32).reshape(*values.shape[:-1], nwords)


def unpack_bits(words: np.ndarray, bits: int, group_size: int) -> np.ndarray:
    """Inverse of :func:`pack_bits` -- reference ``packing.py:51-81``."""
    packed = np.asarray(words, dtype=np.uint32)
    if packed.ndim == 0:
        raise ValueError("words must have at least one dimension")
    nwords = words_per_group(group_size, bits)
    if packed.shape[-1] != nwords:
        raise ValueError("word count does not match group_size and bits")
    flat = packed.reshape(-1, nwords).astype(np.uint64)
    # append a zero word so a straddling read of the last symbol stays in range
    ext = np.concatenate([flat, np.zeros((flat.shape[0], 1), dtype=np.uint64)], axis=1)
    mask = np.uint64((1 << bits) - 1)
    out = np.zeros((flat.shape[0], group_size), dtype=np.uint8)
    for k in range(group_size):
        word, off = divmod(k * bits, 32)
        pair = ext[:, word] | (ext[:, word + 1] << np.uint64(32))
        out[:, k] = ((pair >> np.uint64(off)) & mask).astype(np.uint8)
    return out.reshape(*packed.shape[:-1], group_size)


def build_payload(codes: np.ndarray, bits: int, layout: str) -> np.ndarray:
    """``codes [T, G, gs]`` -> group_major ``[G, T, W]`` or token_major ``[T, G, W]``.

    Reference ``page_format.py:19-23``.
    """
    if layout == "group_major":
        return pack_bits(np.transpose(codes, (1, 0, 2)), bits)
    return pack_bits(codes, bits)


def load_group_words(page: "OraclePage", group_index: int) -> np.ndarray:
    """Reference ``page_format.py:26-33``."""
    if page.payload is None:
        raise ValueError("M3 pages do not have packed payload")
    if group_index < 0 or group_index >= page.header.num_groups:
        raise IndexError("group_index out of range")
    if page.header.layout == "group_major":
        return page.payload[group_index]
    return page.payload[:, group_index, :]


# --------------------------------------------------------------------------
# M0 codec (reference dotcache/modes/m0_affine.py)
# --------------------------------------------------------------------------

def quantize_tensor(values: np.ndarray, *, group_size: int, bits: int, scheme: str = "affine", eps: float = 1e-8):
    """Per (token, group) quantisation -- reference ``m0_affine.py:15-53``.

    affine:    ``s = max((xmax - xmin) / (2^b - 1), eps)``, ``code = clip(rint((x - xmin) / s), 0, 2^b - 1)``,
               ``bias = xmin``.
    symmetric: ``qmax = 2^(b-1) - 1``; ``s = max(max|x| / qmax, eps)``;
               ``code = clip(rint(x / s), -qmax, qmax) + qmax``.
    All arithmetic is IEEE fp32; ``rint`` rounds half to even.  Channels past
    ``head_dim`` are zero padding and take part in min / max.
    """
    x = np.asarray(values, dtype=np.float32)
    if x.ndim != 2:
        raise ValueError("values must have shape [token_count, head_dim]")
    t, hd = x.shape
    g = ceil(hd / group_size)
    phd = g * group_size
    if phd != hd:
        x = np.concatenate([x, np.zeros((t, phd - hd), dtype=np.float32)], axis=1)
    grouped = x.reshape(t, g, group_size)
    eps32 = np.float32(eps)
    if scheme == "affine":
        levels = np.float32(max((1 << bits) - 1, 1))
        lo = grouped.min(axis=-1)
        hi = grouped.max(axis=-1)
        scales = np.maximum((hi - lo) / levels, eps32).astype(np.float32)
        q = np.rint((grouped - lo[..., None]) / scales[..., None])
        codes = np.clip(q, 0, (1 << bits) - 1).astype(np.uint8)
        return codes, scales, lo.astype(np.float32), phd
    if scheme == "symmetric":
        qmax = (1 << (bits - 1)) - 1
        amax = np.abs(grouped).max(axis=-1)
        scales = np.maximum(amax / np.float32(max(qmax, 1)), eps32).astype(np.float32)
        q = np.clip(np.rint(grouped / scales[..., None]), -qmax, qmax).astype(np.int32) + qmax
        codes = np.clip(q, 0, (1 << bits) - 1).astype(np.uint8)
        return codes, scales, None, phd
    raise ValueError("scheme must be affine or symmetric")


def dequantize_group(codes, *, scales, bias, bits: int, scheme: str) -> np.ndarray:
    """Reference ``m0_affine.py:56-76``."""
    c = np.asarray(codes, dtype=np.float32)
    s = np.asarray(scales, dtype=np.float32)
    if scheme == "affine":
        if bias is None:
            raise ValueError("affine mode requires bias")
        return s * c + np.asarray(bias, dtype=np.float32)
    if scheme == "symmetric":
        return s * (c - np.float32((1 << (bits - 1)) - 1))
    raise ValueError("scheme must be affine or symmetric")


def dequantize_groups(codes, *, scales, bias, bits: int, scheme: str) -> np.ndarray:
    """Reference ``m0_affine.py:79-90``."""
    s = np.asarray(scales, dtype=np.float32)[..., None]
    b = None if bias is None else np.asarray(bias, dtype=np.float32)[..., None]
    return dequantize_group(codes, scales=s, bias=b, bits=bits, scheme=scheme)


# --------------------------------------------------------------------------
# M3 escape (reference dotcache/modes/m3_escape.py)
# --------------------------------------------------------------------------

def encode_escape_storage(values, dtype: str = "float16"):
    """Reference ``m3_escape.py:10-19``."""
    x = np.asarray(values, dtype=np.float32)
    if dtype in ("float16", "float32"):
        return x.astype(np.dtype(dtype)), None
    if dtype == "int8":
        amax = np.abs(x).max(axis=1)
        scales = np.maximum(amax / np.float32(127.0), np.float32(1e-8)).astype(np.float16)
        q = np.clip(np.rint(x / scales[:, None]), -127.0, 127.0).astype(np.int8)
        return q, scales
    raise ValueError(f"unsupported escape dtype: {dtype}")


def decode_escape_payload(payload, *, head_dim=None, scales=None) -> np.ndarray:
    """Reference ``m3_escape.py:22-37``."""
    a = np.asarray(payload)
    if a.dtype == np.int8:
        if scales is None:
            raise ValueError("int8 escape payloads require scales")
        out = a.astype(np.float32) * np.asarray(scales, dtype=np.float32)[:, None]
    else:
        out = a.astype(np.float32)
    return out if head_dim is None else out[:, :head_dim]


# --------------------------------------------------------------------------
# page container + encode (reference dotcache/types.py, dotcache/encode.py)
# --------------------------------------------------------------------------

@dataclass
class OracleHeader:
    """The 20 header fields of reference ``types.py:15-36``."""

    layer_id: int
    kv_head_id: int
    kind: str
    token_start: int
    token_count: int
    head_dim: int
    padded_head_dim: int
    group_size: int
    num_groups: int
    bits: int
    words_per_group: int
    mode_default: str
    layout: str
    quant_scheme: str
    policy_id: str = "exact_baseline"
    sensitivity_tier: str = "exact"
    fallback_reason: str = ""
    age_bucket: str = "aged"
    escape_dtype: str = "float16"
    project_basis: str = "hadamard"

    def to_dict(self) -> dict:
        return asdict(self)

    def to_json(self) -> str:
        return json.dumps(self.to_dict(), sort_keys=True)


@dataclass
class OraclePage:
    header: OracleHeader
    payload: np.ndarray | None = None
    scales: np.ndarray | None = None
    bias: np.ndarray | None = None
    escape_payload: np.ndarray | None = None
    escape_scales: np.ndarray | None = None
    runtime_page_mean: np.ndarray | None = None
    runtime_page_sketch: np.ndarray | None = None
    runtime_page_min: np.ndarray | None = None
    runtime_page_max: np.ndarray | None = None
    full_page_decode_calls: int = 0
    extra: dict = field(default_factory=dict)

    @property
    def payload_nbytes(self) -> int:
        n = 0
        if self.payload is not None:
            n += int(self.payload.nbytes)
        if self.escape_payload is not None:
            n += int(self.escape_payload.nbytes)
        return n


def encode_page(
    values,
    *,
    head_dim: int,
    group_size: int,
    kind: str,
    bits: int = 4,
    mode: str = "M0",
    scheme: str = "affine",
    layout: str = "group_major",
    escape_dtype: str = "float16",
    layer_id: int = 0,
    kv_head_id: int = 0,
    token_start: int = 0,
    policy_id: str = "exact_baseline",
    sensitivity_tier: str = "exact",
    fallback_reason: str = "",
    age_bucket: str = "aged",
    build_runtime_metadata: bool = False,
) -> OraclePage:
    """Encode ``values [T, head_dim]`` into one page.

    Reference ``encode.py:122-219`` (M3) and ``:399-445`` (M0).  Differences
    of presentation only: the config / page-mode resolution of ``:144-155``
    is done by the caller, who passes the resolved ``bits``, ``mode``,
    ``scheme`` and ``layout``; the runtime sketch/envelope metadata of
    ``:163-165`` (shortlist-only, not read by score or mix) is built only
    with ``build_runtime_metadata=True`` (:func:`runtime_page_metadata`).
    M0 scales and biases are stored as fp16 (``:427-428``); the codes are
    computed with the fp32 scale before that rounding (``m0_affine.py``).
    """
    x = np.asarray(values, dtype=np.float32)
    if x.ndim != 2:
        raise ValueError("tensor_slice must have shape [token_count, head_dim]")
    if x.shape[1] != head_dim:
        raise ValueError("tensor_slice head_dim must match config.head_dim")
    ng = ceil(head_dim / group_size)
    common = dict(
        layer_id=layer_id, kv_head_id=kv_head_id, kind=kind, token_start=token_start,
        token_count=int(x.shape[0]), head_dim=head_dim, group_size=group_size, num_groups=ng,
        bits=bits, words_per_group=words_per_group(group_size, bits), layout=layout,
        quant_scheme=scheme, policy_id=policy_id, sensitivity_tier=sensitivity_tier,
        fallback_reason=fallback_reason, age_bucket=age_bucket,
    )
    runtime = runtime_page_metadata(x) if build_runtime_metadata and x.shape[0] > 0 else {}
    if mode == "M3":
        header = OracleHeader(padded_head_dim=ng * group_size, mode_default="M3", escape_dtype=escape_dtype, **common)
        esc, esc_scales = encode_escape_storage(x, dtype=escape_dtype)
        return OraclePage(header=header, escape_payload=esc, escape_scales=esc_scales, **runtime)
    if mode != "M0":
        raise ValueError("only M0 and M3 pages are on this path")
    codes, scales, bias, phd = quantize_tensor(x, group_size=group_size, bits=bits, scheme=scheme)
    header = OracleHeader(padded_head_dim=phd, mode_default="M0", escape_dtype=escape_dtype, **common)
    return OraclePage(
        header=header,
        payload=build_payload(codes, bits, layout),
        scales=scales.astype(np.float16),
        bias=None if bias is None else bias.astype(np.float16),
        **runtime,
    )


RUNTIME_SKETCH_ROWS = 4  # reference encode.py:17


def runtime_page_metadata(values) -> dict:
    """The shortlist metadata the reference encoder stores with a page, from
    the raw (unquantised) rows: fp16 mean, fp16 means of
    ``np.array_split(rows, min(4, T))``, fp16 per-channel min and max --
    reference ``encode.py:64-75`` (built at ``:163-165``)."""
    x = np.asarray(values, dtype=np.float32)
    rows = min(max(1, RUNTIME_SKETCH_ROWS), x.shape[0])
    chunks = np.array_split(x, rows, axis=0)
    return dict(
        runtime_page_mean=x.mean(axis=0).astype(np.float16),
        runtime_page_sketch=np.stack([c.mean(axis=0) for c in chunks], axis=0).astype(np.float16),
        runtime_page_min=x.min(axis=0).astype(np.float16),
        runtime_page_max=x.max(axis=0).astype(np.float16),
    )


def encode_pages(values, *, tokens_per_page: int, **kw) -> list[OraclePage]:
    """Split ``values [N, hd]`` into consecutive pages (last one partial)."""
    x = np.asarray(values, dtype=np.float32)
    pages = []
    for start in range(0, x.shape[0], tokens_per_page):
        pages.append(encode_page(x[start:start + tokens_per_page], token_start=start, **kw))
    return pages


def page_device_nbytes(page: OraclePage) -> int:
    """Compressed bytes a reader must fetch for this page: packed codes, fp16
    scales, fp16 biases, escape rows (and int8-escape row scales)."""
    n = page.payload_nbytes
    for a in (page.scales, page.bias, page.escape_scales):
        if a is not None:
            n += int(a.nbytes)
    return n


# --------------------------------------------------------------------------
# read path (reference dotcache/attention_reference.py, decode_reference.py)
# --------------------------------------------------------------------------

def softmax(logits) -> np.ndarray:
    """Reference ``attention_reference.py:27-31``."""
    v = np.asarray(logits, dtype=np.float32)
    e = np.exp(v - np.max(v))
    return e / np.sum(e)


def _pad_query(q, padded_head_dim: int) -> np.ndarray:
    q = np.asarray(q, dtype=np.float32)
    if q.ndim != 1:
        raise ValueError("query_slice must have shape [head_dim]")
    if q.shape[0] > padded_head_dim:
        raise ValueError("query head_dim exceeds padded_head_dim")
    if q.shape[0] == padded_head_dim:
        return q
    return np.concatenate([q, np.zeros(padded_head_dim - q.shape[0], dtype=np.float32)])


def score_page_ref(query, page: OraclePage) -> np.ndarray:
    """Streaming score over one page -- reference ``attention_reference.py:34-128``.

    M3: ``fp32(escape) @ q``.  M0 affine: ``sum_g s[t,g] (c[t,g,:] . q_g) + b[t,g] sum(q_g)``.
    M0 symmetric: ``sum_g s[t,g] ((c[t,g,:] - zp) . q_g)``.
    """
    h = page.header
    if h.mode_default == "M3":
        dense = decode_escape_payload(page.escape_payload, head_dim=h.head_dim, scales=page.escape_scales)
        return dense @ np.asarray(query, dtype=np.float32)
    q = _pad_query(query, h.padded_head_dim)
    qg = q.reshape(h.num_groups, h.group_size)
    qsum = qg.sum(axis=-1)
    logits = np.zeros(h.token_count, dtype=np.float32)
    for g in range(h.num_groups):
        codes = unpack_bits(load_group_words(page, g), h.bits, h.group_size).astype(np.float32)
        s = page.scales[:, g].astype(np.float32)
        if h.quant_scheme == "affine":
            b = page.bias[:, g].astype(np.float32)
            logits += s * (codes @ qg[g]) + b * qsum[g]
        else:
            zp = np.float32((1 << (h.bits - 1)) - 1)
            logits += s * ((codes - zp) @ qg[g])
    return logits


def mix_page_ref(weights, page: OraclePage, out_acc=None) -> np.ndarray:
    """Streaming mix over one page -- reference ``attention_reference.py:131-194``."""
    h = page.header
    w = np.asarray(weights, dtype=np.float32)
    if w.shape != (h.token_count,):
        raise ValueError("attn_weights must have shape [token_count]")
    out = np.zeros(h.padded_head_dim, dtype=np.float32) if out_acc is None else np.array(out_acc, dtype=np.float32)
    if out.shape != (h.padded_head_dim,):
        raise ValueError("out_acc must have shape [padded_head_dim]")
    if h.mode_default == "M3":
        dense = decode_escape_payload(page.escape_payload, head_dim=h.head_dim, scales=page.escape_scales)
        out[: h.head_dim] += w @ dense
        return out[: h.head_dim].copy()
    for g in range(h.num_groups):
        codes = unpack_bits(load_group_words(page, g), h.bits, h.group_size).astype(np.float32)
        s = page.scales[:, g].astype(np.float32)[:, None]
        if h.quant_scheme == "affine":
            grp = s * codes + page.bias[:, g].astype(np.float32)[:, None]
        else:
            grp = s * (codes - np.float32((1 << (h.bits - 1)) - 1))
        out[g * h.group_size:(g + 1) * h.group_size] += w @ grp
    return out[: h.head_dim].copy()


def decode_page(page: OraclePage) -> np.ndarray:
    """Dense dequantisation of a whole page -- reference ``decode_reference.py:16-88``."""
    page.full_page_decode_calls += 1
    h = page.header
    if h.mode_default == "M3":
        return decode_escape_payload(page.escape_payload, head_dim=h.head_dim, scales=page.escape_scales)
    parts = []
    for g in range(h.num_groups):
        codes = unpack_bits(load_group_words(page, g), h.bits, h.group_size)
        s = page.scales[:, g].astype(np.float32)[:, None]
        b = None if page.bias is None else page.bias[:, g].astype(np.float32)[:, None]
        parts.append(dequantize_group(codes, scales=s, bias=b, bits=h.bits, scheme=h.quant_scheme))
    return np.concatenate(parts, axis=-1)[:, : h.head_dim]


def explicit_dequantized_score(query, page: OraclePage) -> np.ndarray:
    """Reference ``attention_reference.py:197-200``."""
    return decode_page(page) @ np.asarray(query, dtype=np.float32)


def explicit_dequantized_mix(weights, page: OraclePage) -> np.ndarray:
    """Reference ``attention_reference.py:203-206``."""
    return np.asarray(weights, dtype=np.float32) @ decode_page(page)


def decode_step(query, key_pages: Sequence[OraclePage], value_pages: Sequence[OraclePage], *, page_logits=None):
    """One decode step over a page list -- reference ``attention_runtime.py:260-315``.

    Logits of all pages are concatenated, one global softmax is taken, and
    each value page mixes its slice of the weights.  Returns
    ``(logits, weights, output[head_dim])``.
    """
    if len(key_pages) != len(value_pages):
        raise ValueError("key_pages and value_pages must contain the same number of pages")
    if not key_pages:
        raise ValueError("decode_step requires at least one page")
    if page_logits is not None and len(page_logits) != len(key_pages):
        raise ValueError("page_logits must align with key_pages")
    parts = []
    for i, kp in enumerate(key_pages):
        cached = None if page_logits is None else page_logits[i]
        parts.append(np.asarray(score_page_ref(query, kp) if cached is None else cached, dtype=np.float32))
    logits = np.concatenate(parts).astype(np.float32)
    weights = softmax(logits)
    out = np.zeros(key_pages[0].header.head_dim, dtype=np.float32)
    off = 0
    for vp in value_pages:
        n = vp.header.token_count
        out = out + mix_page_ref(weights[off:off + n], vp)
        off += n
    return logits, weights, out


def decode_multi_query_step(queries, key_pages, value_pages):
    """Per-query loop -- reference ``attention_runtime.py:203-257`` (cpu path)."""
    q = np.asarray(queries, dtype=np.float32)
    if q.ndim != 2:
        raise ValueError("query_slices must have shape [query_count, head_dim]")
    res = [decode_step(qi, key_pages, value_pages) for qi in q]
    return (np.stack([r[0] for r in res]), np.stack([r[1] for r in res]), np.stack([r[2] for r in res]))


def decode_grouped(queries, key_pages_by_group, value_pages_by_group) -> np.ndarray:
    """``queries [G, Q, hd]`` against per-group page lists -> ``[G, Q, hd]``.

    The group axis is the KV head (and, for a batch, the (sequence, KV head)
    pair); the Q axis is the GQA query heads sharing that KV head.  Semantics
    of reference ``torch_mps.py:4110-4273`` computed with the cpu path's
    per-query ``decode_step``.
    """
    q = np.asarray(queries, dtype=np.float32)
    out = np.zeros(q.shape, dtype=np.float32)
    for g in range(q.shape[0]):
        out[g] = decode_multi_query_step(q[g], key_pages_by_group[g], value_pages_by_group[g])[2]
    return out


def default_q_head_to_kv_head(num_attention_heads: int, num_key_value_heads: int) -> np.ndarray:
    """``q // (Hq / Hkv)`` -- reference ``model_kv_cache.py:85-95``."""
    if num_attention_heads % num_key_value_heads:
        raise ValueError("num_attention_heads must be divisible by num_key_value_heads")
    rep = num_attention_heads // num_key_value_heads
    return (np.arange(num_attention_heads, dtype=np.int64) // rep).astype(np.int64)
