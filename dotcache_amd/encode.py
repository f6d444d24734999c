"""Page encode on the GPU (``dc_encode_rows``), behind the reference's
``encode_page`` entry point (reference ``dotcache/encode.py:122-445``, M0 and
M3 branches).

``encode_page`` keeps the reference signature and returns a host
:class:`~dotcache_amd.types.EncodedPage` whose payload, scales, biases and
escape rows are bit-identical to the reference's.  ``encode_into_pool``
encodes device tensors straight into a :class:`DevicePagePool` without a host
round trip (prefill ingest, page finalise and per-token append).
"""
from __future__ import annotations

import numpy as np

from . import _lib
from .config import DotCacheConfig, PageModeSpec
from .page_pool import DevicePagePool, PoolGeometry, page_format_of
from .types import EncodedPage, PageHeader, words_per_group

_scratch_pools: dict[PoolGeometry, DevicePagePool] = {}


def _torch():
    import torch

    return torch


def resolve_encode_spec(config: DotCacheConfig, *, kind: str, mode=None, page_mode: PageModeSpec | None = None,
                        layout=None, quant_scheme=None) -> dict:
    """Bits / mode / layout / scheme / escape resolution of reference
    ``encode.py:144-155`` and ``:185-190`` (a page_mode spec wins)."""
    bits = config.bits_k if kind == "K" else config.bits_v
    default_mode = config.default_mode_k if kind == "K" else config.default_mode_v
    mode_name = page_mode.mode if page_mode is not None else (mode or default_mode)
    if page_mode is not None:
        bits = int(page_mode.bits)
    page_layout = layout or (config.payload_layout_k if kind == "K" else config.payload_layout_v)
    scheme = page_mode.quant_scheme if page_mode is not None else (
        quant_scheme or (config.quant_scheme_k if kind == "K" else config.quant_scheme_v))
    escape = page_mode.escape_dtype if page_mode is not None and page_mode.escape_dtype is not None else config.escape_dtype
    return dict(
        bits=bits, mode=mode_name, layout=page_layout, scheme=scheme, escape_dtype=escape,
        policy_id=page_mode.policy_id if page_mode is not None else "exact_baseline",
        sensitivity_tier=page_mode.sensitivity_tier if page_mode is not None else "exact",
        fallback_reason=page_mode.fallback_reason if page_mode is not None else "",
        age_bucket=page_mode.age_bucket if page_mode is not None else "aged",
    )


def make_header(config: DotCacheConfig, spec: dict, *, kind: str, layer_id: int, kv_head_id: int, token_start: int,
                token_count: int) -> PageHeader:
    """Header fields of reference ``encode.py:191-208`` (M3) / ``:409-426`` (M0)."""
    if spec["mode"] not in ("M0", "M3"):
        raise ValueError(f"page mode {spec['mode']} is not supported by hip_mi355x")
    return PageHeader(
        layer_id=layer_id, kv_head_id=kv_head_id, kind=kind, token_start=token_start, token_count=token_count,
        head_dim=config.head_dim, padded_head_dim=config.padded_head_dim, group_size=config.group_size,
        num_groups=config.num_groups, bits=spec["bits"], words_per_group=words_per_group(config.group_size, spec["bits"]),
        mode_default=spec["mode"], layout=spec["layout"], quant_scheme=spec["scheme"], policy_id=spec["policy_id"],
        sensitivity_tier=spec["sensitivity_tier"], fallback_reason=spec["fallback_reason"],
        age_bucket=spec["age_bucket"], escape_dtype=spec["escape_dtype"] if spec["mode"] == "M3" else config.escape_dtype,
    )


def _scratch_pool(geo: PoolGeometry, device) -> DevicePagePool:
    pool = _scratch_pools.get(geo)
    if pool is None:
        pool = DevicePagePool(geo, device=device, reserve_bytes=1 << 20, reserve_pages=64)
        _scratch_pools[geo] = pool
    return pool


def encode_into_pool(pool: DevicePagePool, values, page_ids, slots) -> None:
    """Encode device rows into pool pages (formats come from the page descriptors)."""
    pool.encode_rows(values, page_ids, slots)


def encode_page(
    tensor_slice,
    config: DotCacheConfig,
    *,
    kind: str,
    layer_id: int = 0,
    kv_head_id: int = 0,
    token_start: int = 0,
    mode: str | None = None,
    page_mode: PageModeSpec | None = None,
    layout: str | None = None,
    quant_scheme: str | None = None,
    build_runtime_metadata: bool = True,
    device="cuda",
) -> EncodedPage:
    """Reference ``encode_page`` computed by the HIP encoder.

    ``tensor_slice`` is ``[token_count, head_dim]`` (numpy or torch; it is
    read as fp32, or as its own fp16/bf16 dtype when it is a torch tensor).
    With ``build_runtime_metadata`` (the reference's default) the page also
    carries the shortlist metadata of its raw rows, computed with numpy as
    the reference computes it (``encode.py:64-75``): fp16 mean, fp16 means
    of ``np.array_split(rows, min(4, T))``, fp16 min and max.
    """
    torch = _torch()
    if isinstance(tensor_slice, torch.Tensor):
        values = tensor_slice.to(device)
        if values.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            values = values.float()
    else:
        arr = np.asarray(tensor_slice, dtype=np.float32)
        values = torch.from_numpy(np.ascontiguousarray(arr)).to(device)
    if values.dim() != 2:
        raise ValueError("tensor_slice must have shape [token_count, head_dim]")
    if values.shape[1] != config.head_dim:
        raise ValueError("tensor_slice head_dim must match config.head_dim")
    spec = resolve_encode_spec(config, kind=kind, mode=mode, page_mode=page_mode, layout=layout, quant_scheme=quant_scheme)
    T = int(values.shape[0])
    header = make_header(config, spec, kind=kind, layer_id=layer_id, kv_head_id=kv_head_id, token_start=token_start,
                         token_count=T)
    fmt, bits = page_format_of(spec["mode"], spec["scheme"], spec["bits"], spec["escape_dtype"])
    cap = max(16, 1 << (max(T, 1) - 1).bit_length())
    pool = _scratch_pool(PoolGeometry(config.head_dim, config.group_size, cap, spec["layout"]), values.device)
    pid = pool.allocate(fmt, bits, 1, tokens=T)
    try:
        if T:
            pool.encode_rows(values, np.full(T, pid[0], dtype=np.int32), np.arange(T, dtype=np.int32))
        page = pool.download_page(int(pid[0]), header)
    finally:
        pool.free(pid)
    page.requested_mode = spec["mode"]
    if build_runtime_metadata and T:
        x = values.float().cpu().numpy()
        chunks = np.array_split(x, min(4, T), axis=0)
        page.runtime_page_mean = x.mean(axis=0).astype(np.float16)
        page.runtime_page_sketch = np.stack([c.mean(axis=0) for c in chunks], axis=0).astype(np.float16)
        page.runtime_page_min = x.min(axis=0).astype(np.float16)
        page.runtime_page_max = x.max(axis=0).astype(np.float16)
    return page
