"""ctypes binding of ``libdotcache_hip.so`` (declared in ``include/dotcache_hip.h``).

The library is loaded lazily from the package directory.  A missing library
raises :class:`RuntimeError` -- there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libdotcache_hip.so"

DC_OK, DC_EINVAL, DC_EDEVICE, DC_ESPACE = 0, 1, 2, 3
FMT_M3_F16, FMT_M0_AFFINE, FMT_M0_SYMMETRIC, FMT_M3_F32, FMT_M3_I8 = 0, 1, 2, 3, 4
DT_F32, DT_F16, DT_BF16 = 0, 1, 2


class PageDesc(C.Structure):
    _fields_ = [("block", C.c_uint32), ("tokens", C.c_uint16), ("format", C.c_uint8), ("bits", C.c_uint8)]


class PageRecord(C.Structure):
    _fields_ = [("key", PageDesc), ("value", PageDesc)]


class PageGeometry(C.Structure):
    _fields_ = [("head_dim", C.c_int32), ("group_size", C.c_int32), ("page_capacity", C.c_int32), ("layout", C.c_int32)]


class Pool(C.Structure):
    _fields_ = [
        ("arena", C.c_void_p),
        ("arena_bytes", C.c_int64),
        ("descs", C.c_void_p),
        ("n_descs", C.c_int32),
        ("geometry", PageGeometry),
        ("format_mask", C.c_uint64),
    ]


def format_bit(fmt: int, bits: int) -> int:
    """Bit of a page format in dc_pool.format_mask (format * 9 + bits, bits 0 for M3)."""
    return 1 << (int(fmt) * 9 + (0 if fmt in (FMT_M3_F16, FMT_M3_F32, FMT_M3_I8) else int(bits)))


class WorkItem(C.Structure):
    _fields_ = [
        ("seq", C.c_int32), ("kv_head", C.c_int32), ("page_begin", C.c_int32), ("page_end", C.c_int32),
        ("partial", C.c_int32), ("chunk_begin", C.c_int32), ("chunk_end", C.c_int32), ("reserved", C.c_int32),
    ]


class MergeItem(C.Structure):
    _fields_ = [("seq", C.c_int32), ("kv_head", C.c_int32), ("partial_begin", C.c_int32), ("count", C.c_int32)]


assert C.sizeof(PageDesc) == 8 and C.sizeof(WorkItem) == 32 and C.sizeof(MergeItem) == 16

# name -> (restype, argtypes); this table is also the list of exported
# symbols the CPU tests check against include/dotcache_hip.h.
SIGNATURES = {
    "dc_last_error": (C.c_char_p, []),
    "dc_abi_version": (C.c_int32, []),
    "dc_page_blob_bytes": (C.c_int64, [C.c_int32, C.c_int32, PageGeometry]),
    "dc_page_read_bytes": (C.c_int64, [C.c_int32, C.c_int32, C.c_int32, PageGeometry]),
    "dc_encode_rows": (C.c_int, [C.c_void_p, C.c_int32, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, Pool, C.c_void_p]),
    "dc_encode_rows_kv": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p,
                                    C.c_void_p, C.c_void_p, Pool, Pool, C.c_void_p]),
    "dc_set_encode_path": (C.c_int, [C.c_int32]),
    "dc_score_pages": (C.c_int, [Pool, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_int32, C.c_void_p, C.c_int64, C.c_void_p]),
    "dc_mix_pages": (C.c_int, [Pool, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_int32, C.c_int64, C.c_void_p, C.c_int32, C.c_void_p]),
    "dc_score_pages_grouped": (C.c_int, [Pool, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_void_p,
                                         C.c_int32, C.c_void_p, C.c_int64, C.c_void_p]),
    "dc_mix_pages_grouped": (C.c_int, [Pool, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_void_p,
                                       C.c_int32, C.c_int64, C.c_void_p, C.c_int32, C.c_void_p]),
    "dc_softmax_rows": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_int64, C.c_void_p]),
    "dc_page_summaries": (C.c_int, [Pool, C.c_void_p, C.c_int32, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p,
                                    C.c_void_p, C.c_void_p]),
    "dc_page_relevance": (C.c_int, [C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_int32,
                                    C.c_int32, C.c_void_p, C.c_void_p]),
    "dc_select_top_k": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_void_p, C.c_void_p]),
    "dc_plan_decode": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_void_p, C.c_int32, C.POINTER(C.c_int32),
                                 C.c_void_p, C.c_int32, C.POINTER(C.c_int32), C.POINTER(C.c_int32)]),
    "dc_plan_decode_fill": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_void_p, C.c_int64,
                                      C.c_int32,
                                      C.c_int32, C.c_void_p, C.c_int32, C.POINTER(C.c_int32), C.c_void_p, C.c_int32,
                                      C.POINTER(C.c_int32), C.POINTER(C.c_int32), C.POINTER(C.c_int32)]),
    "dc_decode_paged": (C.c_int, [Pool, Pool, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_int32, C.c_void_p, C.c_int32,
                                  C.c_void_p, C.c_int32, C.c_float, C.c_int32, C.c_int32, C.c_int32, C.c_void_p,
                                  C.c_void_p, C.c_int64, C.c_void_p]),
    "dc_gather_page_records": (C.c_int, [Pool, Pool, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_int32,
                                         C.c_int32, C.c_int32, C.c_void_p, C.c_int32, C.c_void_p]),
    "dc_decode_paged_records": (C.c_int, [Pool, Pool, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_int32,
                                          C.c_void_p, C.c_int32, C.c_void_p, C.c_int32, C.c_float, C.c_int32,
                                          C.c_int32, C.c_int32, C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p,
                                          C.c_int32, C.c_void_p]),
    "dc_decode_waves_per_simd": (C.c_int32, [Pool, Pool, C.c_int32]),
    "dc_decode_workspace_bytes": (C.c_int64, [C.c_int32, C.c_int32, C.c_int32]),
    "dc_decode_paged_noalloc": (C.c_int, [Pool, Pool, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_int32,
                                          C.c_void_p, C.c_int32, C.c_int32, C.c_void_p, C.c_int32, C.c_float,
                                          C.c_int32, C.c_int32, C.c_int32, C.c_void_p, C.c_void_p]),
    "dc_decode_noalloc_scratch_bytes": (C.c_int64, []),
    "dc_set_decode_path": (C.c_int, [C.c_int32]),
    "dc_set_mfma_head_block": (C.c_int, [C.c_int32]),
    "dc_lse_merge": (C.c_int, [C.c_void_p, C.c_int32, C.c_void_p, C.c_int64, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                               C.c_void_p, C.c_void_p]),
    "dc_window_merge": (C.c_int, [Pool, Pool, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p, C.c_int32,
                                  C.c_void_p, C.c_int32, C.c_float, C.c_int32, C.c_int32, C.c_int32, C.c_void_p,
                                  C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p]),
}

_lib: C.CDLL | None = None


def lib() -> C.CDLL:
    """The loaded library; raises RuntimeError if it was never built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built; run `python -m dotcache_amd._build` "
                "(or __graft_entry__.build()) first -- there is no CPU fallback"
            )
        handle = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    """Map a dc_status to the reference's exception convention."""
    if status == DC_OK:
        return
    msg = lib().dc_last_error().decode("utf-8", "replace")
    if status == DC_EINVAL:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


def geometry(head_dim: int, group_size: int, page_capacity: int, layout: str = "group_major") -> PageGeometry:
    if layout not in ("group_major", "token_major"):
        raise ValueError("layout must be group_major or token_major")
    return PageGeometry(head_dim, group_size, page_capacity, 0 if layout == "group_major" else 1)


def page_blob_bytes(fmt: int, bits: int, geo: PageGeometry) -> int:
    n = int(lib().dc_page_blob_bytes(fmt, bits, geo))
    if n < 0:
        raise ValueError(f"unsupported page format {fmt}/{bits} for geometry")
    return n


def page_read_bytes(fmt: int, bits: int, tokens: int, geo: PageGeometry) -> int:
    n = int(lib().dc_page_read_bytes(fmt, bits, tokens, geo))
    if n < 0:
        raise ValueError(f"unsupported page format {fmt}/{bits} for geometry")
    return n
