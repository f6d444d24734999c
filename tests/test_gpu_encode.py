"""GPU encode parity: dc_encode_rows (through the product's encode_page and
the pool API) is bit-exact with the oracle's encode_page -- packed codes,
fp16 scales, fp16 biases, escape rows and header fields."""
import numpy as np
import pytest

from oracle import dotcache_oracle as O
from tests.helpers import hard_values

pytestmark = pytest.mark.gpu


def _torch():
    import torch

    return torch


def _assert_same_page(got, want):
    assert got.header.to_dict() == want.header.to_dict()
    for name in ("payload", "scales", "bias", "escape_payload", "escape_scales"):
        a, b = getattr(got, name), getattr(want, name)
        assert (a is None) == (b is None), name
        if a is not None:
            assert a.dtype == b.dtype and a.shape == b.shape, name
            np.testing.assert_array_equal(a.view(np.uint8), b.view(np.uint8), err_msg=name)


CASES = [
    # (head_dim, group_size, bits, scheme, tokens)
    (128, 32, 4, "symmetric", 64),
    (128, 32, 4, "affine", 64),
    (64, 32, 4, "affine", 64),
    (128, 64, 8, "symmetric", 64),
    (256, 32, 4, "affine", 128),
    (48, 32, 4, "affine", 7),
    (128, 32, 2, "affine", 33),
    (128, 32, 3, "affine", 40),
    (96, 32, 3, "symmetric", 64),
    (128, 32, 8, "affine", 1),
    (32, 16, 2, "symmetric", 17),
]


@pytest.mark.parametrize("hd,gs,bits,scheme,T", CASES)
def test_encode_page_bit_exact(hd, gs, bits, scheme, T):
    from dotcache_amd.config import DotCacheConfig, PageModeSpec
    from dotcache_amd.encode import encode_page

    rng = np.random.default_rng(hd * 1000 + gs * 10 + bits)
    x = hard_values(rng, T, hd)
    cfg = DotCacheConfig(head_dim=hd, group_size=gs)
    spec = PageModeSpec("M0", bits, scheme)
    got = encode_page(x, cfg, kind="V", layer_id=3, kv_head_id=1, token_start=128, page_mode=spec)
    want = O.encode_page(x, head_dim=hd, group_size=gs, bits=bits, kind="V", scheme=scheme, layer_id=3, kv_head_id=1,
                         token_start=128)
    _assert_same_page(got, want)


@pytest.mark.parametrize("escape", ["float16", "float32", "int8"])
def test_encode_m3_bit_exact(escape):
    from dotcache_amd.config import DotCacheConfig, PageModeSpec
    from dotcache_amd.encode import encode_page

    rng = np.random.default_rng(7)
    x = hard_values(rng, 50, 128) * 3
    cfg = DotCacheConfig(head_dim=128, group_size=32, escape_dtype=escape)
    got = encode_page(x, cfg, kind="K", mode="M3")
    want = O.encode_page(x, head_dim=128, group_size=32, bits=4, kind="K", mode="M3", escape_dtype=escape)
    _assert_same_page(got, want)


def test_encode_token_major_layout():
    from dotcache_amd.config import DotCacheConfig
    from dotcache_amd.encode import encode_page

    x = hard_values(np.random.default_rng(8), 20, 64)
    cfg = DotCacheConfig(head_dim=64, group_size=32, payload_layout_k="token_major")
    got = encode_page(x, cfg, kind="K")
    want = O.encode_page(x, head_dim=64, group_size=32, bits=4, kind="K", layout="token_major")
    _assert_same_page(got, want)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_encode_reads_half_inputs_exactly(dtype):
    torch = _torch()
    from dotcache_amd.config import DotCacheConfig, PageModeSpec
    from dotcache_amd.encode import encode_page

    x = torch.from_numpy(hard_values(np.random.default_rng(9), 64, 128)).to(getattr(torch, dtype))
    cfg = DotCacheConfig(head_dim=128, group_size=32)
    got = encode_page(x.cuda(), cfg, kind="K", page_mode=PageModeSpec("M0", 4, "affine"))
    want = O.encode_page(x.float().numpy(), head_dim=128, group_size=32, bits=4, kind="K")
    _assert_same_page(got, want)


def test_row_by_row_append_equals_whole_page_encode():
    """Per-step append of one token into a tail page (any order) produces the
    same blob as encoding the full page -- scales are per (token, group)."""
    torch = _torch()
    from dotcache_amd import _lib
    from dotcache_amd.page_pool import DevicePagePool, PoolGeometry

    rng = np.random.default_rng(10)
    x = hard_values(rng, 64, 128)
    pool = DevicePagePool(PoolGeometry(128, 32, 64), reserve_bytes=1 << 20)
    whole, rows = pool.allocate(_lib.FMT_M0_AFFINE, 4, 2, tokens=64)
    xt = torch.from_numpy(x).cuda()
    pool.encode_rows(xt, np.full(64, whole, np.int32), np.arange(64, dtype=np.int32))
    for t in rng.permutation(64):
        pool.encode_rows(xt[t: t + 1], np.array([rows], np.int32), np.array([t], np.int32))
    a = pool.download_page(int(whole), _header(128, 64))
    b = pool.download_page(int(rows), _header(128, 64))
    np.testing.assert_array_equal(a.payload, b.payload)
    np.testing.assert_array_equal(a.scales.view(np.uint16), b.scales.view(np.uint16))
    np.testing.assert_array_equal(a.bias.view(np.uint16), b.bias.view(np.uint16))
    want = O.encode_page(x, head_dim=128, group_size=32, bits=4, kind="K")
    np.testing.assert_array_equal(b.payload, want.payload)


def _header(hd, T):
    from dotcache_amd.types import PageHeader

    return PageHeader(layer_id=0, kv_head_id=0, kind="K", token_start=0, token_count=T, head_dim=hd,
                      padded_head_dim=hd, group_size=32, num_groups=hd // 32, bits=4, words_per_group=4,
                      mode_default="M0", layout="group_major", quant_scheme="affine")


def test_encode_rejects_bad_shapes():
    from dotcache_amd.config import DotCacheConfig
    from dotcache_amd.encode import encode_page

    cfg = DotCacheConfig(head_dim=64)
    with pytest.raises(ValueError):
        encode_page(np.zeros((4, 32), np.float32), cfg, kind="K")
    with pytest.raises(ValueError):
        encode_page(np.zeros((4,), np.float32), cfg, kind="K")


# ---- the wavefront encode kernel against the general one and the oracle ----

GEOMS = [  # (head_dim, group_size): the wavefront kernel's shapes and two it leaves to the general kernel
    (128, 32), (64, 32), (256, 32), (128, 64), (48, 32), (32, 16), (128, 128), (64, 8),
    (96, 32),   # padded head_dim / 8 = 12 lanes: general kernel
    (40, 20),   # group of 20 channels: general kernel
]
FMTS = [("M0", "affine", b) for b in (2, 3, 4, 8)] + [("M0", "symmetric", b) for b in (2, 3, 4, 8)] + [
    ("M3", "float16", 0), ("M3", "float32", 0), ("M3", "int8", 0)]


def _encode_all(pool, fmts, x, slots):
    """One page per format of ``fmts``; every row of x into every page at
    ``slots``; the pages downloaded."""
    from dotcache_amd.page_pool import page_format_of

    torch = _torch()
    out = []
    for mode, sch, bits in fmts:
        fmt, b = page_format_of(mode, "affine" if mode == "M3" else sch, bits or 4, sch if mode == "M3" else "float16")
        pid = int(pool.allocate(fmt, b, 1, tokens=int(slots.max()) + 1)[0])
        pool.encode_rows(x, np.full(len(slots), pid, np.int32), slots.astype(np.int32))
        out.append(pool.download_page(pid))
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("stride_pad", [0, 3])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("hd,gs", GEOMS)
def test_wavefront_encode_matches_general_kernel_and_oracle(hd, gs, dtype, stride_pad):
    """Every format, rows written to scattered slots of a 64-token page, rows
    read through a padded stride (stride_pad 3: not 16-byte aligned, the
    per-element load path): the wavefront kernel's blobs equal the general
    kernel's byte for byte and the oracle's encode of the same rows."""
    torch = _torch()
    from dotcache_amd.page_pool import DevicePagePool, PoolGeometry, set_encode_path

    rng = np.random.default_rng(hd * 100 + gs + stride_pad)
    T = 37
    x32 = hard_values(rng, T, hd)
    full = torch.zeros((T, hd + stride_pad), dtype=getattr(torch, dtype))
    full[:, :hd] = torch.from_numpy(x32).to(full.dtype)
    x = full.cuda()[:, :hd]
    xr = full[:, :hd].float().numpy()  # the values the encoder reads
    slots = rng.permutation(64)[:T]
    res = {}
    for path in ("auto", "general"):
        set_encode_path(path)
        try:
            pool = DevicePagePool(PoolGeometry(hd, gs, 64), reserve_bytes=1 << 22)
            res[path] = _encode_all(pool, FMTS, x, slots)
        finally:
            set_encode_path("auto")
    order = np.argsort(slots)
    for (mode, sch, bits), a, b in zip(FMTS, res["auto"], res["general"]):
        for name in ("payload", "scales", "bias", "escape_payload", "escape_scales"):
            u, v = getattr(a, name), getattr(b, name)
            assert (u is None) == (v is None), name
            if u is not None:
                np.testing.assert_array_equal(u.view(np.uint8), v.view(np.uint8), err_msg=f"{mode}/{sch}/{bits} {name}")
        # the oracle on the rows in slot order (slots past the rows are never read back)
        want = O.encode_page(xr[order], head_dim=hd, group_size=gs, kind="K", mode=mode,
                             scheme="affine" if mode == "M3" else sch, bits=bits or 4,
                             escape_dtype=sch if mode == "M3" else "float16")
        rows = np.sort(slots)
        if mode == "M0":
            got_codes = a.payload if a.header.layout == "group_major" else None
            np.testing.assert_array_equal(got_codes[:, rows], want.payload, err_msg=f"{mode}/{sch}/{bits} codes")
            np.testing.assert_array_equal(a.scales[rows].view(np.uint16), want.scales.view(np.uint16))
            if want.bias is not None:
                np.testing.assert_array_equal(a.bias[rows].view(np.uint16), want.bias.view(np.uint16))
        else:
            np.testing.assert_array_equal(a.escape_payload[rows].view(np.uint8), want.escape_payload.view(np.uint8))
            if want.escape_scales is not None:
                np.testing.assert_array_equal(a.escape_scales[rows].view(np.uint16), want.escape_scales.view(np.uint16))




def tie_rows(rng, T, hd, gs, fmt):
    """Rows whose codes sit on rounding ties and within a few ulps of them.
    Even rows use a power-of-two scale (s = 2^e, the group's range set by
    channels 0 and 1, so fl(range / top) = s exactly and (k + 1/2) s is an
    exact tie); odd rows a random scale, where fl(d / s) lands on or next to
    k + 1/2 as the fp32 arithmetic has it.  Every value is then left on the
    tie or moved by a few ulps: 1 or 2 (inside the wavefront kernel's
    division zone) up to 64 (outside it)."""
    mode, scheme, bits = fmt
    x = np.zeros((T, hd), np.float32)
    top = 2 ** bits - 1 if mode == "M0" else 127
    qmax = 2 ** (bits - 1) - 1 if mode == "M0" else 127
    span = gs if mode == "M0" else hd  # int8 escapes: one scale per row
    for t in range(T):
        for base in range(0, hd, span):
            n = min(span, hd - base)
            s = np.float32(2.0 ** int(rng.integers(-6, 3))) if t % 2 == 0 else np.float32(rng.uniform(0.01, 3.0))
            if mode == "M0" and scheme == "affine":
                lo = np.float32(0.0) if t % 4 == 0 else np.float32(rng.uniform(-2, 2))
                x[t, base], x[t, base + 1] = lo, np.float32(lo + np.float32(top) * s)
                vals = lo + (rng.integers(0, top, size=n - 2).astype(np.float32) + np.float32(0.5)) * s
            else:
                x[t, base], x[t, base + 1] = np.float32(qmax) * s, -np.float32(qmax) * s
                vals = (rng.integers(-qmax, qmax, size=n - 2).astype(np.float32) + np.float32(0.5)) * s
            vals = vals.astype(np.float32)
            ks = rng.choice([-64, -9, -3, -2, -1, 0, 0, 0, 1, 2, 3, 9, 64], size=n - 2).astype(np.float32)
            x[t, base + 2: base + n] = (vals + ks * np.spacing(vals)).astype(np.float32)
    return x


TIE_FMTS = [("M0", "affine", b) for b in (2, 3, 4, 8)] + [("M0", "symmetric", b) for b in (2, 3, 4, 8)] + [
    ("M3", "int8", 0)]


@pytest.mark.parametrize("fmt", TIE_FMTS, ids=lambda f: f"{f[0]}-{f[1]}-{f[2]}")
def test_encode_codes_on_and_next_to_ties(fmt):
    """Codes whose fp32 quotient d / s is a rounding tie (k + 1/2, rounded
    half to even) or a few ulps from one: the wavefront kernel (codes from
    the reciprocal of the scale, the division only near ties) and the
    general kernel (the division always) give the oracle's bytes."""
    torch = _torch()
    from dotcache_amd.page_pool import DevicePagePool, PoolGeometry, set_encode_path

    rng = np.random.default_rng(sum(map(ord, str(fmt))))
    hd, gs, T = 128, 32, 64
    x = tie_rows(rng, T, hd, gs, fmt)
    mode, sch, bits = fmt
    want = O.encode_page(x, head_dim=hd, group_size=gs, kind="K", mode=mode,
                         scheme="affine" if mode == "M3" else sch, bits=bits or 4,
                         escape_dtype=sch if mode == "M3" else "float16")
    slots = np.arange(T)
    for path in ("auto", "general"):
        set_encode_path(path)
        try:
            pool = DevicePagePool(PoolGeometry(hd, gs, 64), reserve_bytes=1 << 22)
            (got,) = _encode_all(pool, [fmt], torch.from_numpy(x).cuda(), slots)
        finally:
            set_encode_path("auto")
        if mode == "M0":
            np.testing.assert_array_equal(got.payload, want.payload, err_msg=f"{path} codes")
            np.testing.assert_array_equal(got.scales.view(np.uint16), want.scales.view(np.uint16))
        else:
            np.testing.assert_array_equal(got.escape_payload.view(np.uint8), want.escape_payload.view(np.uint8),
                                          err_msg=f"{path} int8 codes")
            np.testing.assert_array_equal(got.escape_scales.view(np.uint16), want.escape_scales.view(np.uint16))


def test_tie_rows_hit_exact_ties():
    """The tie generator's even rows put exact ties in front of the encoder:
    with the oracle's own fp32 arithmetic, many quotients are exactly k + 1/2."""
    rng = np.random.default_rng(5)
    x = tie_rows(rng, 8, 128, 32, ("M0", "affine", 4))
    ties = 0
    for t in range(0, 8, 2):  # the power-of-two rows
        for g in x[t].reshape(4, 32):
            lo, s = g.min(), np.float32((g.max() - g.min()) / np.float32(15))
            q = ((g - lo) / s).astype(np.float32)
            ties += int(np.sum(np.abs(q - np.floor(q) - 0.5) == 0))
    assert ties >= 40, ties  # about 3 / 13 of 16 x 30 values


def test_encode_rows_kv_equals_two_calls():
    """dc_encode_rows_kv (keys and values in one launch, different pools,
    value group 64) writes exactly what two dc_encode_rows calls write."""
    torch = _torch()
    from dotcache_amd import _lib
    from dotcache_amd.page_pool import DevicePagePool, PoolGeometry

    rng = np.random.default_rng(31)
    n, hd = 24, 128
    k = torch.from_numpy(hard_values(rng, n, hd)).cuda()
    v = torch.from_numpy(hard_values(rng, n, hd)).cuda()
    slots = np.tile(rng.permutation(64)[: n // 2], 2).astype(np.int32)
    pages = {}
    for tag in ("one", "two"):
        kp = DevicePagePool(PoolGeometry(hd, 32, 64), reserve_bytes=1 << 20)
        vp = DevicePagePool(PoolGeometry(hd, 64, 64), reserve_bytes=1 << 20)
        kid = np.concatenate([kp.allocate(_lib.FMT_M3_F16, 0, 1, tokens=64),
                              kp.allocate(_lib.FMT_M0_AFFINE, 4, 1, tokens=64)])
        vid = vp.allocate(_lib.FMT_M0_SYMMETRIC, 8, 2, tokens=64)
        kpage, vpage = np.repeat(kid, n // 2).astype(np.int32), np.repeat(vid, n // 2).astype(np.int32)
        if tag == "one":
            kp.encode_rows_with(vp, k, v, kpage, slots, vpage, slots)
        else:
            kp.encode_rows(k, kpage, slots)
            vp.encode_rows(v, vpage, slots)
        torch.cuda.synchronize()
        pages[tag] = [kp.download_page(int(i), kind="K") for i in kid] + [vp.download_page(int(i), kind="V") for i in vid]
    rows = np.sort(slots[: n // 2])
    for a, b in zip(pages["one"], pages["two"]):
        for name in ("payload", "scales", "bias", "escape_payload"):
            u, w = getattr(a, name), getattr(b, name)
            assert (u is None) == (w is None), name
            if u is not None:
                axis = 1 if name == "payload" else 0
                np.testing.assert_array_equal(np.take(u, rows, axis=axis).view(np.uint8),
                                              np.take(w, rows, axis=axis).view(np.uint8), err_msg=name)
