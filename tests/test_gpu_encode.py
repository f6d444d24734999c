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
