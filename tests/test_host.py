"""Host-side logic: config and page-mode parsing, headers, planner policy."""
import numpy as np
import pytest

from dotcache_amd.config import DotCacheConfig, PageModeSpec, parse_page_mode_token, recent_window_page_mode
from dotcache_amd.decode import choose_pages_per_split
from dotcache_amd.types import PageHeader, deserialize_header, serialize_header


def test_header_serialization_roundtrip():
    header = PageHeader(layer_id=1, kv_head_id=2, kind="K", token_start=64, token_count=8, head_dim=48,
                        padded_head_dim=64, group_size=32, num_groups=2, bits=4, words_per_group=4,
                        mode_default="M0", layout="group_major", quant_scheme="affine")
    assert deserialize_header(serialize_header(header)) == header


def test_config_validation_matches_reference_messages():
    with pytest.raises(ValueError, match="bits_k must be 2, 3, or 4"):
        DotCacheConfig(head_dim=64, bits_k=8)
    with pytest.raises(ValueError):
        DotCacheConfig(head_dim=0)
    c = DotCacheConfig(head_dim=48, group_size=32)
    assert c.num_groups == 2 and c.padded_head_dim == 64


def test_dotcache_config_resolves_specific_mode_overrides():
    c = DotCacheConfig(head_dim=64, key_mode_overrides=("layer:1=M3", "layer:2:kv:1=M3"))
    assert c.resolve_page_mode(kind="K", layer_id=0, kv_head_id=0) == "M0"
    assert c.resolve_page_mode(kind="K", layer_id=1, kv_head_id=3) == "M3"
    assert c.resolve_page_mode(kind="K", layer_id=2, kv_head_id=0) == "M0"
    assert c.resolve_page_mode(kind="K", layer_id=2, kv_head_id=1) == "M3"
    assert c.resolve_page_mode(kind="V", layer_id=1, kv_head_id=0) == "M0"
    with pytest.raises(ValueError):
        DotCacheConfig(head_dim=64, key_mode_overrides=("layer:x",))


def test_parse_page_mode_token():
    assert parse_page_mode_token("M0/symmetric/8") == PageModeSpec("M0", 8, "symmetric")
    assert parse_page_mode_token("m3/affine/4/int8").escape_dtype == "int8"
    with pytest.raises(ValueError):
        parse_page_mode_token("M0/affine/4/int8")
    with pytest.raises(ValueError):
        parse_page_mode_token("M0/affine")


def test_recent_window_rule():
    aged = PageModeSpec("M0", 4, "affine")
    assert recent_window_page_mode(10, 128, aged).mode == "M3"
    assert recent_window_page_mode(10, 128, aged).age_bucket == "recent"
    assert recent_window_page_mode(128, 128, aged) is aged


def test_split_policy_fills_the_chip():
    per = choose_pages_per_split(np.full(8, 256), 4)
    assert per >= 8 and 8 * 4 * (-(-256 // per)) >= 256
    assert choose_pages_per_split(np.array([1]), 1) == 1


def test_workload_key_bits_variant_is_validated_before_any_device_work():
    """``key_bits`` re-codes M0 key pages only: configurations whose keys are
    M3 rows, and widths the encoder does not have, are refused up front."""
    from dotcache_amd.workloads import build_workload

    with pytest.raises(ValueError, match="M0 key pages"):
        build_workload("c3", key_bits=8, device="cpu")
    with pytest.raises(ValueError, match="M0 key pages"):
        build_workload("c2", key_bits=5, device="cpu")
