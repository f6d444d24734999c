"""Host-side checks of the device KV cache that run before any device work:
argument validation and the token-index contract of ``append_step``
(reference ``model_kv_cache.py:3873-3876``)."""
import numpy as np
import pytest

from dotcache_amd.config import DotCacheConfig
from dotcache_amd.kv_cache import DevicePagedKVCache, default_q_head_to_kv_head


def _cache(**kw):
    cfg = DotCacheConfig(head_dim=64, group_size=32, tokens_per_page=16)
    args = dict(num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2, batch_size=1, device="cpu")
    args.update(kw)
    return DevicePagedKVCache(cfg, **args)


def test_default_head_map_is_the_reference_grouping():
    np.testing.assert_array_equal(default_q_head_to_kv_head(8, 2), [0, 0, 0, 0, 1, 1, 1, 1])
    with pytest.raises(ValueError):
        default_q_head_to_kv_head(6, 4)


def test_constructor_rejects_bad_head_counts():
    with pytest.raises(ValueError):
        _cache(num_attention_heads=6, num_key_value_heads=4)
    with pytest.raises(ValueError):
        _cache(num_attention_heads=34, num_key_value_heads=2)  # more than 16 query heads per KV head
    with pytest.raises(ValueError):
        _cache(batch_size=0)


def test_append_rejects_a_token_index_that_is_not_the_cached_length():
    c = _cache()
    rows = np.zeros((2, 1, 64), np.float32)
    with pytest.raises(ValueError, match="expected token_index 0"):
        c.append_step(0, rows, rows, 5)


def test_shapes_and_layers_are_checked():
    c = _cache()
    with pytest.raises(ValueError):
        c.append_step(0, np.zeros((3, 1, 64), np.float32), np.zeros((3, 1, 64), np.float32), 0)  # 3 KV heads
    with pytest.raises(ValueError):
        c.append_step(0, np.zeros((2, 1, 64), np.float32), np.zeros((2, 2, 64), np.float32), 0)  # token counts differ
    with pytest.raises(ValueError):
        c.ingest_prefill_cache(2, np.zeros((2, 4, 64), np.float32), np.zeros((2, 4, 64), np.float32))
    with pytest.raises(ValueError, match="no cached tokens"):
        c.decode_layer(1, np.zeros((4, 64), np.float32))
    with pytest.raises(ValueError):
        c.ingest_prefill_cache(0, np.zeros((2, 4, 64), np.float32), np.zeros((2, 4, 64), np.float32), context_length=3)


def test_block_cache_checks_before_device_work():
    from dotcache_amd.block_cache import DeviceVllmPagedKVCache

    cfg = DotCacheConfig(head_dim=32, group_size=32, tokens_per_page=4)
    with pytest.raises(ValueError, match="block_size"):
        DeviceVllmPagedKVCache(config=cfg, num_hidden_layers=1, num_attention_heads=4, num_key_value_heads=2,
                               block_size=8, device="cpu")
    c = DeviceVllmPagedKVCache(config=cfg, num_hidden_layers=1, num_attention_heads=4, num_key_value_heads=2,
                               block_size=4, device="cpu")
    rows = np.zeros((1, 2, 32), np.float32)
    with pytest.raises(ValueError, match="out of order"):
        c.write_slots(0, rows, rows, [7 * 4 + 2])  # offset 2 of an empty block
    with pytest.raises(ValueError):
        c.write_slots(0, rows, rows, [0, 1])  # one slot per row
    with pytest.raises(ValueError, match="unique"):
        c.sync_layer_blocks(0, np.zeros((2, 2, 4, 32)), np.zeros((2, 2, 4, 32)), block_ids=[3, 3])
    with pytest.raises(ValueError, match="no cached tokens"):
        c.decode_layer(0, np.zeros((4, 32), np.float32))
    with pytest.raises(ValueError, match="expected token_index 0"):
        c.append_step(0, np.zeros((2, 1, 32)), np.zeros((2, 1, 32)), 4)
