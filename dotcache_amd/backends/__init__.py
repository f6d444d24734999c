"""Backend registry of this package: the ``hip_mi355x`` function set
(reference ``dotcache/backends/__init__.py:1-102`` re-exports the
``cpu_ref`` / ``torch_cuda`` / ``torch_mps`` sets the same way)."""
from .hip_mi355x import (
    PreparedPageHIP,
    clear_prepared_pools,
    decode_grouped_multiquery_step_hip_tensor,
    decode_grouped_multiquery_step_prepared_hip_tensor,
    decode_grouped_multiquery_step_prepared_hip_tensor_output_only,
    decode_multi_query_step_hip,
    decode_multi_query_step_hip_tensor,
    decode_step_hip,
    hip_available,
    mix_page_hip,
    page_supported_hip,
    pool_for,
    prepare_page_hip,
    prepare_pages_hip,
    score_page_hip,
    score_pages_hip,
)

__all__ = [
    "PreparedPageHIP",
    "clear_prepared_pools",
    "decode_grouped_multiquery_step_hip_tensor",
    "decode_grouped_multiquery_step_prepared_hip_tensor",
    "decode_grouped_multiquery_step_prepared_hip_tensor_output_only",
    "decode_multi_query_step_hip",
    "decode_multi_query_step_hip_tensor",
    "decode_step_hip",
    "hip_available",
    "mix_page_hip",
    "page_supported_hip",
    "pool_for",
    "prepare_page_hip",
    "prepare_pages_hip",
    "score_page_hip",
    "score_pages_hip",
]
