"""MI355X-native DotCache decode-attention backend.

Attention runs directly on compressed KV pages (M0 affine / symmetric
grouped INT2-8 pages, M3 fp16 / fp32 / int8 escape pages) with hand-written
gfx950 HIP kernels behind the reference's backend surface.  The native
library is ``libdotcache_hip.so`` (C ABI in ``include/dotcache_hip.h``),
built by ``python -m dotcache_amd._build``.
"""
from .config import DotCacheConfig, PageModeSpec, parse_page_mode_token
from .types import EncodedPage, PageHeader

__all__ = ["DotCacheConfig", "EncodedPage", "PageHeader", "PageModeSpec", "parse_page_mode_token"]
__version__ = "0.1.0"
