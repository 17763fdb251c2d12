"""Paged KV caches (dense, FP8 E4M3 and affine-quantized)."""

from .rope import RotaryEmbedding
from .compiled import CompiledPagedCacheProxy
from .pagecache import CacheConfigError, PageCache, PageCacheConfig, validate_cache_dtype
from .paged import AffinePageCacheView, Fp8PageCacheView, PageCacheView, PageMetadata, affine_pool, build_query_start_loc

__all__ = ("AffinePageCacheView", "CacheConfigError", "CompiledPagedCacheProxy", "PageCache", "PageCacheConfig",
           "validate_cache_dtype", "Fp8PageCacheView", "PageCacheView", "PageMetadata", "affine_pool", "build_query_start_loc", "RotaryEmbedding")
