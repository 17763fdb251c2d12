"""Paged KV caches (dense and affine-quantized)."""

from .paged import AffinePageCacheView, PageCacheView, PageMetadata, affine_pool, build_query_start_loc

__all__ = ("AffinePageCacheView", "PageCacheView", "PageMetadata", "affine_pool", "build_query_start_loc")
