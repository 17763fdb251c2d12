"""Multi-layer paged cache configuration and container.

Mirrors ``PageCacheConfig`` / ``PageCache`` (``lib/python/easymlx/caching/paged/cache.py:1309-1445``)
and the ``cache_dtype`` validation of the model config
(``lib/python/easymlx/infra/base_config.py:132-138``), with this build's affine
KV modes added: ``"affine4"`` / ``"affine8"`` (int4 / int8 codes with a per-
(token, group) fp16 scale and bias, quantized on write).
"""

from __future__ import annotations

import math
import typing as tp

import torch

from .paged import PageCacheView, block_mapping_on_device

# The reference's accepted storage modes (base_config.py:132) plus the affine modes.
VALID_CACHE_DTYPES = ("auto", "float16", "bfloat16", "float32", "fp8", "affine4", "affine8")


class CacheConfigError(ValueError):
    """An unsupported cache configuration (the reference raises ``EasyMLXConfigError``)."""


def validate_cache_dtype(cache_dtype: str | None, cache_bits: int | None = None) -> None:
    """``base_config.py:132-138`` with the affine modes: raise :class:`CacheConfigError` for anything else.

    TurboQuant (``"turboquant*"``) is a valid mode of the reference that this build does not implement: it is
    refused with a message that says so."""
    if cache_dtype is None:
        return
    name = str(cache_dtype).lower()
    if name.startswith("turboquant"):
        raise CacheConfigError(f"cache_dtype={cache_dtype!r}: TurboQuant caches are not part of this build")
    if name not in VALID_CACHE_DTYPES:
        raise CacheConfigError(f"Unsupported cache_dtype={cache_dtype!r}; supported: {VALID_CACHE_DTYPES}")
    if cache_bits is not None and name in ("affine4", "affine8") and int(cache_bits) != int(name[-1]):
        raise CacheConfigError(f"cache_bits={cache_bits} contradicts cache_dtype={cache_dtype!r}")


def resolve_cache_dtype(cache_dtype: str | None, cache_bits: int | None = None) -> tuple[str, int | None]:
    """``(kind, bits)``: kind ``"float"`` (store the view's dtype), ``"fp8"`` or ``"affine"`` (bits 4 / 8)."""
    validate_cache_dtype(cache_dtype, cache_bits)
    name = str(cache_dtype or "auto").lower()
    if name == "fp8":
        return "fp8", None
    if name in ("affine4", "affine8"):
        return "affine", int(name[-1])
    return "float", None


class PageCacheConfig:
    """Static configuration of a paged KV cache (``cache.py:1309-1376``).

    Same fields as the reference; ``cache_dtype`` also takes ``"affine4"`` /
    ``"affine8"``, and ``cache_group_size`` sets the affine quantization group.
    """

    __slots__ = ("cache_bits", "cache_dtype", "cache_group_size", "device", "dtype", "head_dim", "max_model_length",
                 "max_num_reqs", "memory_utilization", "num_hidden_layers", "num_kv_heads", "page_size")

    def __init__(
        self,
        *,
        num_hidden_layers: int,
        num_kv_heads: int,
        head_dim: int,
        page_size: int = 16,
        max_num_reqs: int = 4,
        max_model_length: int = 4096,
        memory_utilization: float = 0.85,
        dtype: torch.dtype | str = torch.float16,
        cache_dtype: str | None = None,
        cache_bits: int | None = None,
        cache_group_size: int = 64,
        device: tp.Any = "cuda",
    ) -> None:
        validate_cache_dtype(cache_dtype, cache_bits)
        self.num_hidden_layers = int(num_hidden_layers)
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = int(head_dim)
        self.page_size = int(page_size)
        self.max_num_reqs = int(max_num_reqs)
        self.max_model_length = int(max_model_length)
        self.memory_utilization = float(memory_utilization)
        self.dtype = dtype
        self.cache_dtype = cache_dtype
        self.cache_bits = int(cache_bits) if cache_bits is not None else None
        self.cache_group_size = int(cache_group_size)
        self.device = device

    @property
    def num_pages(self) -> int:
        """Total pages: ``ceil(max_model_length / page_size) * max_num_reqs`` (``cache.py:1358-1362``)."""
        return math.ceil(self.max_model_length / self.page_size) * self.max_num_reqs

    @classmethod
    def create(cls, **kwargs) -> "PageCacheConfig":
        """Factory matching ``BaseCacheConfig.create`` (``cache.py:1364-1367``)."""
        return cls(**kwargs)


class PageCache:
    """Per-layer :class:`PageCacheView` container (``cache.py:1370-1445``)."""

    __slots__ = ("config", "views")

    def __init__(self, views: list[PageCacheView], config: PageCacheConfig | None = None) -> None:
        self.views = views
        self.config = config

    def __getitem__(self, index: int) -> PageCacheView:
        return self.views[index]

    def __setitem__(self, index: int, view: PageCacheView) -> None:
        self.views[index] = view

    def __len__(self) -> int:
        return len(self.views)

    def __iter__(self):
        return iter(self.views)

    @classmethod
    def init_cache(cls, config: PageCacheConfig) -> "PageCache":
        """One zero-initialised view per layer from the shared config (``cache.py:1404-1427``)."""
        views = [
            PageCacheView.init(
                num_seqs=config.max_num_reqs,
                max_seq_len=config.max_model_length,
                num_kv_heads=config.num_kv_heads,
                head_dim=config.head_dim,
                block_size=config.page_size,
                dtype=config.dtype,
                cache_dtype=config.cache_dtype,
                cache_bits=config.cache_bits,
                group_size=config.cache_group_size,
                device=config.device,
            )
            for _ in range(config.num_hidden_layers)
        ]
        return cls(views=views, config=config)

    def clear(self) -> None:
        """Zero every layer (``cache.py:1429-1432``)."""
        for view in self.views:
            view.clear()

    def copy_blocks(self, block_mapping) -> None:
        """Copy-on-write block copies in every layer (``cache.py:1434-1445``); checked once, one device copy."""
        if not self.views:
            return
        mapping = block_mapping_on_device(block_mapping, self.views[0].key_cache.device)
        for view in self.views:
            view.copy_blocks(mapping)

    def zero_pages(self, page_ids) -> None:
        """The runner's ``_zero_pages`` over every layer (``model_runner.py:1058-1094``)."""
        ids = page_ids
        if self.views and not isinstance(ids, torch.Tensor):
            ids = torch.as_tensor(list(ids), dtype=torch.int32).to(self.views[0].key_cache.device)
        for view in self.views:
            view.zero_pages(ids)


__all__ = ("CacheConfigError", "PageCache", "PageCacheConfig", "VALID_CACHE_DTYPES", "resolve_cache_dtype",
           "validate_cache_dtype")
