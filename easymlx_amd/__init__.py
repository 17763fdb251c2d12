"""easymlx_amd -- MI355X-native eSurge attention hot path.

Paged / unified attention over affine-quantized (int4 / int8) and FP8 (E4M3)
KV pages and the fused quantize-on-write that fills them, as hand-written HIP kernels for gfx950
behind a C ABI (``include/emx_attn.h``), exposed through the reference's
attention-operation plugin interface.
"""

from .caching.paged import AffinePageCacheView, Fp8PageCacheView, PageCacheView, PageMetadata, build_query_start_loc
from .caching.compiled import CompiledPagedCacheProxy
from .caching.pagecache import PageCache, PageCacheConfig, validate_cache_dtype
from .caching.rope import RotaryEmbedding
from .operations import AttentionOutput, BaseOperation, OperationRegistry, UnifiedAttention, paged_attention
from .quantize import affine_quantize

__all__ = (
    "AffinePageCacheView",
    "AttentionOutput",
    "BaseOperation",
    "CompiledPagedCacheProxy",
    "Fp8PageCacheView",
    "OperationRegistry",
    "PageCache",
    "PageCacheConfig",
    "PageCacheView",
    "PageMetadata",
    "RotaryEmbedding",
    "UnifiedAttention",
    "affine_quantize",
    "build_query_start_loc",
    "paged_attention",
    "validate_cache_dtype",
)
