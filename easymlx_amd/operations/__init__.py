"""Attention operations (plugin boundary + the paged attention op)."""

from ._base_operation import (
    AttentionOutput,
    BaseOperation,
    CacheType,
    ExecutionMode,
    MetadataField,
    Operation,
    OperationRegistry,
    OperationRequirements,
    RequirementsBuilder,
)
from .unified_attention import UnifiedAttention, UnifiedAttnMetadata, paged_attention

__all__ = (
    "AttentionOutput",
    "BaseOperation",
    "CacheType",
    "ExecutionMode",
    "MetadataField",
    "Operation",
    "OperationRegistry",
    "OperationRequirements",
    "RequirementsBuilder",
    "UnifiedAttention",
    "UnifiedAttnMetadata",
    "paged_attention",
)
