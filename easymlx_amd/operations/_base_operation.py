"""The attention-operation plugin boundary.

Interface mirror of the reference's operation framework so that an op written
for it reads the same here:

* ``BaseOperation`` / ``OperationRegistry`` --
  ``lib/python/easymlx/operations/_base_operation.py:123-287``
* ``ExecutionMode`` / ``MetadataField`` / ``CacheType`` --
  ``lib/python/easymlx/operations/requirements/types.py:26-117``
* ``OperationRequirements`` / ``RequirementsBuilder`` --
  ``requirements/requirements.py:28-110``, ``requirements/builder.py:29-100``
* ``AttentionOutput`` -- ``lib/python/easymlx/operations/_attention_outputs.py:33-49``

Names, argument meaning and error types are kept; arrays are torch tensors on
the GPU instead of ``mx.array``.
"""

from __future__ import annotations

import typing as tp
from abc import ABC, abstractmethod
from dataclasses import dataclass
from enum import Enum, Flag, auto


class ExecutionMode(Enum):
    PREFILL = "prefill"
    DECODE = "decode"
    MIXED = "mixed"


class MetadataField(Flag):
    NONE = 0
    MASK = auto()
    SINKS = auto()
    QUERY_START_LOC = auto()
    BLOCK_TABLES = auto()
    KV_LENS = auto()
    BLOCK_SIZE = auto()
    SLIDING_WINDOW = auto()

    @classmethod
    def basic(cls) -> "MetadataField":
        return cls.MASK | cls.SINKS

    @classmethod
    def paged(cls) -> "MetadataField":
        return cls.QUERY_START_LOC | cls.BLOCK_TABLES | cls.KV_LENS | cls.BLOCK_SIZE | cls.SLIDING_WINDOW


class CacheType(Flag):
    NONE = 0
    TRANSFORMER = auto()
    PAGED = auto()
    RECURRENT = auto()
    HYBRID = auto()


@dataclass(frozen=True)
class OperationRequirements:
    name: str = ""
    required_metadata: MetadataField = MetadataField.NONE
    optional_metadata: MetadataField = MetadataField.NONE
    requires_cache: bool = False
    cache_view_cls: type | None = None

    def __or__(self, other: "OperationRequirements") -> "OperationRequirements":
        cls_ = self.cache_view_cls
        if cls_ is None:
            cls_ = other.cache_view_cls
        elif other.cache_view_cls is not None and cls_ is not other.cache_view_cls:
            cls_ = object
        return OperationRequirements(
            name="+".join(p for p in (self.name, other.name) if p),
            required_metadata=self.required_metadata | other.required_metadata,
            optional_metadata=self.optional_metadata | other.optional_metadata,
            requires_cache=self.requires_cache or other.requires_cache,
            cache_view_cls=cls_,
        )

    @classmethod
    def default(cls, name: str = "") -> "OperationRequirements":
        return cls(name=name, optional_metadata=MetadataField.basic())


@dataclass
class RequirementsBuilder:
    name: str
    _required: MetadataField = MetadataField.NONE
    _optional: MetadataField = MetadataField.NONE
    _requires_cache: bool = False
    _cache_view_cls: type | None = None

    def require_metadata(self, *fields: MetadataField) -> "RequirementsBuilder":
        for f in fields:
            self._required |= f
        return self

    def optional_metadata(self, *fields: MetadataField) -> "RequirementsBuilder":
        for f in fields:
            self._optional |= f
        return self

    def require_cache(self, cache_view_cls: type | None = None) -> "RequirementsBuilder":
        self._requires_cache = True
        self._cache_view_cls = cache_view_cls
        return self

    def build(self) -> OperationRequirements:
        return OperationRequirements(
            name=self.name,
            required_metadata=self._required,
            optional_metadata=self._optional,
            requires_cache=self._requires_cache,
            cache_view_cls=self._cache_view_cls,
        )


@dataclass
class AttentionOutput:
    attention_outputs: tp.Any = None
    attention_weights: tp.Any = None
    cache_view: tp.Any = None


class BaseOperation(ABC):
    """Abstract attention operation (``_base_operation.py:123-214``)."""

    metadata: tp.Any = None

    def __init__(self, metadata: tp.Any = None):
        self.metadata = metadata

    @classmethod
    @abstractmethod
    def get_impl_name(cls) -> str | tuple[str, ...]: ...

    @classmethod
    def get_requirements(cls, mode: ExecutionMode = ExecutionMode.MIXED) -> OperationRequirements:
        name = cls.get_impl_name()
        if isinstance(name, tuple):
            name = name[0]
        return OperationRequirements.default(str(name))

    def get_instance_requirements(self, mode: ExecutionMode = ExecutionMode.MIXED) -> OperationRequirements:
        return self.get_requirements(mode)

    @abstractmethod
    def forward_native(self, *args, **kwargs) -> tp.Any: ...

    def __call__(self, *args, **kwargs) -> tp.Any:
        return self.forward_native(*args, **kwargs)


class OperationRegistry:
    """Global name -> operation-class registry (``_base_operation.py:217-287``)."""

    _registry: tp.ClassVar[dict[str, type[BaseOperation]]] = {}

    @classmethod
    def register(cls, operation_cls: type[BaseOperation]) -> type[BaseOperation]:
        names = operation_cls.get_impl_name()
        if isinstance(names, str):
            names = (names,)
        for name in names:
            cls._registry[str(name)] = operation_cls
        return operation_cls

    @classmethod
    def get(cls, name: str) -> type[BaseOperation]:
        try:
            return cls._registry[name]
        except KeyError as exc:
            available = ", ".join(sorted(cls._registry))
            raise KeyError(f"Unknown operation '{name}'. Available: {available}") from exc

    @classmethod
    def create(cls, name: str, *, metadata: tp.Any = None) -> BaseOperation:
        return cls.get(name)(metadata=metadata)

    @classmethod
    def available_impls(cls) -> list[str]:
        return sorted(cls._registry)


Operation = BaseOperation
