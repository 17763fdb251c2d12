"""Paged (unified) attention over block-tabled KV caches on MI355X.

Drop-in counterpart of the reference's default attention operation:

* ``paged_attention(...)`` -- ``lib/python/easymlx/operations/kernels/unified_attention.py:1377-1512``
  (same positional arguments and keyword meaning).  An FP8 (E4M3) cache takes
  the reference's per-page ``k_scale/v_scale``; affine pages take
  ``k_scales/k_biases/v_scales/v_biases`` with ``bits`` and ``group_size``.
* ``UnifiedAttention`` -- ``unified_attention.py:1515-1684``, registered under
  the same names, with ``forward_native(query=, key=, value=, cache_metadata=,
  cache_view=, scale=, ...) -> AttentionOutput``.

All compute runs in ``libemx_attn.so`` (hand-written HIP for gfx950).  There is
no CPU / NumPy fallback: a kernel failure raises (the reference falls back
silently, ``unified_attention.py:1499-1512``).
"""

from __future__ import annotations

import math
import threading
import typing as tp
from dataclasses import dataclass

import torch

from .. import _native
from ..caching.paged import AffinePageCacheView, Fp8PageCacheView, PageCacheView, PageMetadata
from ._base_operation import (
    AttentionOutput,
    BaseOperation,
    ExecutionMode,
    MetadataField,
    OperationRegistry,
    RequirementsBuilder,
)

_DTYPE_CODE = {torch.float16: _native.DTYPE_F16, torch.bfloat16: _native.DTYPE_BF16, torch.float32: _native.DTYPE_F32}


@dataclass
class UnifiedAttnMetadata:
    """``unified_attention.py:44-66``."""

    block_tables: tp.Any
    kv_lens: tp.Any
    query_start_loc: tp.Any
    block_size: int
    sliding_window: int | None = None
    is_single_token_decode: bool = False


def _validate_inputs(queries, key_cache, value_cache, block_tables, kv_lens, query_start_loc, affine) -> None:
    """Shape checks with the reference's messages (``unified_attention.py:85-121``)."""
    if queries.ndim != 3:
        raise ValueError("queries must be rank-3: [total_tokens, num_q_heads, head_dim]")
    if not affine and (key_cache.ndim != 4 or value_cache.ndim != 4):
        raise ValueError("key_cache/value_cache must be rank-4: [num_blocks, block_size, num_kv_heads, head_dim]")
    if affine and (key_cache.ndim != 4 or value_cache.ndim != 5):
        raise ValueError("affine pages must be key codes [num_blocks, num_kv_heads, block_size, W] and value codes "
                         "[num_blocks, num_kv_heads, block_size/T, head_dim, T*bits/32]")
    if not affine:
        if key_cache.shape != value_cache.shape:
            raise ValueError("key_cache and value_cache must have the same shape")
        if queries.shape[2] != key_cache.shape[3]:
            raise ValueError("queries head_dim must match key/value cache head_dim")
        if queries.shape[1] % key_cache.shape[2] != 0:
            raise ValueError("num_q_heads must be divisible by num_kv_heads (GQA)")
    else:
        if key_cache.shape[0] != value_cache.shape[0] or key_cache.shape[1] != value_cache.shape[1]:
            raise ValueError("key_cache and value_cache must have the same [num_blocks, num_kv_heads]")
        if value_cache.shape[3] != queries.shape[2]:
            raise ValueError("queries head_dim must match key/value cache head_dim")
        if queries.shape[1] % key_cache.shape[1] != 0:
            raise ValueError("num_q_heads must be divisible by num_kv_heads (GQA)")
    if block_tables.ndim != 2:
        raise ValueError("block_tables must be rank-2: [num_seqs, max_blocks_per_seq]")
    if kv_lens.ndim != 1 or query_start_loc.ndim != 1:
        raise ValueError("kv_lens/query_start_loc must be rank-1")
    if query_start_loc.shape[0] != block_tables.shape[0] + 1:
        raise ValueError("query_start_loc must have length num_seqs + 1")


def _is_single_token_decode(query_start_loc: torch.Tensor, total_tokens: int) -> bool:
    """``unified_attention.py:175-184``.  Reads ``query_start_loc`` on the host only when its length allows a
    pure decode batch (one token per sequence needs ``num_seqs == total_tokens``): the shape decides the rest
    without a device synchronisation."""
    if total_tokens <= 0 or query_start_loc.ndim != 1 or query_start_loc.shape[0] != total_tokens + 1:
        return False
    qsl = query_start_loc.detach().to("cpu", torch.int64)
    if qsl.ndim != 1 or qsl.shape[0] != total_tokens + 1 or int(qsl[0]) != 0:
        return False
    return bool(torch.all(qsl[1:] - qsl[:-1] == 1))


_ws_lock = threading.Lock()
_ws_cache: dict[tuple[int, int], torch.Tensor] = {}


def _workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor | None:
    """Split-K workspace shared by the launches of one stream (grow-only).

    Launches on one stream are serialised, so one buffer per (device, stream)
    is race-free.  It is zero-filled when allocated: the library keeps its
    arrival counters zero between calls.
    """
    if nbytes == 0:
        return None
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    with _ws_lock:
        ws = _ws_cache.get(key)
        if ws is None or ws.numel() < nbytes:
            if ws is not None:
                torch.cuda.current_stream(device).synchronize()  # the old buffer may still be in use
            ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
            _ws_cache[key] = ws
        return ws


def _i32(t, device) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        t = torch.as_tensor(t)
    if t.dtype == torch.int32 and t.device == device and t.is_contiguous():
        return t  # the common case: the cache's own device tables (no conversion call)
    return t.to(device=device, dtype=torch.int32).contiguous()


def paged_attention(
    queries: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables,
    kv_lens,
    query_start_loc,
    *,
    softmax_scale: float | None = None,
    sliding_window: int | None = None,
    single_token_decode: bool | None = None,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
    k_scales: torch.Tensor | None = None,
    k_biases: torch.Tensor | None = None,
    v_scales: torch.Tensor | None = None,
    v_biases: torch.Tensor | None = None,
    bits: int | None = None,
    group_size: int | None = None,
    workspace: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Execute paged attention over block-tabled KV caches.

    Dense caches use the reference layout ``[num_blocks, block_size, Hkv, D]``; affine caches may also come in
    the reference's logical layout (``mlx.core.quantize`` of that dense cache: codes ``[nb, bs, Hkv, W]``,
    scales / biases ``[nb, bs, Hkv, D/group_size]``), converted to pages for the call;
    an FP8 (E4M3) cache is that layout in ``uint8`` with per-page fp32 scales
    ``k_scale/v_scale [num_blocks]`` (``unified_attention.py:1431``).
    Affine caches (``k_scales`` given) use the page layout of
    :class:`~easymlx_amd.caching.paged.AffinePageCacheView`:
    ``key_cache [nb, Hkv, bs, D*bits/32]``, ``value_cache [nb, Hkv, bs/T, D, T*bits/32]``
    (``T = min(bs, 256/bits)``),
    scales/biases ``[nb, Hkv, D/group_size, bs]``.

    Returns ``[total_tokens, num_q_heads, head_dim]`` in the queries' dtype.
    """
    affine = k_scales is not None
    if affine and (k_biases is None or v_scales is None or v_biases is None or bits is None or group_size is None):
        raise ValueError("affine caches need k_scales, k_biases, v_scales, v_biases, bits and group_size")
    dev = queries.device
    if affine and key_cache.ndim == 4 and value_cache.ndim == 4:
        # the reference's layout: mlx.core.quantize of its dense [num_blocks, block_size, Hkv, D] caches,
        # codes [nb, bs, Hkv, W] and scales / biases [nb, bs, Hkv, D/group_size].  Converted to pages for
        # this call, on the device (a whole-pool pass: a caller that keeps the cache converts it once,
        # AffinePageCacheView.from_logical, and passes the pages)
        from ..caching.paged import pages_from_logical

        if key_cache.device.type != "cuda":
            raise RuntimeError("paged_attention runs on the GPU only; the cache is on " + str(key_cache.device))
        key_cache, value_cache, k_scales, k_biases, v_scales, v_biases = pages_from_logical(
            key_cache, k_scales, k_biases, value_cache, v_scales, v_biases, bits, group_size)
    block_tables = _i32(block_tables, dev)
    kv_lens = _i32(kv_lens, dev)
    query_start_loc = _i32(query_start_loc, dev)
    _validate_inputs(queries, key_cache, value_cache, block_tables, kv_lens, query_start_loc, affine)

    total, hq, d = (int(x) for x in queries.shape)
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(d)
    if sliding_window is None:
        sliding_window = 0
    if out is None:
        out = torch.empty_like(queries)
    if total == 0:
        return out.zero_()
    if single_token_decode is None:
        single_token_decode = _is_single_token_decode(query_start_loc, total)
    if dev.type != "cuda":
        raise RuntimeError("paged_attention runs on the GPU only; queries are on " + str(dev))
    queries = queries.contiguous()
    lib = _native.load()
    stream = _native.stream_ptr(dev)
    S, max_blocks = int(block_tables.shape[0]), int(block_tables.shape[1])

    if affine:
        if queries.dtype != torch.float16:
            raise NotImplementedError("affine paged attention takes fp16 queries")
        nb, hkv, bs = int(key_cache.shape[0]), int(key_cache.shape[1]), int(key_cache.shape[2])
        need = int(lib.emx_paged_workspace_bytes(S, hq, hkv, d, max_blocks, bs))
        if need and not single_token_decode:  # room for the prefill key split
            need += int(lib.emx_paged_prefill_workspace_bytes(total, S, hq, hkv, d))
        if need and workspace is None:
            workspace = _workspace(dev, stream, need)
        ws_ptr = workspace.data_ptr() if workspace is not None else None
        ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
        tensors = [key_cache, value_cache, k_scales, k_biases, v_scales, v_biases]
        if any(not t.is_contiguous() for t in tensors):
            raise ValueError("affine cache tensors must be contiguous")
        _native.check(
            lib.emx_paged_attention_affine(
                queries.data_ptr(), total, hq, d,
                key_cache.data_ptr(), k_scales.data_ptr(), k_biases.data_ptr(),
                value_cache.data_ptr(), v_scales.data_ptr(), v_biases.data_ptr(),
                nb, bs, hkv, int(bits), int(group_size),
                block_tables.data_ptr(), S, max_blocks, kv_lens.data_ptr(), query_start_loc.data_ptr(),
                float(softmax_scale), int(sliding_window), int(bool(single_token_decode)),
                ws_ptr, ws_bytes, out.data_ptr(), stream,
            )
        )
        return out

    if queries.dtype not in _DTYPE_CODE:
        raise NotImplementedError(f"unsupported dtype {queries.dtype}")
    fp8 = key_cache.dtype == torch.uint8 and k_scale is not None and v_scale is not None
    if fp8:
        if value_cache.dtype != torch.uint8:
            raise ValueError("an FP8 cache needs uint8 key and value caches")
        key_cache = key_cache.contiguous()
        value_cache = value_cache.contiguous()
        nb, bs, hkv = int(key_cache.shape[0]), int(key_cache.shape[1]), int(key_cache.shape[2])
        k_scale = k_scale.to(device=dev, dtype=torch.float32).contiguous()
        v_scale = v_scale.to(device=dev, dtype=torch.float32).contiguous()
        if k_scale.numel() != nb or v_scale.numel() != nb:
            raise ValueError("k_scale/v_scale must hold one scale per block: [num_blocks]")
        need = int(lib.emx_paged_workspace_bytes(S, hq, hkv, d, max_blocks, bs))
        if need and not single_token_decode:  # room for the prefill key split
            need += int(lib.emx_paged_prefill_workspace_bytes(total, S, hq, hkv, d))
        if need and workspace is None:
            workspace = _workspace(dev, stream, need)
        ws_ptr = workspace.data_ptr() if workspace is not None else None
        ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
        _native.check(
            lib.emx_paged_attention_fp8(
                queries.data_ptr(), total, hq, d, _DTYPE_CODE[queries.dtype],
                key_cache.data_ptr(), value_cache.data_ptr(), k_scale.data_ptr(), v_scale.data_ptr(),
                nb, bs, hkv, block_tables.data_ptr(), S, max_blocks, kv_lens.data_ptr(), query_start_loc.data_ptr(),
                float(softmax_scale), int(sliding_window), int(bool(single_token_decode)),
                ws_ptr, ws_bytes, out.data_ptr(), stream,
            )
        )
        return out
    if key_cache.dtype != queries.dtype or value_cache.dtype != queries.dtype:
        raise NotImplementedError("dense paged attention needs the cache in the queries' dtype")
    if queries.dtype not in _DTYPE_CODE:
        raise NotImplementedError(f"unsupported dtype {queries.dtype}")
    key_cache = key_cache.contiguous()
    value_cache = value_cache.contiguous()
    nb, bs, hkv = int(key_cache.shape[0]), int(key_cache.shape[1]), int(key_cache.shape[2])
    need = int(lib.emx_paged_workspace_bytes(S, hq, hkv, d, max_blocks, bs)) if single_token_decode else 0
    if need and workspace is None:
        workspace = _workspace(dev, stream, need)
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _native.check(
        lib.emx_paged_attention_dense(
            queries.data_ptr(), total, hq, d, _DTYPE_CODE[queries.dtype],
            key_cache.data_ptr(), value_cache.data_ptr(), nb, bs, hkv,
            block_tables.data_ptr(), S, max_blocks, kv_lens.data_ptr(), query_start_loc.data_ptr(),
            float(softmax_scale), int(sliding_window), int(bool(single_token_decode)),
            ws_ptr, ws_bytes, out.data_ptr(), stream,
        )
    )
    return out


@OperationRegistry.register
class UnifiedAttention(BaseOperation):
    """Paged (unified) attention operation (``unified_attention.py:1515-1684``)."""

    def __init__(self, metadata: tp.Any | None = None):
        super().__init__(metadata=metadata)

    @classmethod
    def get_impl_name(cls) -> str | tuple[str, ...]:
        return ("unified_attention", "unified", "paged", "full_attention", "linear_attention")

    @classmethod
    def get_requirements(cls, mode: ExecutionMode = ExecutionMode.MIXED):
        return (
            RequirementsBuilder("unified_attention")
            .require_metadata(
                MetadataField.QUERY_START_LOC,
                MetadataField.BLOCK_TABLES,
                MetadataField.KV_LENS,
                MetadataField.BLOCK_SIZE,
            )
            .optional_metadata(MetadataField.SLIDING_WINDOW)
            .require_cache(PageCacheView)
            .build()
        )

    def forward_native(
        self,
        *,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        cache_metadata: UnifiedAttnMetadata | PageMetadata | None = None,
        cache_view: PageCacheView | None = None,
        scale: float | None = None,
        **_: tp.Any,
    ) -> AttentionOutput:
        if cache_metadata is None:
            raise ValueError("UnifiedAttention requires cache_metadata.")
        if isinstance(cache_metadata, PageMetadata):
            if cache_metadata.block_tables is None or cache_metadata.kv_lens is None or cache_metadata.block_size is None:
                raise ValueError("PageMetadata must be resolved before unified attention execution.")
        kwargs: dict[str, tp.Any] = {
            "softmax_scale": scale,
            "sliding_window": cache_metadata.sliding_window,
            "single_token_decode": bool(cache_metadata.is_single_token_decode),
        }
        if cache_view is not None and getattr(cache_view, "is_affine", False):
            kwargs.update(
                k_scales=cache_view.k_scales,
                k_biases=cache_view.k_biases,
                v_scales=cache_view.v_scales,
                v_biases=cache_view.v_biases,
                bits=cache_view.bits,
                group_size=cache_view.group_size,
            )
        elif cache_view is not None and getattr(cache_view, "cache_dtype_is_fp8", False) and key.dtype == torch.uint8:
            # unified_attention.py:1633-1656: the view's per-page scales
            kwargs.update(k_scale=cache_view.k_scales, v_scale=cache_view.v_scales)
        elif key.dtype == torch.int32:
            raise ValueError("affine KV pages require an AffinePageCacheView as cache_view")
        elif key.dtype == torch.uint8:
            raise ValueError("an FP8 cache requires a cache_view with per-page k_scales/v_scales")
        outputs = paged_attention(
            query,
            key,
            value,
            cache_metadata.block_tables,
            cache_metadata.kv_lens,
            cache_metadata.query_start_loc,
            **kwargs,
        )
        return AttentionOutput(attention_outputs=outputs, cache_view=cache_view)


__all__ = ("UnifiedAttention", "UnifiedAttnMetadata", "paged_attention")
