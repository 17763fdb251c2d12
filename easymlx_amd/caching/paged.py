"""Paged KV cache views on the GPU (torch tensors, HIP write kernels).

Mirrors the write-side contract of the reference's ``PageCacheView``
(``lib/python/easymlx/caching/paged/cache.py:499-1306``) and its metadata
(``PageMetadata`` ``:1468-1543``, ``build_query_start_loc`` ``:1448-1465``):

* ``PageCacheView`` -- unquantized cache in the reference layout
  ``[num_blocks, block_size, Hkv, D]``.
* ``AffinePageCacheView`` -- int4/int8 affine pages (codes + per-(token, group)
  fp16 scale and bias), written by the fused quantize-on-write kernel.

``concatenate_to_cache`` keeps the reference's signature and return value
``(queries, key_cache, value_cache, resolved_metadata)``.  Block tables and
``kv_lens`` live on the device; the slot arithmetic of a write is one kernel
(``emx_cache_slots``) that also advances ``kv_lens``, so a write never reads
device data back to the host.
"""

from __future__ import annotations

import math
import typing as tp
from dataclasses import dataclass

import torch

from .. import _native


@dataclass
class PageMetadata:
    """Kernel-agnostic paged-attention metadata (``cache.py:1468-1543``)."""

    query_start_loc: tp.Any
    block_tables: tp.Any = None
    kv_lens: tp.Any = None
    block_size: int | None = None
    sliding_window: int | None = None
    is_single_token_decode: bool = False
    slot_ids: tuple[int, ...] | None = None

    def with_cache_state(self, *, block_tables, kv_lens, block_size: int) -> "PageMetadata":
        return PageMetadata(
            query_start_loc=self.query_start_loc,
            block_tables=block_tables,
            kv_lens=kv_lens,
            block_size=int(block_size),
            sliding_window=self.sliding_window,
            is_single_token_decode=self.is_single_token_decode,
            slot_ids=self.slot_ids,
        )

    def with_sliding_window(self, sliding_window: int | None) -> "PageMetadata":
        return PageMetadata(
            query_start_loc=self.query_start_loc,
            block_tables=self.block_tables,
            kv_lens=self.kv_lens,
            block_size=self.block_size,
            sliding_window=sliding_window,
            is_single_token_decode=self.is_single_token_decode,
            slot_ids=self.slot_ids,
        )


def build_query_start_loc(query_lens: tp.Iterable[int], device=None) -> torch.Tensor:
    """Cumulative query start offsets starting at zero, int32 (``cache.py:1448-1465``)."""
    offsets = [0]
    for n in query_lens:
        offsets.append(offsets[-1] + int(n))
    return torch.tensor(offsets, dtype=torch.int32, device=device)


def _torch_float_dtype(dtype) -> torch.dtype:
    """``dtype`` as a torch float dtype; names as the reference maps them (``cache.py:758-773``), else fp16."""
    if isinstance(dtype, torch.dtype):
        return dtype
    names = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}
    return names.get(str(dtype).replace("torch.", ""), torch.float16)


def block_mapping_on_device(block_mapping, device) -> torch.Tensor:
    """``[num_pairs, 2]`` (src, dst) rows as an int32 device tensor (the reference's shape check,
    ``cache.py:953-954``)."""
    m = block_mapping if isinstance(block_mapping, torch.Tensor) else torch.as_tensor(block_mapping)
    if m.ndim != 2 or m.shape[1] != 2:
        raise ValueError("block_mapping must be rank-2 with shape [num_pairs, 2]")
    return m.to(device=device, dtype=torch.int32).contiguous()


def _stream_ptr(device: torch.device) -> int:
    return _native.stream_ptr(device)


def _contiguous_tables(num_seqs: int, blocks_per_seq: int, device) -> torch.Tensor:
    # Each sequence owns ``blocks_per_seq`` consecutive blocks (``cache.py:779-786``).
    return torch.arange(num_seqs * blocks_per_seq, dtype=torch.int32, device=device).reshape(num_seqs, blocks_per_seq)


def _v_shape(nb: int, hkv: int, d: int, bs: int, bits: int) -> tuple[int, ...]:
    # value codes in tiles of T = min(bs, 256 // bits) tokens, dim-major inside a tile
    t = min(bs, 256 // bits)
    return (nb, hkv, bs // t, d, t * bits // 32)


class PageCacheView:
    """Unquantized paged cache ``[num_blocks, block_size, Hkv, D]`` (``cache.py:700-825``)."""

    is_affine = False

    def __init__(self, *, key_cache, value_cache, block_tables, kv_lens, block_size, num_kv_heads, head_dim):
        self.key_cache = key_cache
        self.value_cache = value_cache
        self.block_tables = block_tables
        self.kv_lens = kv_lens
        self.block_size = int(block_size)
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = int(head_dim)

    @classmethod
    def init(
        cls,
        *,
        num_seqs: int,
        max_seq_len: int,
        num_kv_heads: int,
        head_dim: int,
        block_size: int = 16,
        dtype: torch.dtype | str = torch.float16,
        cache_dtype: str | None = None,
        cache_bits: int | None = None,
        group_size: int = 64,
        device: tp.Any = "cuda",
    ) -> "PageCacheView":
        """Allocate a zero-initialised cache (``cache.py:700-825``).

        ``cache_dtype`` selects the storage as the reference's does: ``None`` /
        ``"auto"`` / a float name stores ``dtype``; ``"fp8"`` an
        :class:`Fp8PageCacheView`; ``"affine4"`` / ``"affine8"`` an
        :class:`AffinePageCacheView` (this build's affine modes, ``group_size``
        per quantization group).  TurboQuant modes are outside this build.
        """
        from .pagecache import resolve_cache_dtype

        kind, bits = resolve_cache_dtype(cache_dtype, cache_bits)
        if cls is PageCacheView and kind == "fp8":
            return Fp8PageCacheView.init(num_seqs=num_seqs, max_seq_len=max_seq_len, num_kv_heads=num_kv_heads,
                                         head_dim=head_dim, block_size=block_size, device=device)
        if cls is PageCacheView and kind == "affine":
            return AffinePageCacheView.init(num_seqs=num_seqs, max_seq_len=max_seq_len, num_kv_heads=num_kv_heads,
                                            head_dim=head_dim, block_size=block_size, bits=bits,
                                            group_size=group_size, device=device)
        if kind == "float" and cache_dtype not in (None, "auto"):
            dtype = cache_dtype
        dtype = _torch_float_dtype(dtype)
        if num_seqs <= 0:
            raise ValueError("num_seqs must be positive")
        if max_seq_len <= 0:
            raise ValueError("max_seq_len must be positive")
        if block_size <= 0:
            raise ValueError("block_size must be positive")
        bps = math.ceil(max_seq_len / block_size)
        nb = bps * num_seqs
        shape = (nb, block_size, num_kv_heads, head_dim)
        return cls(
            key_cache=torch.zeros(shape, dtype=dtype, device=device),
            value_cache=torch.zeros(shape, dtype=dtype, device=device),
            block_tables=_contiguous_tables(num_seqs, bps, device),
            kv_lens=torch.zeros((num_seqs,), dtype=torch.int32, device=device),
            block_size=block_size,
            num_kv_heads=num_kv_heads,
            head_dim=head_dim,
        )

    allocate = init

    @property
    def num_seqs(self) -> int:
        return int(self.block_tables.shape[0])

    @property
    def blocks_per_seq(self) -> int:
        return int(self.block_tables.shape[1])

    @property
    def max_seq_len(self) -> int:
        return self.blocks_per_seq * self.block_size

    @property
    def num_blocks(self) -> int:
        return int(self.key_cache.shape[0])

    # -- slot arithmetic shared by all views (cache.py:1126-1170, 1211-1261), on the device
    def _check_tables(self) -> torch.device:
        dev = self.block_tables.device
        if dev.type != "cuda" or self.kv_lens.device != dev:
            raise RuntimeError(f"cache writes run on the GPU only; block_tables / kv_lens are on {dev}")
        if self.block_tables.dtype != torch.int32 or self.kv_lens.dtype != torch.int32:
            raise ValueError("block_tables and kv_lens must be int32")
        return dev

    def _slots(self, slot_ids, qlens):
        """Slot mapping and position of every written token, by ``emx_cache_slots``; advances ``kv_lens``.

        Returns ``(slot_mapping, slots, positions, query_start_loc)`` as int32
        device tensors.  The only host work is one copy of the call's slot ids
        and query offsets (host data in the reference's API) to the device.
        """
        dev = self._check_tables()
        n = len(slot_ids)
        # the device copy of (slot ids, offsets) is kept per distinct call shape: every
        # layer of a step (and most steps) writes the same slots, and a host-to-device
        # copy from pageable memory waits for the stream
        key = (tuple(slot_ids), tuple(qlens))
        cache = self.__dict__.setdefault("_meta_cache", {})
        hit = cache.get(key)
        if hit is None:
            qsl = [0]
            for q in qlens:
                qsl.append(qsl[-1] + max(0, int(q)))
            if len(cache) >= 64:
                cache.pop(next(iter(cache)))
            meta = torch.tensor(list(slot_ids) + qsl, dtype=torch.int32, device=dev)
            hit = cache[key] = (meta[:n], meta[n:], qsl[-1])
        slots, qsl_d, total = hit
        mapping = torch.empty((total,), dtype=torch.int32, device=dev)
        positions = torch.empty((total,), dtype=torch.int32, device=dev)
        if n:
            bt = self.block_tables.contiguous()
            _native.check(_native.load().emx_cache_slots(
                slots.data_ptr(), qsl_d.data_ptr(), n, total, bt.data_ptr(), int(bt.shape[0]), int(bt.shape[1]),
                self.block_size, self.kv_lens.data_ptr(), mapping.data_ptr(), positions.data_ptr(),
                _stream_ptr(dev)))
        return mapping, slots, positions, qsl_d

    def _resolve(self, cache_metadata, slot_ids, query_lens, n_tokens):
        if slot_ids is None:
            slot_ids = getattr(cache_metadata, "slot_ids", None) or ()
        # a runner passes the same (immutable) tuples at every layer of a step: their
        # conversion is kept for the last pair seen
        memo = self.__dict__.get("_resolve_memo")
        if memo is not None and memo[0] is slot_ids and memo[1] is query_lens and memo[2] == n_tokens:
            return memo[3]
        ids = tuple(int(s) for s in slot_ids)
        if query_lens is not None:
            qlens = tuple(int(q) for q in query_lens)
        else:
            qsl = cache_metadata.query_start_loc
            qsl = qsl.tolist() if isinstance(qsl, torch.Tensor) else list(qsl)
            qlens = tuple(int(qsl[i + 1]) - int(qsl[i]) for i in range(len(ids)))
        single = bool(qlens) and n_tokens == len(qlens) and all(q == 1 for q in qlens)
        res = (ids, qlens, single)
        if type(slot_ids) is tuple and type(query_lens) is tuple:
            self._resolve_memo = (slot_ids, query_lens, n_tokens, res)
        return res

    def _apply_rope(self, rope, queries, keys, positions, qsl, qlens, single):
        """A RoPE callable applied as the reference applies it (``cache.py:1161-1166``, ``:1223-1229``).

        A :class:`RotaryEmbedding` over fp16 rows turns on the device by
        ``emx_rope_rows`` at every token's position (the rotation of the fused
        writes); any other callable gets per-sequence offsets."""
        from .rope import RotaryEmbedding

        if rope is None:
            return queries, keys
        if (isinstance(rope, RotaryEmbedding) and queries.dtype == torch.float16 and keys.dtype == torch.float16
                and rope.dims <= self.head_dim and queries.shape[-1] == self.head_dim):
            n = int(positions.shape[0])
            lib = _native.load()
            inv = rope.inv_freq(queries.device)
            stream = _stream_ptr(queries.device)
            q_out, k_out = queries[:n].contiguous().clone(), keys[:n].contiguous().clone()
            for x in (q_out, k_out):
                if n:
                    _native.check(lib.emx_rope_rows(x.data_ptr(), n, int(x.shape[1]), self.head_dim,
                                                    positions.data_ptr(), inv.data_ptr(), rope.dims,
                                                    int(rope.traditional), stream))
            return q_out, k_out
        if single:
            qb = queries.unsqueeze(1).transpose(1, 2)
            kb = keys.unsqueeze(1).transpose(1, 2)
            return (
                rope(qb, offset=positions).transpose(1, 2)[:, 0],
                rope(kb, offset=positions).transpose(1, 2)[:, 0],
            )
        q_out, k_out, start = [], [], 0
        # per-chunk integer offsets for an arbitrary callable (the fused RotaryEmbedding path needs none)
        first = [int(qsl[i]) for i in range(len(qlens)) if qlens[i] > 0]
        base_host = positions[first].tolist() if first else []
        for n in qlens:
            if n <= 0:
                continue
            qc = queries[start : start + n][None].transpose(1, 2)
            kc = keys[start : start + n][None].transpose(1, 2)
            off = int(base_host[len(q_out)])
            q_out.append(rope(qc, offset=off).transpose(1, 2)[0])
            k_out.append(rope(kc, offset=off).transpose(1, 2)[0])
            start += n
        if not q_out:
            return queries[:0], keys[:0]
        return torch.cat(q_out), torch.cat(k_out)

    def _write(self, keys, values, slot_mapping):
        # cast like the cache (cache.py:1186-1190), then the scatter kernel (-1 skips)
        codes = {torch.float16: _native.DTYPE_F16, torch.bfloat16: _native.DTYPE_BF16, torch.float32: _native.DTYPE_F32}
        if self.key_cache.dtype not in codes:
            raise NotImplementedError(f"unquantized caches hold fp16/bf16/fp32, not {self.key_cache.dtype}")
        keys = keys.to(self.key_cache.dtype).contiguous()
        values = values.to(self.value_cache.dtype).contiguous()
        slot_mapping = slot_mapping.to(torch.int32).contiguous()
        _native.check(_native.load().emx_dense_cache_write(
            keys.data_ptr(), values.data_ptr(), codes[self.key_cache.dtype], slot_mapping.data_ptr(),
            int(keys.shape[0]), self.num_kv_heads, self.head_dim, self.block_size, self.num_blocks,
            self.key_cache.data_ptr(), self.value_cache.data_ptr(), _stream_ptr(keys.device)))

    def concatenate_to_cache(
        self,
        queries: torch.Tensor,
        keys: torch.Tensor,
        values: torch.Tensor,
        *,
        cache_metadata: tp.Any,
        rope: tp.Any = None,
        slot_ids: tp.Sequence[int] | None = None,
        query_lens: tp.Sequence[int] | None = None,
    ):
        """Append K/V for the scheduled slots (``cache.py:1088-1306``)."""
        slot_ids, qlens, single = self._resolve(cache_metadata, slot_ids, query_lens, int(queries.shape[0]))
        slot_mapping, slots, positions, qsl = self._slots(slot_ids, qlens)
        queries, keys = self._apply_rope(rope, queries, keys, positions, qsl, qlens, single)
        if slot_mapping.numel():
            self._write(keys.contiguous(), values.contiguous(), slot_mapping)
        return queries, self.key_cache, self.value_cache, self._resolved(cache_metadata, slots, single, slot_ids)

    def _resolved(self, cache_metadata, slots, single, slot_ids=None):
        """Metadata with this cache's tables and lengths for the written slots (``cache.py:1297-1305``).

        A call that writes every sequence in order gets the cache's own ``block_tables`` and
        ``kv_lens`` (no copies): a later write to this cache advances the lengths the returned
        metadata holds, so use it for this layer-step's attention, as the runner does."""
        n = int(slots.shape[0])
        in_order = self.__dict__.setdefault("_in_order", {})  # slot-id tuple -> writes every sequence in order
        if slot_ids is not None:
            key = tuple(slot_ids)
            whole = in_order.get(key)
            if whole is None:
                whole = in_order[key] = n == self.num_seqs and key == tuple(range(n))
                if len(in_order) > 64:
                    in_order.pop(next(iter(in_order)))
        else:
            whole = False
        if whole:
            tables, lens = self.block_tables, self.kv_lens
        else:
            tables = self.block_tables.index_select(0, slots) if n else self.block_tables[:0]
            lens = self.kv_lens.index_select(0, slots) if n else self.kv_lens[:0]
        md = cache_metadata.with_cache_state(block_tables=tables, kv_lens=lens, block_size=self.block_size)
        md.is_single_token_decode = single
        return md

    def _slot_ids_device(self, slot_ids: tuple) -> torch.Tensor:
        """The call's slot ids as a device int32 tensor, kept per distinct tuple (as ``_slots`` keeps them)."""
        cache = self.__dict__.setdefault("_slot_id_cache", {})
        t = cache.get(slot_ids)
        if t is None:
            if len(cache) >= 64:
                cache.pop(next(iter(cache)))
            t = cache[slot_ids] = torch.tensor(slot_ids, dtype=torch.int32, device=self.block_tables.device)
        return t

    def _append_counter(self, stream: int) -> torch.Tensor:
        """The device ints the decode append counts its workgroups on (zero between calls), one set per
        stream: appends ordered on one stream share it, appends issued on another stream never do."""
        counters = self.__dict__.setdefault("_counters", {})
        c = counters.get(stream)
        if c is None:
            c = counters[stream] = torch.zeros(_native.APPEND_COUNTER_INTS, dtype=torch.int32,
                                               device=self.block_tables.device)
        return c

    def _concatenate_rope_fused(self, queries, keys, values, cache_metadata, rope, slot_ids, query_lens, write,
                                rot_multiple, writes_queries=False, append=None):
        """The write with a :class:`RotaryEmbedding` fused into ``write`` (a cache's C entry point) and Q turned
        by ``emx_rope_rows``; any other ``rope`` (or fp16-incompatible inputs) takes the reference's order."""
        from .rope import RotaryEmbedding

        if (not isinstance(rope, RotaryEmbedding) or rope.dims > self.head_dim or rope.dims % rot_multiple
                or queries.shape[-1] != self.head_dim or queries.dtype != torch.float16):
            return PageCacheView.concatenate_to_cache(self, queries, keys, values, cache_metadata=cache_metadata,
                                                      rope=rope, slot_ids=slot_ids, query_lens=query_lens)
        slot_ids, qlens, single = self._resolve(cache_metadata, slot_ids, query_lens, int(queries.shape[0]))
        if append is not None and single and int(keys.shape[0]) == len(slot_ids):
            # one token per sequence: positions, slots, the K/V write, Q's rotation and the
            # kv_lens update in one launch (emx_affine_cache_append_rope)
            self._check_tables()
            q_in = queries.contiguous()
            q_out = torch.empty_like(q_in)
            slots = self._slot_ids_device(slot_ids)
            stream = _stream_ptr(q_in.device)
            rc = append(keys, values, slots, rope.inv_freq(q_in.device), rope, stream, q_in, q_out,
                        self._append_counter(stream))
            if rc == _native.EMX_OK:
                return q_out, self.key_cache, self.value_cache, self._resolved(cache_metadata, slots, single,
                                                                               slot_ids)
            if rc != _native.EMX_ERR_UNSUPPORTED:
                _native.check(rc)
        slot_mapping, slots, positions, _ = self._slots(slot_ids, qlens)
        lib = _native.load()
        n = int(slot_mapping.numel())
        q_in = queries.contiguous()
        if n and writes_queries and n == int(q_in.shape[0]):
            # the write kernel turns every query row into a fresh tensor (no copy first)
            q_out = torch.empty_like(q_in)
            _native.check(write(keys, values, slot_mapping, positions, rope.inv_freq(q_in.device), rope,
                                _stream_ptr(q_in.device), q_in, q_out))
        else:
            q_out = q_in.clone()
            if n:
                inv = rope.inv_freq(q_out.device)
                stream = _stream_ptr(q_out.device)
                if not writes_queries:
                    _native.check(lib.emx_rope_rows(q_out.data_ptr(), n, int(q_out.shape[1]), self.head_dim,
                                                    positions.data_ptr(), inv.data_ptr(), rope.dims,
                                                    int(rope.traditional), stream))
                _native.check(write(keys, values, slot_mapping, positions, inv, rope, stream, None, q_out))
        return q_out, self.key_cache, self.value_cache, self._resolved(cache_metadata, slots, single, slot_ids)

    def append(self, seq_idx: int, key: torch.Tensor, value: torch.Tensor) -> None:
        """Append ``[num_tokens, Hkv, D]`` tokens to one sequence (``cache.py:834-872``)."""
        if key.shape != value.shape:
            raise ValueError("key and value must have the same shape")
        if key.ndim != 3:
            raise ValueError("key/value must be rank-3: [num_tokens, num_kv_heads, head_dim]")
        if key.shape[1] != self.num_kv_heads or key.shape[2] != self.head_dim:
            raise ValueError("key/value head dims do not match cache")
        if seq_idx < 0 or seq_idx >= self.num_seqs:
            raise IndexError(f"Invalid seq_idx {seq_idx}")
        start = int(self.kv_lens[seq_idx].item())
        n = int(key.shape[0])
        if start + n > self.max_seq_len:
            raise ValueError("Cannot append tokens: sequence length would exceed cache capacity")
        slot_mapping, _, _, _ = self._slots([seq_idx], [n])  # advances kv_lens[seq_idx] by n
        if n:
            self._write(key.to(self.block_tables.device).contiguous(), value.to(self.block_tables.device).contiguous(),
                        slot_mapping)

    # -- page lifecycle (cache.py:874-972; runner model_runner.py:1058-1094), on the device
    def page_arrays(self) -> list[torch.Tensor]:
        """Every array of the cache indexed by block first (codes, then scales / biases where present)."""
        return [self.key_cache, self.value_cache]

    def _page_call(self, fn, ids: torch.Tensor, count: int, staging: bool = False) -> None:
        import ctypes

        arrays = self.page_arrays()
        for t in arrays:
            if not t.is_cuda or not t.is_contiguous() or int(t.shape[0]) != self.num_blocks:
                raise RuntimeError("page arrays must be contiguous device tensors with num_blocks rows")
        ptrs = (ctypes.c_void_p * len(arrays))(*[t.data_ptr() for t in arrays])
        sizes = (ctypes.c_int64 * len(arrays))(*[t[0].numel() * t.element_size() for t in arrays])
        extra = ()
        if staging:  # copy_blocks: the pairs' source blocks are staged before any destination is written
            nbytes = int(_native.load().emx_copy_blocks_workspace_bytes(len(arrays), sizes, count))
            ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=arrays[0].device)
            extra = (ws.data_ptr(), ws.numel())
        _native.check(fn(len(arrays), ptrs, sizes, self.num_blocks, ids.data_ptr(), count, *extra,
                         _stream_ptr(arrays[0].device)))

    def zero_pages(self, page_ids) -> None:
        """Zero the given pages of every array (the runner's ``_zero_pages``, ``model_runner.py:1058-1094``).

        ``page_ids``: host ints or a device int32 tensor; ids outside ``[0, num_blocks)`` are skipped."""
        ids = torch.as_tensor(page_ids, dtype=torch.int32).reshape(-1).to(self.key_cache.device).contiguous()
        if ids.numel():
            self._page_call(_native.load().emx_zero_blocks, ids, int(ids.numel()))

    def copy_blocks(self, block_mapping) -> None:
        """Copy-on-write block copies (``cache.py:944-972``): rows ``(src, dst)`` of ``[num_pairs, 2]``.

        Every destination receives its source block as it was before the call
        (the reference's kernel reads its inputs), so swapped and chained pairs
        are well defined; of several pairs with one destination the last counts."""
        m = block_mapping_on_device(block_mapping, self.key_cache.device)
        if m.shape[0]:
            self._page_call(_native.load().emx_copy_blocks, m, int(m.shape[0]), staging=True)

    def gather_kv_cache(self, block_table, cu_seq_lens, *, out_dtype: torch.dtype | None = None):
        """Dense ``(k, v)`` ``[total_tokens, Hkv, D]`` of a ragged batch from the pages (``cache.py:974-1027``).

        Token ``t`` of sequence ``b`` (``cu_seq_lens[b] <= t < cu_seq_lens[b+1]``)
        is entry ``j % block_size`` of page ``block_table[b, j // block_size]``,
        ``j = t - cu_seq_lens[b]``.  ``out_dtype`` defaults to the cache dtype
        for unquantized caches and to fp16 for FP8 / affine pages, which are
        returned dequantized (the reference gathers its unquantized packed copy)."""
        dev = self.key_cache.device
        bt = torch.as_tensor(block_table).to(device=dev, dtype=torch.int32).contiguous()
        cu = torch.as_tensor(cu_seq_lens).to(device=dev, dtype=torch.int32).contiguous()
        if bt.ndim != 2 or cu.ndim != 1 or cu.shape[0] != bt.shape[0] + 1:
            raise ValueError("block_table must be [num_seqs, max_blocks] and cu_seq_lens [num_seqs + 1]")
        total = int(cu[-1].item())  # the output size, as the reference reads it (cache.py:1000-1002)
        if out_dtype is None:
            out_dtype = self.key_cache.dtype if self.key_cache.dtype.is_floating_point else torch.float16
        codes = {torch.float16: _native.DTYPE_F16, torch.bfloat16: _native.DTYPE_BF16, torch.float32: _native.DTYPE_F32}
        if out_dtype not in codes:
            raise NotImplementedError(f"gather_kv_cache returns fp16/bf16/fp32, not {out_dtype}")
        k_out = torch.empty((total, self.num_kv_heads, self.head_dim), dtype=out_dtype, device=dev)
        v_out = torch.empty_like(k_out)
        if total:
            self._gather(bt, cu, total, codes[out_dtype], k_out, v_out)
        return k_out, v_out

    def _gather(self, bt, cu, total, out_code, k_out, v_out):
        codes = {torch.float16: _native.DTYPE_F16, torch.bfloat16: _native.DTYPE_BF16, torch.float32: _native.DTYPE_F32}
        if self.key_cache.dtype not in codes:
            raise NotImplementedError(f"no gather for a {self.key_cache.dtype} cache")
        _native.check(_native.load().emx_gather_kv_dense(
            self.key_cache.data_ptr(), self.value_cache.data_ptr(), codes[self.key_cache.dtype], self.num_blocks,
            self.block_size, self.num_kv_heads, self.head_dim, bt.data_ptr(), int(bt.shape[0]), int(bt.shape[1]),
            cu.data_ptr(), total, out_code, k_out.data_ptr(), v_out.data_ptr(), _stream_ptr(k_out.device)))

    def reset(self, seq_idx: int) -> None:
        """Zero one sequence's pages and its length (``cache.py:874-906``, pages addressed by id)."""
        if seq_idx < 0 or seq_idx >= self.num_seqs:
            raise IndexError(f"Invalid seq_idx {seq_idx}")
        self.zero_pages(self.block_tables[seq_idx])  # invalid ids (-1) are skipped by the kernel
        self.kv_lens[seq_idx] = 0

    def reset_batch(self, seq_indices) -> None:
        """``cache.py:908-915``."""
        for seq_idx in seq_indices:
            self.reset(int(seq_idx))

    def clear(self, seq_idx: int | None = None) -> None:
        """Zero the whole cache and every length, or one sequence (``cache.py:917-933``)."""
        if seq_idx is not None:
            self.reset(int(seq_idx))
            return
        for t in self.page_arrays():
            t.zero_()
        self.kv_lens.zero_()

    def clear_many(self, seq_indices) -> None:
        """``cache.py:935-942``."""
        self.reset_batch(seq_indices)


class Fp8PageCacheView(PageCacheView):
    """FP8 (E4M3) page cache with per-page fp32 scales (``cache.py:770-797, 1171-1184``).

    ``key_cache/value_cache [num_blocks, block_size, Hkv, D]`` uint8 codes and
    ``k_scales/v_scales [num_blocks]`` float32 (zero at allocation), as the
    reference's FP8 cache.  Writes go through ``emx_fp8_cache_write``: one scale
    per call (``max|x| / 240``), codes ``enc(x / scale)``, and each written page's
    scale raised to ``max(page scale, call scale)`` without requantizing the
    page's earlier codes -- the reference's rule (``cache.py:1181-1184``).
    """

    cache_dtype_is_fp8 = True

    def __init__(self, *, key_cache, value_cache, k_scales, v_scales, block_tables, kv_lens, block_size,
                 num_kv_heads, head_dim):
        super().__init__(key_cache=key_cache, value_cache=value_cache, block_tables=block_tables, kv_lens=kv_lens,
                         block_size=block_size, num_kv_heads=num_kv_heads, head_dim=head_dim)
        self.k_scales = k_scales
        self.v_scales = v_scales
        self._ws: torch.Tensor | None = None

    @classmethod
    def init(
        cls,
        *,
        num_seqs: int,
        max_seq_len: int,
        num_kv_heads: int,
        head_dim: int,
        block_size: int = 16,
        dtype: torch.dtype = torch.uint8,
        device: tp.Any = "cuda",
    ) -> "Fp8PageCacheView":
        if dtype != torch.uint8:
            raise ValueError("an FP8 cache stores uint8 codes")
        base = PageCacheView.init(num_seqs=num_seqs, max_seq_len=max_seq_len, num_kv_heads=num_kv_heads,
                                  head_dim=head_dim, block_size=block_size, dtype=torch.uint8, device=device)
        nb = int(base.key_cache.shape[0])
        return cls(key_cache=base.key_cache, value_cache=base.value_cache,
                   k_scales=torch.zeros((nb,), dtype=torch.float32, device=device),
                   v_scales=torch.zeros((nb,), dtype=torch.float32, device=device),
                   block_tables=base.block_tables, kv_lens=base.kv_lens, block_size=block_size,
                   num_kv_heads=num_kv_heads, head_dim=head_dim)

    allocate = init

    def _write(self, keys, values, slot_mapping):
        from .._native import DTYPE_BF16, DTYPE_F16, DTYPE_F32, check, load

        codes = {torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16, torch.float32: DTYPE_F32}
        if keys.dtype not in codes or values.dtype != keys.dtype:
            raise NotImplementedError(f"FP8 cache writes take fp16/bf16/fp32 keys and values, got {keys.dtype}")
        lib = load()
        if self._ws is None:
            self._ws = torch.empty(int(lib.emx_fp8_write_workspace_bytes()), dtype=torch.uint8,
                                   device=self.key_cache.device)
        keys = keys.contiguous()
        values = values.contiguous()
        slot_mapping = slot_mapping.to(device=keys.device, dtype=torch.int32).contiguous()
        check(
            lib.emx_fp8_cache_write(
                keys.data_ptr(), values.data_ptr(), codes[keys.dtype], slot_mapping.data_ptr(), int(keys.shape[0]),
                self.num_kv_heads, self.head_dim, self.block_size, self.num_blocks,
                self.key_cache.data_ptr(), self.value_cache.data_ptr(), self.k_scales.data_ptr(),
                self.v_scales.data_ptr(), self._ws.data_ptr(), self._ws.numel(), _stream_ptr(keys.device),
            )
        )

    def concatenate_to_cache(self, queries, keys, values, *, cache_metadata, rope=None, slot_ids=None,
                             query_lens=None):
        """With a :class:`RotaryEmbedding`, the call's K scale and codes come from the keys turned inside the
        write kernels (``cache.py:1161-1166`` then ``:1171-1184``); Q turns in one launch."""
        from .._native import DTYPE_BF16, DTYPE_F16, DTYPE_F32

        codes = {torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16, torch.float32: DTYPE_F32}

        def write(keys, values, slot_mapping, positions, inv, rope, stream, q_in, q_out):
            if keys.dtype not in codes or values.dtype != keys.dtype:
                raise NotImplementedError(f"FP8 cache writes take fp16/bf16/fp32 keys and values, got {keys.dtype}")
            lib = _native.load()
            if self._ws is None:
                self._ws = torch.empty(int(lib.emx_fp8_write_workspace_bytes()), dtype=torch.uint8,
                                       device=self.key_cache.device)
            keys = keys.contiguous()
            values = values.contiguous()
            return lib.emx_fp8_cache_write_rope(
                keys.data_ptr(), values.data_ptr(), codes[keys.dtype], slot_mapping.data_ptr(), int(keys.shape[0]),
                self.num_kv_heads, self.head_dim, self.block_size, self.num_blocks, self.key_cache.data_ptr(),
                self.value_cache.data_ptr(), self.k_scales.data_ptr(), self.v_scales.data_ptr(), self._ws.data_ptr(),
                self._ws.numel(), positions.data_ptr(), inv.data_ptr(), rope.dims, int(rope.traditional),
                None if q_in is None else q_in.data_ptr(), q_out.data_ptr(), int(q_out.shape[1]), stream)

        def append(keys, values, slots, inv, rope, stream, q_in, q_out, counter):
            if keys.dtype not in codes or values.dtype != keys.dtype or not self.block_tables.is_contiguous():
                return _native.EMX_ERR_UNSUPPORTED
            keys = keys.contiguous()
            values = values.contiguous()
            bt = self.block_tables
            return _native.load().emx_fp8_cache_append_rope(
                keys.data_ptr(), values.data_ptr(), codes[keys.dtype], slots.data_ptr(), int(keys.shape[0]),
                bt.data_ptr(), int(bt.shape[0]), int(bt.shape[1]), self.kv_lens.data_ptr(), counter.data_ptr(),
                self.num_kv_heads, self.head_dim, self.block_size, self.num_blocks, self.key_cache.data_ptr(),
                self.value_cache.data_ptr(), self.k_scales.data_ptr(), self.v_scales.data_ptr(), inv.data_ptr(),
                rope.dims, int(rope.traditional), q_in.data_ptr(), q_out.data_ptr(), int(q_out.shape[1]), stream)

        return self._concatenate_rope_fused(queries, keys, values, cache_metadata, rope, slot_ids, query_lens, write,
                                            rot_multiple=4 if getattr(rope, "traditional", False) else 8,
                                            writes_queries=True, append=append)

    def write_slots(self, keys: torch.Tensor, values: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        """Write tokens to explicit slots (``block * block_size + offset``; -1 skips)."""
        if keys.shape != values.shape or keys.ndim != 3:
            raise ValueError("keys/values must be [num_tokens, num_kv_heads, head_dim] of one shape")
        if keys.shape[0]:
            self._write(keys, values, slot_mapping)

    def page_arrays(self) -> list[torch.Tensor]:
        # the per-page scales travel with their pages (zeroed pages restart from scale 0)
        return [self.key_cache, self.value_cache, self.k_scales, self.v_scales]

    def _gather(self, bt, cu, total, out_code, k_out, v_out):
        _native.check(_native.load().emx_gather_kv_fp8(
            self.key_cache.data_ptr(), self.value_cache.data_ptr(), self.k_scales.data_ptr(), self.v_scales.data_ptr(),
            self.num_blocks, self.block_size, self.num_kv_heads, self.head_dim, bt.data_ptr(), int(bt.shape[0]),
            int(bt.shape[1]), cu.data_ptr(), total, out_code, k_out.data_ptr(), v_out.data_ptr(),
            _stream_ptr(k_out.device)))


class AffinePageCacheView(PageCacheView):
    """Affine int4/int8 KV pages with fused quantize-on-write.

    Storage (see ``include/emx_attn.h``): key codes ``[nb, Hkv, bs, D*b/32]``,
    value codes ``[nb, Hkv, bs/T, D, T*b/32]`` with ``T = min(bs, 256/b)`` (int32
    tensors holding uint32 words),
    scales/biases ``[nb, Hkv, D/gs, bs]`` fp16.  The reference has no affine KV
    cache; its FP8 cache (``cache.py:770-797, 1171-1184``) is the structural
    analogue, with the per-block running-max scale replaced by MLX's affine
    per-(token, group) scale and bias.
    """

    is_affine = True

    def __init__(self, *, k_codes, k_scales, k_biases, v_codes, v_scales, v_biases, block_tables, kv_lens, block_size,
                 num_kv_heads, head_dim, bits, group_size):
        super().__init__(key_cache=k_codes, value_cache=v_codes, block_tables=block_tables, kv_lens=kv_lens,
                         block_size=block_size, num_kv_heads=num_kv_heads, head_dim=head_dim)
        self.k_scales = k_scales
        self.k_biases = k_biases
        self.v_scales = v_scales
        self.v_biases = v_biases
        self.bits = int(bits)
        self.group_size = int(group_size)

    @classmethod
    def init(
        cls,
        *,
        num_seqs: int,
        max_seq_len: int,
        num_kv_heads: int,
        head_dim: int,
        block_size: int = 128,
        bits: int = 4,
        group_size: int = 64,
        num_blocks: int | None = None,
        device: tp.Any = "cuda",
    ) -> "AffinePageCacheView":
        if num_seqs <= 0:
            raise ValueError("num_seqs must be positive")
        if max_seq_len <= 0:
            raise ValueError("max_seq_len must be positive")
        if block_size <= 0:
            raise ValueError("block_size must be positive")
        if bits not in (4, 8):
            raise ValueError("bits must be 4 or 8")
        if group_size <= 0 or head_dim % group_size or group_size % 8:
            raise ValueError("head_dim must be a multiple of group_size, itself a multiple of 8")
        if (block_size * bits) % 32 or (head_dim * bits) % 32:
            raise ValueError("block_size * bits and head_dim * bits must be multiples of 32")
        if block_size > 256 // bits and block_size % (256 // bits):
            raise ValueError("block_size above 256 // bits must be a multiple of 256 // bits")
        bps = math.ceil(max_seq_len / block_size)
        nb = num_blocks if num_blocks is not None else bps * num_seqs
        if nb < bps * num_seqs:
            raise ValueError("num_blocks is smaller than num_seqs * ceil(max_seq_len / block_size)")
        G = head_dim // group_size
        z = lambda shape, dt: torch.zeros(shape, dtype=dt, device=device)  # noqa: E731
        return cls(
            k_codes=z((nb, num_kv_heads, block_size, head_dim * bits // 32), torch.int32),
            k_scales=z((nb, num_kv_heads, G, block_size), torch.float16),
            k_biases=z((nb, num_kv_heads, G, block_size), torch.float16),
            v_codes=z(_v_shape(nb, num_kv_heads, head_dim, block_size, bits), torch.int32),
            v_scales=z((nb, num_kv_heads, G, block_size), torch.float16),
            v_biases=z((nb, num_kv_heads, G, block_size), torch.float16),
            block_tables=_contiguous_tables(num_seqs, bps, device),
            kv_lens=z((num_seqs,), torch.int32),
            block_size=block_size,
            num_kv_heads=num_kv_heads,
            head_dim=head_dim,
            bits=bits,
            group_size=group_size,
        )

    allocate = init

    @property
    def k_codes(self) -> torch.Tensor:
        return self.key_cache

    @property
    def v_codes(self) -> torch.Tensor:
        return self.value_cache

    def _write(self, keys, values, slot_mapping):
        if keys.dtype != torch.float16 or values.dtype != torch.float16:
            keys = keys.to(torch.float16)
            values = values.to(torch.float16)
        keys = keys.contiguous()
        values = values.contiguous()
        slot_mapping = slot_mapping.to(torch.int32).contiguous()
        lib = _native.load()
        _native.check(
            lib.emx_affine_cache_write(
                keys.data_ptr(),
                values.data_ptr(),
                slot_mapping.data_ptr(),
                int(keys.shape[0]),
                self.num_kv_heads,
                self.head_dim,
                self.group_size,
                self.bits,
                self.block_size,
                self.num_blocks,
                self.key_cache.data_ptr(),
                self.k_scales.data_ptr(),
                self.k_biases.data_ptr(),
                self.value_cache.data_ptr(),
                self.v_scales.data_ptr(),
                self.v_biases.data_ptr(),
                _stream_ptr(keys.device),
            )
        )

    def write_slots(self, keys: torch.Tensor, values: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        """Quantize-on-write ``[T, Hkv, D]`` tokens to flat slots ``block * bs + offset`` (-1 = skip).

        The affine counterpart of the reference's ``reshape_and_cache``
        (``cache.py:36-93, 281-337``); ``kv_lens`` is not touched.
        """
        if keys.shape != values.shape or keys.ndim != 3:
            raise ValueError("keys/values must be [num_tokens, num_kv_heads, head_dim] of equal shape")
        if keys.shape[1] != self.num_kv_heads or keys.shape[2] != self.head_dim:
            raise ValueError("key/value head dims do not match cache")
        if slot_mapping.shape != (keys.shape[0],):
            raise ValueError("slot_mapping must be [num_tokens]")
        if keys.shape[0]:
            self._write(keys, values, slot_mapping)

    def concatenate_to_cache(self, queries, keys, values, *, cache_metadata, rope=None, slot_ids=None,
                             query_lens=None):
        """``PageCacheView.concatenate_to_cache`` with a :class:`RotaryEmbedding` fused in: K turns inside the
        quantize-on-write kernel and Q in the same launch (``cache.py:1161-1166`` then ``:1186-1190``)."""

        def write(keys, values, slot_mapping, positions, inv, rope, stream, q_in, q_out):
            if keys.dtype != torch.float16 or not keys.is_contiguous():
                keys = keys.to(torch.float16).contiguous()
            if values.dtype != torch.float16 or not values.is_contiguous():
                values = values.to(torch.float16).contiguous()
            return _native.load().emx_affine_cache_write_rope(
                keys.data_ptr(), values.data_ptr(), slot_mapping.data_ptr(), int(keys.shape[0]), self.num_kv_heads,
                self.head_dim, self.group_size, self.bits, self.block_size, self.num_blocks,
                self.key_cache.data_ptr(), self.k_scales.data_ptr(), self.k_biases.data_ptr(),
                self.value_cache.data_ptr(), self.v_scales.data_ptr(), self.v_biases.data_ptr(),
                positions.data_ptr(), inv.data_ptr(), rope.dims, int(rope.traditional),
                None if q_in is None else q_in.data_ptr(), q_out.data_ptr(), int(q_out.shape[1]), stream)

        def append(keys, values, slots, inv, rope, stream, q_in, q_out, counter):
            if keys.dtype != torch.float16 or not keys.is_contiguous():
                keys = keys.to(torch.float16).contiguous()
            if values.dtype != torch.float16 or not values.is_contiguous():
                values = values.to(torch.float16).contiguous()
            bt = self.block_tables
            if not bt.is_contiguous():
                return _native.EMX_ERR_UNSUPPORTED
            return _native.load().emx_affine_cache_append_rope(
                keys.data_ptr(), values.data_ptr(), slots.data_ptr(), int(keys.shape[0]), bt.data_ptr(),
                int(bt.shape[0]), int(bt.shape[1]), self.kv_lens.data_ptr(), counter.data_ptr(), self.num_kv_heads,
                self.head_dim, self.group_size, self.bits, self.block_size, self.num_blocks,
                self.key_cache.data_ptr(), self.k_scales.data_ptr(), self.k_biases.data_ptr(),
                self.value_cache.data_ptr(), self.v_scales.data_ptr(), self.v_biases.data_ptr(), inv.data_ptr(),
                rope.dims, int(rope.traditional), q_in.data_ptr(), q_out.data_ptr(), int(q_out.shape[1]), stream)

        return self._concatenate_rope_fused(queries, keys, values, cache_metadata, rope, slot_ids, query_lens, write,
                                            rot_multiple=2, writes_queries=True, append=append)

    def page_arrays(self) -> list[torch.Tensor]:
        return [self.key_cache, self.value_cache, self.k_scales, self.k_biases, self.v_scales, self.v_biases]

    @classmethod
    def from_logical(cls, *, k_codes, k_scales, k_biases, v_codes, v_scales, v_biases, block_tables, kv_lens, bits,
                     group_size) -> "AffinePageCacheView":
        """A view over pages converted on the device from the logical layout (``emx_affine_pages_from_logical``):
        codes ``[nb, bs, Hkv, D*bits/32]`` (int32/uint32 words), scales/biases ``[nb, bs, Hkv, D/group_size]``
        fp16 -- ``mlx.core.quantize`` of the reference's dense cache ``[nb, bs, Hkv, D]`` (``cache.py:790-791``)."""
        nb, bs, hkv, w = (int(x) for x in k_codes.shape)
        d = w * 32 // int(bits)
        view = affine_pool(num_blocks=nb, num_kv_heads=hkv, head_dim=d, block_size=bs, bits=int(bits),
                           group_size=int(group_size), block_tables=block_tables.to(k_codes.device),
                           kv_lens=kv_lens.to(k_codes.device))
        pages_from_logical(k_codes, k_scales, k_biases, v_codes, v_scales, v_biases, bits, group_size,
                           out=view.page_arrays())
        return view

    def to_logical(self) -> dict[str, torch.Tensor]:
        """The pages in the logical layout (device tensors; ``emx_affine_logical_from_pages``)."""
        nb, hkv, bs, d = self.num_blocks, self.num_kv_heads, self.block_size, self.head_dim
        w, G = d * self.bits // 32, d // self.group_size
        dev = self.key_cache.device
        out = {"k_codes": torch.empty((nb, bs, hkv, w), dtype=torch.int32, device=dev),
               "v_codes": torch.empty((nb, bs, hkv, w), dtype=torch.int32, device=dev)}
        for n in ("k_scales", "k_biases", "v_scales", "v_biases"):
            out[n] = torch.empty((nb, bs, hkv, G), dtype=torch.float16, device=dev)
        _native.check(_native.load().emx_affine_logical_from_pages(
            self.key_cache.data_ptr(), self.value_cache.data_ptr(), self.k_scales.data_ptr(),
            self.k_biases.data_ptr(), self.v_scales.data_ptr(), self.v_biases.data_ptr(), nb, bs, hkv, d, self.bits,
            self.group_size, out["k_codes"].data_ptr(), out["v_codes"].data_ptr(), out["k_scales"].data_ptr(),
            out["k_biases"].data_ptr(), out["v_scales"].data_ptr(), out["v_biases"].data_ptr(), _stream_ptr(dev)))
        return out

    def _gather(self, bt, cu, total, out_code, k_out, v_out):
        _native.check(_native.load().emx_gather_kv_affine(
            self.key_cache.data_ptr(), self.k_scales.data_ptr(), self.k_biases.data_ptr(), self.value_cache.data_ptr(),
            self.v_scales.data_ptr(), self.v_biases.data_ptr(), self.num_blocks, self.block_size, self.num_kv_heads,
            self.head_dim, self.bits, self.group_size, bt.data_ptr(), int(bt.shape[0]), int(bt.shape[1]),
            cu.data_ptr(), total, out_code, k_out.data_ptr(), v_out.data_ptr(), _stream_ptr(k_out.device)))


def pages_from_logical(k_codes, k_scales, k_biases, v_codes, v_scales, v_biases, bits, group_size, out=None):
    """Affine pages ``[key codes, value codes, k_scales, k_biases, v_scales, v_biases]`` in this library's
    layout (``AffinePageCacheView``), converted on the device from the logical layout: codes
    ``[nb, bs, Hkv, D*bits/32]``, scales/biases ``[nb, bs, Hkv, D/group_size]`` (``emx_affine_pages_from_logical``).
    ``out``: the six page tensors to fill (new ones when None)."""
    dev = k_codes.device
    if dev.type != "cuda":
        raise RuntimeError("layout conversion runs on the GPU only")
    if k_codes.ndim != 4:
        raise ValueError("logical-layout codes must be rank-4: [num_blocks, block_size, num_kv_heads, W]")
    nb, bs, hkv, w = (int(x) for x in k_codes.shape)
    bits, group_size = int(bits), int(group_size)
    d = w * 32 // bits
    G = d // group_size
    for name, t, shape in (("v_codes", v_codes, (nb, bs, hkv, w)), ("k_scales", k_scales, (nb, bs, hkv, G)),
                           ("k_biases", k_biases, (nb, bs, hkv, G)), ("v_scales", v_scales, (nb, bs, hkv, G)),
                           ("v_biases", v_biases, (nb, bs, hkv, G))):
        if tuple(t.shape) != shape:
            raise ValueError(f"{name} must be {list(shape)} in the logical layout, got {list(t.shape)}")
    if out is None:
        out = [torch.empty((nb, hkv, bs, w), dtype=torch.int32, device=dev),
               torch.empty(_v_shape(nb, hkv, d, bs, bits), dtype=torch.int32, device=dev)]
        out += [torch.empty((nb, hkv, G, bs), dtype=torch.float16, device=dev) for _ in range(4)]
    src = [x.contiguous() for x in (k_codes, v_codes)]
    par = [x.to(torch.float16).contiguous() for x in (k_scales, k_biases, v_scales, v_biases)]
    _native.check(_native.load().emx_affine_pages_from_logical(
        src[0].data_ptr(), src[1].data_ptr(), *(x.data_ptr() for x in par), nb, bs, hkv, d, bits, group_size,
        *(t.data_ptr() for t in out), _stream_ptr(dev)))
    return out


def affine_pool(
    *,
    num_blocks: int,
    num_kv_heads: int,
    head_dim: int,
    block_size: int,
    bits: int,
    group_size: int,
    block_tables: torch.Tensor,
    kv_lens: torch.Tensor,
) -> AffinePageCacheView:
    """An empty affine page pool with caller-provided block tables / lengths."""
    dev = block_tables.device
    G = head_dim // group_size
    z = lambda shape, dt: torch.zeros(shape, dtype=dt, device=dev)  # noqa: E731
    return AffinePageCacheView(
        k_codes=z((num_blocks, num_kv_heads, block_size, head_dim * bits // 32), torch.int32),
        k_scales=z((num_blocks, num_kv_heads, G, block_size), torch.float16),
        k_biases=z((num_blocks, num_kv_heads, G, block_size), torch.float16),
        v_codes=z(_v_shape(num_blocks, num_kv_heads, head_dim, block_size, bits), torch.int32),
        v_scales=z((num_blocks, num_kv_heads, G, block_size), torch.float16),
        v_biases=z((num_blocks, num_kv_heads, G, block_size), torch.float16),
        block_tables=block_tables.to(torch.int32).contiguous(),
        kv_lens=kv_lens.to(torch.int32).contiguous(),
        block_size=block_size,
        num_kv_heads=num_kv_heads,
        head_dim=head_dim,
        bits=bits,
        group_size=group_size,
    )
