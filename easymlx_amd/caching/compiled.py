"""Decode-step cache write that can be captured in a HIP graph.

Counterpart of the reference's ``_CompiledPagedCacheProxy``
(``lib/python/easymlx/inference/esurge/runners/model_runner.py:46-189``), the
cache object its runner hands to the model when the decode step runs under
``mx.compile``.  Here the compiled form of a decode step is a HIP graph
(``torch.cuda.CUDAGraph``), and a captured step may not allocate device memory
from a fresh pool nor read device data back to the host.  The proxy therefore

* keeps, per tuple of slot ids, the device tensors a step needs (slot ids,
  query offsets, slot mapping, positions), made on the first call with that
  tuple -- run that call eagerly before capturing;
* computes every token's slot and position on the device (``emx_cache_slots``,
  which also advances ``kv_lens``), then writes with the view's fused kernel:
  quantize-on-write for affine pages (RoPE turned inside it), the FP8 write
  for FP8 pages (unlike the reference's proxy, which casts without quantizing,
  ``model_runner.py:174-175``), the scatter kernel for unquantized pages;
* returns metadata built from device tensors only.

Like the reference's proxy it accepts single-token decode only and raises
``ValueError("Compiled paged cache proxy only supports single-token decode.")``
otherwise (``model_runner.py:158-160``).
"""

from __future__ import annotations

import typing as tp

import torch

from .. import _native
from .paged import AffinePageCacheView, Fp8PageCacheView, PageCacheView


class CompiledPagedCacheProxy:
    """Graph-capturable decode-step writes into a :class:`PageCacheView` (``model_runner.py:46-189``)."""

    def __init__(self, cache: PageCacheView):
        if cache.block_tables.dtype != torch.int32 or cache.kv_lens.dtype != torch.int32:
            raise ValueError("block_tables and kv_lens must be int32")
        self.cache = cache
        self.block_size = cache.block_size
        self.num_kv_heads = cache.num_kv_heads
        self.head_dim = cache.head_dim
        self.cache_dtype_is_fp8 = bool(getattr(cache, "cache_dtype_is_fp8", False))
        self._steps: dict[tuple[int, ...], dict[str, torch.Tensor]] = {}
        self._fp8_ws: torch.Tensor | None = None

    # the reference proxy's state accessors (model_runner.py:79-131)
    @property
    def key_cache(self):
        return self.cache.key_cache

    @property
    def value_cache(self):
        return self.cache.value_cache

    @property
    def block_tables(self):
        return self.cache.block_tables

    @property
    def kv_lens(self):
        return self.cache.kv_lens

    @property
    def num_seqs(self) -> int:
        return int(self.cache.block_tables.shape[0])

    def _step_buffers(self, slots: tuple[int, ...], device) -> dict[str, torch.Tensor]:
        buf = self._steps.get(slots)
        if buf is None:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("CompiledPagedCacheProxy: slot ids %r were not seen before capture; run one eager "
                                   "step with them first" % (slots,))
            n = len(slots)
            meta = torch.tensor(list(slots) + list(range(n + 1)), dtype=torch.int32, device=device)
            buf = {
                "slots": meta[:n],
                "qsl": meta[n:],
                "mapping": torch.empty((n,), dtype=torch.int32, device=device),
                "positions": torch.empty((n,), dtype=torch.int32, device=device),
            }
            self._steps[slots] = buf
        return buf

    def concatenate_to_cache(
        self,
        queries: torch.Tensor,
        keys: torch.Tensor,
        values: torch.Tensor,
        *,
        cache_metadata: tp.Any,
        slot_ids: tp.Any = None,
        query_lens: tp.Any = None,
        rope: tp.Any = None,
    ):
        """Single-token decode write (``model_runner.py:139-189``); returns ``(q, key_cache, value_cache, md)``."""
        if slot_ids is None:
            slot_ids = getattr(cache_metadata, "slot_ids", None) or ()
        slots = tuple(int(s) for s in slot_ids)
        if query_lens is None:
            query_lens = (1,) * len(slots)
        if not slots or any(int(q) != 1 for q in query_lens):
            raise ValueError("Compiled paged cache proxy only supports single-token decode.")
        if int(queries.shape[0]) != len(slots) or keys.shape[0] != len(slots) or values.shape[0] != len(slots):
            raise ValueError("one query / key / value token per slot")
        c = self.cache
        dev = c.block_tables.device
        buf = self._step_buffers(slots, dev)
        lib = _native.load()
        stream = _native.stream_ptr(dev)
        n = len(slots)
        q_out = self._append(queries, keys, values, buf["slots"], rope, lib, stream)
        if q_out is not None:  # positions, slots, write, Q's rotation and kv_lens in one launch
            return q_out, c.key_cache, c.value_cache, self._metadata(cache_metadata, slots, buf)
        _native.check(lib.emx_cache_slots(
            buf["slots"].data_ptr(), buf["qsl"].data_ptr(), n, n, c.block_tables.data_ptr(),
            int(c.block_tables.shape[0]), int(c.block_tables.shape[1]), c.block_size, c.kv_lens.data_ptr(),
            buf["mapping"].data_ptr(), buf["positions"].data_ptr(), stream))
        mapping, positions = buf["mapping"], buf["positions"]
        q_out = self._write(queries, keys, values, mapping, positions, rope, lib, stream)
        return q_out, c.key_cache, c.value_cache, self._metadata(cache_metadata, slots, buf)

    def _metadata(self, cache_metadata, slots, buf):
        c = self.cache
        n = len(slots)
        if n == self.num_seqs and slots == tuple(range(n)):  # every sequence in order: the tables themselves
            tables, lens = c.block_tables, c.kv_lens
        else:
            tables, lens = c.block_tables.index_select(0, buf["slots"]), c.kv_lens.index_select(0, buf["slots"])
        md = cache_metadata.with_cache_state(block_tables=tables, kv_lens=lens, block_size=c.block_size)
        md.is_single_token_decode = True
        return md

    def _append(self, queries, keys, values, slots_d, rope, lib, stream):
        """The one-launch decode append with a fused RoPE (``emx_affine_cache_append_rope`` /
        ``emx_fp8_cache_append_rope``); None where it does not apply (the caller then takes the two launches)."""
        from .rope import RotaryEmbedding

        c = self.cache
        if not (isinstance(c, (AffinePageCacheView, Fp8PageCacheView)) and isinstance(rope, RotaryEmbedding)
                and rope.dims <= c.head_dim and queries.dtype == torch.float16 and c.block_tables.is_contiguous()):
            return None
        counter = self.__dict__.get("_counter")  # the proxy's own (its steps are ordered on the capturing stream)
        if counter is None:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("CompiledPagedCacheProxy: run one eager step before capture")
            counter = self._counter = torch.zeros(_native.APPEND_COUNTER_INTS, dtype=torch.int32,
                                                  device=c.block_tables.device)
        q_in = queries.contiguous()
        q_out = torch.empty_like(q_in)
        bt = c.block_tables
        if isinstance(c, Fp8PageCacheView):
            codes = {torch.float16: _native.DTYPE_F16, torch.bfloat16: _native.DTYPE_BF16,
                     torch.float32: _native.DTYPE_F32}
            if keys.dtype not in codes or values.dtype != keys.dtype or rope.dims % (4 if rope.traditional else 8):
                return None
            k, v = keys.contiguous(), values.contiguous()
            rc = lib.emx_fp8_cache_append_rope(
                k.data_ptr(), v.data_ptr(), codes[k.dtype], slots_d.data_ptr(), int(k.shape[0]), bt.data_ptr(),
                int(bt.shape[0]), int(bt.shape[1]), c.kv_lens.data_ptr(), counter.data_ptr(),
                c.num_kv_heads, c.head_dim, c.block_size, c.num_blocks, c.key_cache.data_ptr(),
                c.value_cache.data_ptr(), c.k_scales.data_ptr(), c.v_scales.data_ptr(),
                rope.inv_freq(k.device).data_ptr(), rope.dims, int(rope.traditional), q_in.data_ptr(),
                q_out.data_ptr(), int(q_out.shape[1]), stream)
            if rc == _native.EMX_ERR_UNSUPPORTED:
                return None
            _native.check(rc)
            return q_out
        k = keys if keys.dtype == torch.float16 and keys.is_contiguous() else keys.to(torch.float16).contiguous()
        v = values if values.dtype == torch.float16 and values.is_contiguous() else values.to(torch.float16).contiguous()
        rc = lib.emx_affine_cache_append_rope(
            k.data_ptr(), v.data_ptr(), slots_d.data_ptr(), int(k.shape[0]), bt.data_ptr(), int(bt.shape[0]),
            int(bt.shape[1]), c.kv_lens.data_ptr(), counter.data_ptr(), c.num_kv_heads, c.head_dim,
            c.group_size, c.bits, c.block_size, c.num_blocks, c.key_cache.data_ptr(), c.k_scales.data_ptr(),
            c.k_biases.data_ptr(), c.value_cache.data_ptr(), c.v_scales.data_ptr(), c.v_biases.data_ptr(),
            rope.inv_freq(k.device).data_ptr(), rope.dims, int(rope.traditional), q_in.data_ptr(), q_out.data_ptr(),
            int(q_out.shape[1]), stream)
        if rc == _native.EMX_ERR_UNSUPPORTED:
            return None
        _native.check(rc)
        return q_out

    def _write(self, queries, keys, values, mapping, positions, rope, lib, stream):
        from .rope import RotaryEmbedding

        c = self.cache
        n = int(mapping.shape[0])
        fused = isinstance(rope, RotaryEmbedding) and rope.dims <= c.head_dim and queries.dtype == torch.float16
        if isinstance(c, AffinePageCacheView):
            k = keys.to(torch.float16).contiguous()
            v = values.to(torch.float16).contiguous()
            if rope is None:
                c._write(k, v, mapping)
                return queries
            if fused:
                q_in = queries.contiguous()
                q_out = torch.empty_like(q_in)  # every row written by the launch, turned
                inv = rope.inv_freq(k.device)
                _native.check(lib.emx_affine_cache_write_rope(
                    k.data_ptr(), v.data_ptr(), mapping.data_ptr(), n, c.num_kv_heads, c.head_dim, c.group_size,
                    c.bits, c.block_size, c.num_blocks, c.key_cache.data_ptr(), c.k_scales.data_ptr(),
                    c.k_biases.data_ptr(), c.value_cache.data_ptr(), c.v_scales.data_ptr(), c.v_biases.data_ptr(),
                    positions.data_ptr(), inv.data_ptr(), rope.dims, int(rope.traditional), q_in.data_ptr(),
                    q_out.data_ptr(), int(q_out.shape[1]), stream))
                return q_out
        elif isinstance(c, Fp8PageCacheView):
            codes = {torch.float16: _native.DTYPE_F16, torch.bfloat16: _native.DTYPE_BF16,
                     torch.float32: _native.DTYPE_F32}
            if keys.dtype not in codes or values.dtype != keys.dtype:
                raise NotImplementedError(f"FP8 cache writes take fp16/bf16/fp32 keys and values, got {keys.dtype}")
            turn = fused and rope.dims % (4 if rope.traditional else 8) == 0
            if rope is None or turn:
                k, v = keys.contiguous(), values.contiguous()
                if turn:
                    q_in = queries.contiguous()
                    q_out = torch.empty_like(q_in)  # every row written by the launch, turned
                    inv = rope.inv_freq(k.device)
                    ws = self._fp8_workspace(lib, k.device)
                    _native.check(lib.emx_fp8_cache_write_rope(
                        k.data_ptr(), v.data_ptr(), codes[k.dtype], mapping.data_ptr(), n, c.num_kv_heads,
                        c.head_dim, c.block_size, c.num_blocks, c.key_cache.data_ptr(), c.value_cache.data_ptr(),
                        c.k_scales.data_ptr(), c.v_scales.data_ptr(), ws.data_ptr(), ws.numel(),
                        positions.data_ptr(), inv.data_ptr(), rope.dims, int(rope.traditional), q_in.data_ptr(),
                        q_out.data_ptr(), int(q_out.shape[1]), stream))
                    return q_out
                # the proxy's own workspace (the library's process-wide scratch would race with a
                # write on another stream)
                ws = self._fp8_workspace(lib, k.device)
                _native.check(lib.emx_fp8_cache_write(
                    k.data_ptr(), v.data_ptr(), codes[k.dtype], mapping.data_ptr(), n, c.num_kv_heads, c.head_dim,
                    c.block_size, c.num_blocks, c.key_cache.data_ptr(), c.value_cache.data_ptr(),
                    c.k_scales.data_ptr(), c.v_scales.data_ptr(), ws.data_ptr(), ws.numel(), stream))
                return queries
        elif rope is None:
            c._write(keys, values, mapping)
            return queries
        # any other RoPE: Q and K turned first (the reference's order, model_runner.py:163-169),
        # with the device positions as offsets
        q_out, k_out = self._turn(rope, queries, keys, positions, fused, lib, stream)
        if isinstance(c, Fp8PageCacheView):
            return self._write(q_out, k_out, values, mapping, positions, None, lib, stream)
        c._write(k_out, values, mapping)
        return q_out

    def _turn(self, rope, queries, keys, positions, fused, lib, stream):
        if fused and keys.dtype == torch.float16:
            q_out = queries.contiguous().clone()
            k_out = keys.contiguous().clone()
            inv = rope.inv_freq(q_out.device)
            for x in (q_out, k_out):
                _native.check(lib.emx_rope_rows(x.data_ptr(), int(x.shape[0]), int(x.shape[1]), self.head_dim,
                                                positions.data_ptr(), inv.data_ptr(), rope.dims,
                                                int(rope.traditional), stream))
            return q_out, k_out
        qb = queries.unsqueeze(1).transpose(1, 2)
        kb = keys.unsqueeze(1).transpose(1, 2)
        return (rope(qb, offset=positions).transpose(1, 2)[:, 0], rope(kb, offset=positions).transpose(1, 2)[:, 0])

    def _fp8_workspace(self, lib, device) -> torch.Tensor:
        if self._fp8_ws is None:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("CompiledPagedCacheProxy: run one eager step before capture")
            self._fp8_ws = torch.empty(int(lib.emx_fp8_write_workspace_bytes()), dtype=torch.uint8, device=device)
        return self._fp8_ws


__all__ = ("CompiledPagedCacheProxy",)
