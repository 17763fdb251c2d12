"""Restatement of the reference's paged-attention semantics (TEST INFRASTRUCTURE ONLY).

Follows ``_paged_attention_reference``
(``lib/python/easymlx/operations/kernels/unified_attention.py:187-281``; test
copy ``tests/operations/test_unified_attention.py:22-83``) with the edge
semantics of the Metal kernels the product path replaces:

* GQA: ``kv_head = q_head // (Hq // Hkv)`` clamped to ``Hkv-1``
  (``unified_attention.py:318-325``).
* q is scaled by ``softmax_scale`` in fp32 before the dot product (``:388``).
* causal limit ``max_k = min(seq_len-1, (seq_len - q_len) + q_pos)``
  (``:357-361``); sliding window ``start_k = max(0, max_k - window + 1)``
  (``:369-376``).
* ``q_len <= 0`` / ``seq_len <= 0`` / ``max_k < 0`` rows produce zeros
  (``:341-365``); ``l == 0`` produces zeros (``:457``).
* Pages whose block id is ``< 0`` are skipped by the Metal kernels (``:402-404``)
  while the NumPy reference keeps zero keys in the softmax (``:248-254``).
  ``invalid_block="skip"`` (default) follows the kernels; ``"zero"`` follows
  the NumPy reference.  Block ids ``>= num_blocks`` are treated the same way.
"""

from __future__ import annotations

import numpy as np


def gather_sequence(cache: np.ndarray, table_row: np.ndarray, seq_len: int):
    """Gather ``[seq_len, Hkv, D]`` from a logical ``[nb, bs, Hkv, D]`` cache.

    Returns ``(values float64/32, valid bool[seq_len])``; positions whose
    block id is out of range are zero and flagged invalid
    (``unified_attention.py:246-254``).
    """
    nb, bs = cache.shape[0], cache.shape[1]
    pos = np.arange(seq_len)
    blocks = np.asarray(table_row)[pos // bs].astype(np.int64)
    valid = (blocks >= 0) & (blocks < nb)
    safe = np.where(valid, blocks, 0)
    out = cache[safe, pos % bs]
    out = np.where(valid[:, None, None], out, 0)
    return out, valid


def paged_attention(
    queries: np.ndarray,
    key_cache: np.ndarray,
    value_cache: np.ndarray,
    block_tables: np.ndarray,
    kv_lens: np.ndarray,
    query_start_loc: np.ndarray,
    *,
    softmax_scale: float | None = None,
    sliding_window: int = 0,
    invalid_block: str = "skip",
    compute_dtype=np.float32,
    out_dtype=None,
) -> np.ndarray:
    """Paged (unified, ragged, causal) attention over a logical block cache.

    Args:
        queries: ``[T, Hq, D]``.
        key_cache, value_cache: logical ``[num_blocks, block_size, Hkv, D]``.
        block_tables: ``[S, max_blocks]`` int.
        kv_lens: ``[S]`` int, KV length including this step's tokens.
        query_start_loc: ``[S+1]`` int.

    Returns:
        ``[T, Hq, D]`` in ``out_dtype`` (default: the queries' dtype).
    """
    q_all = np.asarray(queries)
    total_tokens, hq, d = q_all.shape
    hkv = key_cache.shape[2]
    if hq % hkv != 0:
        raise ValueError("num_q_heads must be divisible by num_kv_heads (GQA)")
    group = hq // hkv
    if softmax_scale is None:
        softmax_scale = 1.0 / np.sqrt(d)
    bt = np.asarray(block_tables)
    kv = np.asarray(kv_lens)
    qsl = np.asarray(query_start_loc)
    out = np.zeros((total_tokens, hq, d), dtype=compute_dtype)
    kv_head_of = np.minimum(np.arange(hq) // group, hkv - 1)

    for s in range(bt.shape[0]):
        q_start, q_end = int(qsl[s]), int(qsl[s + 1])
        q_len = q_end - q_start
        seq_len = int(kv[s])
        if q_len <= 0 or seq_len <= 0:
            continue
        k_seq, valid = gather_sequence(key_cache, bt[s], seq_len)
        v_seq, _ = gather_sequence(value_cache, bt[s], seq_len)
        k_seq = k_seq.astype(compute_dtype)[:, kv_head_of]  # [L, Hq, D]
        v_seq = v_seq.astype(compute_dtype)[:, kv_head_of]
        q = q_all[q_start:q_end].astype(compute_dtype) * compute_dtype(softmax_scale)  # [q_len, Hq, D]

        q_pos = np.arange(q_len)
        max_k = np.minimum(seq_len - 1, (seq_len - q_len) + q_pos)  # [q_len]
        start_k = np.zeros_like(max_k)
        if sliding_window and sliding_window > 0:
            start_k = np.maximum(0, max_k - sliding_window + 1)
        kpos = np.arange(seq_len)
        mask = (kpos[None, :] <= max_k[:, None]) & (kpos[None, :] >= start_k[:, None])
        if invalid_block == "skip":
            mask &= valid[None, :]
        # batched matmuls over heads (BLAS) instead of einsum: same sums, faster at full sizes
        scores = np.matmul(q.transpose(1, 0, 2), k_seq.transpose(1, 2, 0)).transpose(1, 0, 2)  # [q, h, k]
        scores = np.where(mask[:, None, :], scores, -np.inf)
        row_max = scores.max(axis=-1, keepdims=True)
        has_any = np.isfinite(row_max)
        w = np.exp(scores - np.where(has_any, row_max, 0))
        w = np.where(mask[:, None, :], w, 0)
        l = w.sum(axis=-1, keepdims=True)
        o = np.matmul(w.transpose(1, 0, 2), v_seq.transpose(1, 0, 2)).transpose(1, 0, 2)  # [q, h, d]
        o = np.where(l > 0, o / np.where(l > 0, l, 1), 0)
        o = np.where((max_k >= 0)[:, None, None], o, 0)
        out[q_start:q_end] = o
    return out.astype(out_dtype if out_dtype is not None else q_all.dtype)


def merge_partials(m: np.ndarray, l: np.ndarray, o: np.ndarray) -> np.ndarray:
    """Split-K merge (``page_attention.py:2006-2059``).

    Args:
        m: ``[P, ...]`` per-partition max logit (``-inf`` for empty partitions).
        l: ``[P, ...]`` per-partition exp-sum.
        o: ``[P, ..., D]`` per-partition *unnormalised* accumulator.
    """
    gm = m.max(axis=0)
    finite = np.isfinite(gm)
    w = np.where(l > 0, np.exp(m - np.where(finite, gm, 0)), 0)
    gl = (w * l).sum(axis=0)
    acc = (w[..., None] * o).sum(axis=0)
    return np.where(gl[..., None] > 0, acc / np.where(gl > 0, gl, 1)[..., None], 0)


def causal_single_sequence(query, keys, values, past_len: int, softmax_scale=None, sliding_window=0):
    """Dense single-sequence causal attention (``page_attention.py:84-133``).

    ``query [q_len, Hq, D]``, ``keys/values [kv_len, Hkv, D]`` (already
    gathered); masks with ``-1e9`` like the reference.
    """
    q_len, hq, d = query.shape
    kv_len, hkv, _ = keys.shape
    rep = hq // hkv
    k = np.repeat(keys.astype(np.float32), rep, axis=1)
    v = np.repeat(values.astype(np.float32), rep, axis=1)
    scale = softmax_scale if softmax_scale is not None else d ** -0.5
    scores = np.einsum("qhd,khd->hqk", query.astype(np.float32), k) * np.float32(scale)
    kpos = np.arange(kv_len)
    maxp = past_len + np.arange(q_len)
    mask = kpos[None, :] <= maxp[:, None]
    if sliding_window:
        minp = np.maximum(maxp - sliding_window + 1, 0)
        mask &= kpos[None, :] >= minp[:, None]
    scores = np.where(mask[None], scores, np.float32(-1e9))
    scores = scores - scores.max(axis=-1, keepdims=True)
    p = np.exp(scores)
    p = p / p.sum(axis=-1, keepdims=True)
    return np.einsum("hqk,khd->qhd", p, v).astype(query.dtype)
