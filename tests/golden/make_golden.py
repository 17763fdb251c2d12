"""Regenerate the golden fixtures in this directory.

Inputs are the reference tests' own seeded draws, reproduced bit-exactly with
numpy's PCG64 in the same order as the reference test code:

* ``attn_rng0.npz``  -- ``test_paged_attention_reference_matches``
  (``tests/operations/test_unified_attention.py:86-145``): rng(0), 2 seqs,
  Hq 2 / Hkv 1, D 4, bs 4, seq_lens [5, 3], query_lens [2, 1], fp32.
* ``attn_rng1.npz``  -- ``test_paged_attention_metal_matches_reference`` (``:148-208``):
  rng(1), Hq 4 / Hkv 2, D 8, bs 4, seq_lens [6, 4], query_lens [2, 1].
* ``attn_rng11.npz`` -- ``test_paged_attention_metal_decode_fast_path_matches_reference``
  (``:211-265``): rng(11), seq_lens [5, 7, 3], query_lens [1, 1, 1].
* ``write_rng2.npz`` -- ``test_page_cache_concatenate_to_cache_updates_multiple_slots``
  (``:268-345``): rng(2), initial_lens [1, 0, 2], query_lens [2, 0, 3].
* ``write_rng7.npz`` -- ``test_page_cache_single_token_decode_fast_path_applies_rope_and_updates_cache``
  (``:348-415``): rng(7), initial_lens [2, 1, 3], one decode token each.

The reference's ``PageCacheView.allocate`` gives each sequence
``ceil(max_seq_len / bs)`` consecutive blocks (``cache.py:779-786``) and
``append`` writes token ``p`` at ``[table[p // bs], p % bs]`` (``cache.py:851-866``).
Expected attention outputs come from ``oracle.paged_attention`` in float64
(cross-checked in ``tests/test_oracle_attention.py`` against
``torch.nn.functional.scaled_dot_product_attention``); expected write
positions come from ``oracle.cache_write``.

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.cache_write import build_query_start_loc, write_positions  # noqa: E402
from oracle.paged_attention import paged_attention  # noqa: E402


def _alloc(num_seqs, max_seq_len, hkv, d, bs):
    bps = math.ceil(max_seq_len / bs)
    nb = bps * num_seqs
    tables = np.arange(nb, dtype=np.int32).reshape(num_seqs, bps)
    kc = np.zeros((nb, bs, hkv, d), np.float32)
    vc = np.zeros((nb, bs, hkv, d), np.float32)
    return tables, kc, vc


def _append(tables, kc, vc, kv_lens, seq, k, v, bs):
    start = int(kv_lens[seq])
    for i in range(k.shape[0]):
        p = start + i
        b = tables[seq, p // bs]
        kc[b, p % bs] = k[i]
        vc[b, p % bs] = v[i]
    kv_lens[seq] = start + k.shape[0]


def attention_case(seed, hq, hkv, d, bs, seq_lens, query_lens, decode_queries=False):
    rng = np.random.default_rng(seed)
    tables, kc, vc = _alloc(len(seq_lens), max(seq_lens), hkv, d, bs)
    kv_lens = np.zeros(len(seq_lens), np.int32)
    for s, n in enumerate(seq_lens):
        k = rng.standard_normal((n, hkv, d)).astype(np.float32)
        v = rng.standard_normal((n, hkv, d)).astype(np.float32)
        _append(tables, kc, vc, kv_lens, s, k, v, bs)
    if decode_queries:
        queries = rng.standard_normal((len(seq_lens), hq, d)).astype(np.float32)
    else:
        queries = np.concatenate(
            [rng.standard_normal((q, hq, d)).astype(np.float32) for q in query_lens], axis=0
        )
    qsl = build_query_start_loc(query_lens)
    scale = 1.0 / np.sqrt(d)
    expected = paged_attention(queries.astype(np.float64), kc.astype(np.float64), vc.astype(np.float64), tables,
                               kv_lens, qsl, softmax_scale=scale, sliding_window=0, compute_dtype=np.float64,
                               out_dtype=np.float64)
    return dict(queries=queries, key_cache=kc, value_cache=vc, block_tables=tables, kv_lens=kv_lens,
                query_start_loc=qsl, softmax_scale=np.float64(scale), expected=expected, seed=np.int64(seed))


def write_case(seed, initial_lens, query_lens, hq=2, hkv=1, d=4, bs=4, max_seq_len=8, decode=False):
    rng = np.random.default_rng(seed)
    tables, kc, vc = _alloc(3, max_seq_len, hkv, d, bs)
    kv_lens = np.zeros(3, np.int32)
    for s, n in enumerate(initial_lens):
        if n == 0 and not decode:
            continue
        k = rng.standard_normal((n, hkv, d)).astype(np.float32)
        v = rng.standard_normal((n, hkv, d)).astype(np.float32)
        _append(tables, kc, vc, kv_lens, s, k, v, bs)
    total = int(sum(query_lens))
    queries = rng.standard_normal((total, hq, d)).astype(np.float32)
    keys = rng.standard_normal((total, hkv, d)).astype(np.float32)
    values = rng.standard_normal((total, hkv, d)).astype(np.float32)
    qsl = build_query_start_loc(query_lens)
    slot_mapping, new_lens = write_positions(tables, kv_lens, qsl, [0, 1, 2], bs)
    return dict(key_cache=kc, value_cache=vc, block_tables=tables, kv_lens=kv_lens, queries=queries, keys=keys,
                values=values, query_start_loc=qsl, slot_mapping=slot_mapping, expected_kv_lens=new_lens.astype(np.int32),
                seed=np.int64(seed))


def main() -> None:
    cases = {
        "attn_rng0.npz": attention_case(0, 2, 1, 4, 4, [5, 3], [2, 1]),
        "attn_rng1.npz": attention_case(1, 4, 2, 8, 4, [6, 4], [2, 1]),
        "attn_rng11.npz": attention_case(11, 4, 2, 8, 4, [5, 7, 3], [1, 1, 1], decode_queries=True),
        "write_rng2.npz": write_case(2, [1, 0, 2], [2, 0, 3]),
        "write_rng7.npz": write_case(7, [2, 1, 3], [1, 1, 1], decode=True),
    }
    for name, arrays in cases.items():
        np.savez(os.path.join(HERE, name), **arrays)
        print("wrote", name)


if __name__ == "__main__":
    main()
