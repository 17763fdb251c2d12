"""Write-position arithmetic of the paged cache (TEST INFRASTRUCTURE ONLY).

Restates ``PageCacheView.concatenate_to_cache``
(``lib/python/easymlx/caching/paged/cache.py:1088-1306``) and
``build_query_start_loc`` (``cache.py:1448-1465``) without the storage format:

* a sequence ``i`` scheduled in slot ``slot_ids[i]`` contributes tokens
  ``[qsl[i], qsl[i+1])`` (``:1127-1140``);
* token ``j`` of it is written at position ``pos = kv_lens[slot] + j``
  (``:1155``, ``:1254``), block ``block_tables[slot, pos // bs]``, in-block
  offset ``pos % bs`` (``:1168-1169``, ``:1256-1257``);
* the flat ``slot_mapping = block * bs + offset`` (``:1259``);
* afterwards ``kv_lens[slot] += q_len`` (``:1199``, ``:1297``);
* page lifecycle: copy-on-write block copies (``:944-972``) and the runner's
  page zeroing (``model_runner.py:1058-1094``), both over every array of a
  cache.
"""

from __future__ import annotations

import numpy as np


def build_query_start_loc(query_lens) -> np.ndarray:
    """``cache.py:1448-1465``: cumulative offsets starting at zero (int32)."""
    out = [0]
    for n in query_lens:
        out.append(out[-1] + int(n))
    return np.asarray(out, dtype=np.int32)


def write_positions(block_tables, kv_lens, query_start_loc, slot_ids, block_size: int):
    """Return ``(slot_mapping int64[T], new_kv_lens)`` for one write step.

    Tokens whose block id is negative get ``slot_mapping = -1`` (not written),
    matching ``PageCacheView.append``'s skip of ``block < 0`` (``cache.py:859-861``).
    A position past the end of the block table is also skipped: the reference
    gathers ``block_tables[slot, pos // bs]`` unchecked (``cache.py:1168``), where
    MLX's out-of-range gather is unspecified, so no value there is pinned.
    """
    bt = np.asarray(block_tables)
    kv = np.asarray(kv_lens).astype(np.int64).copy()
    qsl = np.asarray(query_start_loc)
    total = int(qsl[len(slot_ids)]) if len(slot_ids) else 0
    slot_mapping = np.full((total,), -1, dtype=np.int64)
    for i, slot in enumerate(slot_ids):
        start, end = int(qsl[i]), int(qsl[i + 1])
        base = int(kv[slot])
        for j in range(max(0, end - start)):
            pos = base + j
            col = pos // block_size
            block = int(bt[slot, col]) if col < bt.shape[1] else -1
            if block >= 0:
                slot_mapping[start + j] = block * block_size + pos % block_size
        kv[slot] = base + max(0, end - start)
    return slot_mapping, kv


def copy_blocks(arrays, block_mapping):
    """Copy-on-write block copies (``cache.py:944-972``, Metal kernel ``:95-136``), in place on numpy arrays
    indexed by block first: for each row ``(src, dst)``, block ``dst`` of every array becomes block ``src`` as it
    was before the call (the kernel reads its input arrays).  Ids outside ``[0, num_blocks)`` are skipped."""
    before = [np.array(a, copy=True) for a in arrays]
    for src, dst in np.asarray(block_mapping).reshape(-1, 2).tolist():
        for a, b in zip(arrays, before):
            nb = a.shape[0]
            if 0 <= src < nb and 0 <= dst < nb:
                a[dst] = b[src]


def zero_pages(arrays, page_ids):
    """The runner's ``_zero_pages`` (``model_runner.py:1058-1094``): the listed pages of every array become zero;
    negative ids (and ids past the pool) are skipped."""
    for a in arrays:
        for p in np.asarray(page_ids).reshape(-1).tolist():
            if 0 <= p < a.shape[0]:
                a[p] = 0
