"""Seeded synthetic workloads for the paged-attention configurations.

One ``numpy.random.default_rng(seed)`` per workload; draws happen in a fixed
order -- lengths, per-channel gains, values (q, k, v), page permutation -- so a
seed fully determines the inputs.  K/V tokens are returned in *logical* order
(sequence-major, ``[num_tokens, Hkv, D]`` fp16) together with the slot each
token occupies in the page pool; the caller quantizes/writes them.

Configurations (``name`` -> shape):

* ``c0`` plumbing: S=1, Hq 32 / Hkv 8, D 64, page 128, ctx 1024, fp16 KV,
  values N(0,1)/sqrt(D), table = seeded permutation of a 64-page pool.
* ``c1`` / ``c2``: batch 32, Hq 32 / Hkv 8, D 128, page 128, ctx ~ U[512, 4096],
  K/V = N(0,1) x per-(kv_head, channel) gain U[0.5, 4]; pool = sum of pages,
  random page assignment.  c1 is 8-bit, c2 4-bit (group 64).
* ``c3`` unified: 4 prefill chunks of 512 (prior cached ~ U[0, 2048]) + 28
  decode rows (ctx ~ U[256, 4096]), 4-bit.
* ``c4`` long context: S=8, Hq 64 / Hkv 8, ctx 32768 each, 4096-page pool, 4-bit.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass
class Workload:
    name: str
    seed: int
    q: np.ndarray              # [T, Hq, D] fp16
    k: np.ndarray              # [N, Hkv, D] fp16, logical tokens of all sequences
    v: np.ndarray              # [N, Hkv, D] fp16
    slot: np.ndarray           # [N] int64, block * bs + offset of each token
    kv_lens: np.ndarray        # [S] int32
    query_start_loc: np.ndarray  # [S+1] int32
    block_tables: np.ndarray   # [S, max_blocks] int32
    num_blocks: int
    block_size: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    bits: int | None = 4
    group_size: int = 64
    single_token_decode: bool = True
    extra: dict = field(default_factory=dict)

    @property
    def num_seqs(self) -> int:
        return int(self.kv_lens.shape[0])

    def kv_bytes(self) -> int:
        """Algorithmic K/V bytes one decode step reads (codes + scale/bias, or fp16)."""
        d, g = self.head_dim, self.group_size
        if self.bits is None:
            per_tok_head = 2 * d * 2
        else:
            per_tok_head = 2 * (d * self.bits // 8 + (d // g) * 4)
        return int(self.kv_lens.astype(np.int64).sum()) * self.num_kv_heads * per_tok_head

    def logical_cache(self, dtype=np.float16):
        """Scatter K/V tokens into logical ``[num_blocks, bs, Hkv, D]`` arrays."""
        shape = (self.num_blocks, self.block_size, self.num_kv_heads, self.head_dim)
        kc = np.zeros(shape, dtype=dtype)
        vc = np.zeros(shape, dtype=dtype)
        b, o = self.slot // self.block_size, self.slot % self.block_size
        kc[b, o] = self.k
        vc[b, o] = self.v
        return kc, vc


def _assign_pages(rng, lens, bs, pool_pages):
    pages = [int(-(-int(n) // bs)) for n in lens]
    max_blocks = max(pages) if pages else 1
    need = sum(pages)
    pool = max(pool_pages or 0, need)
    perm = rng.permutation(pool).astype(np.int32)
    tables = np.full((len(lens), max_blocks), -1, dtype=np.int32)
    at = 0
    for i, n in enumerate(pages):
        tables[i, :n] = perm[at : at + n]
        at += n
    return tables, pool


def _slots(lens, tables, bs):
    out = []
    for i, n in enumerate(lens):
        pos = np.arange(int(n))
        out.append(tables[i, pos // bs].astype(np.int64) * bs + pos % bs)
    return np.concatenate(out) if out else np.zeros((0,), np.int64)


def _values(rng, n, hkv, d, gain):
    x = rng.standard_normal((n, hkv, d), dtype=np.float32)
    if gain is not None:
        x *= gain[None]
    return x.astype(np.float16)


def decode_workload(
    name: str = "custom",
    *,
    seed: int = 0,
    num_seqs: int = 32,
    num_q_heads: int = 32,
    num_kv_heads: int = 8,
    head_dim: int = 128,
    block_size: int = 128,
    ctx_range: tuple[int, int] = (512, 4096),
    fixed_ctx: int | None = None,
    pool_pages: int | None = None,
    bits: int | None = 4,
    group_size: int = 64,
    gains: bool = True,
    value_scale: float = 1.0,
) -> Workload:
    """Batched single-token decode: one query token per sequence."""
    rng = np.random.default_rng(seed)
    if fixed_ctx is not None:
        lens = np.full((num_seqs,), fixed_ctx, dtype=np.int32)
    else:
        lens = rng.integers(ctx_range[0], ctx_range[1] + 1, size=num_seqs).astype(np.int32)
    gk = gv = None
    if gains:
        gk = rng.uniform(0.5, 4.0, size=(num_kv_heads, head_dim)).astype(np.float32)
        gv = rng.uniform(0.5, 4.0, size=(num_kv_heads, head_dim)).astype(np.float32)
    n = int(lens.sum())
    q = rng.standard_normal((num_seqs, num_q_heads, head_dim), dtype=np.float32)
    k = _values(rng, n, num_kv_heads, head_dim, gk)
    v = _values(rng, n, num_kv_heads, head_dim, gv)
    if value_scale != 1.0:
        q *= value_scale
        k = (k.astype(np.float32) * value_scale).astype(np.float16)
        v = (v.astype(np.float32) * value_scale).astype(np.float16)
    tables, pool = _assign_pages(rng, lens, block_size, pool_pages)
    return Workload(
        name=name,
        seed=seed,
        q=q.astype(np.float16),
        k=k,
        v=v,
        slot=_slots(lens, tables, block_size),
        kv_lens=lens,
        query_start_loc=np.arange(num_seqs + 1, dtype=np.int32),
        block_tables=tables,
        num_blocks=pool,
        block_size=block_size,
        num_q_heads=num_q_heads,
        num_kv_heads=num_kv_heads,
        head_dim=head_dim,
        bits=bits,
        group_size=group_size,
        single_token_decode=True,
    )


def unified_workload(
    name: str = "c3",
    *,
    seed: int = 3,
    num_prefill: int = 4,
    chunk: int = 512,
    prior_range: tuple[int, int] = (0, 2048),
    num_decode: int = 28,
    decode_ctx: tuple[int, int] = (256, 4096),
    num_q_heads: int = 32,
    num_kv_heads: int = 8,
    head_dim: int = 128,
    block_size: int = 128,
    bits: int | None = 4,
    group_size: int = 64,
) -> Workload:
    """Ragged step: prefill chunks (causal inside the chunk) followed by decode rows."""
    rng = np.random.default_rng(seed)
    prior = rng.integers(prior_range[0], prior_range[1] + 1, size=num_prefill)
    dctx = rng.integers(decode_ctx[0], decode_ctx[1] + 1, size=num_decode)
    lens = np.concatenate([prior + chunk, dctx]).astype(np.int32)
    qlens = np.concatenate([np.full(num_prefill, chunk), np.ones(num_decode, dtype=np.int64)])
    n = int(lens.sum())
    t = int(qlens.sum())
    q = rng.standard_normal((t, num_q_heads, head_dim), dtype=np.float32).astype(np.float16)
    k = _values(rng, n, num_kv_heads, head_dim, None)
    v = _values(rng, n, num_kv_heads, head_dim, None)
    tables, pool = _assign_pages(rng, lens, block_size, None)
    qsl = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    return Workload(
        name=name,
        seed=seed,
        q=q,
        k=k,
        v=v,
        slot=_slots(lens, tables, block_size),
        kv_lens=lens,
        query_start_loc=qsl,
        block_tables=tables,
        num_blocks=pool,
        block_size=block_size,
        num_q_heads=num_q_heads,
        num_kv_heads=num_kv_heads,
        head_dim=head_dim,
        bits=bits,
        group_size=group_size,
        single_token_decode=False,
    )


def config(name: str, seed: int | None = None) -> Workload:
    """The named BASELINE configuration at full size."""
    if name == "c0":
        rng = np.random.default_rng(0 if seed is None else seed)
        d, hq, hkv, bs, ctx = 64, 32, 8, 128, 1024
        sc = np.float32(1.0 / np.sqrt(d))
        q = (rng.standard_normal((1, hq, d), dtype=np.float32) * sc).astype(np.float16)
        k = (rng.standard_normal((ctx, hkv, d), dtype=np.float32) * sc).astype(np.float16)
        v = (rng.standard_normal((ctx, hkv, d), dtype=np.float32) * sc).astype(np.float16)
        perm = rng.permutation(64).astype(np.int32)
        tables = perm[: ctx // bs][None].copy()
        lens = np.array([ctx], dtype=np.int32)
        return Workload("c0", 0 if seed is None else seed, q, k, v, _slots(lens, tables, bs), lens,
                        np.array([0, 1], np.int32), tables, 64, bs, hq, hkv, d, bits=None, group_size=64)
    if name == "c1":
        return decode_workload("c1", seed=1 if seed is None else seed, bits=8)
    if name == "c2":
        return decode_workload("c2", seed=2 if seed is None else seed, bits=4)
    if name == "c3":
        return unified_workload("c3", seed=3 if seed is None else seed)
    if name == "c4":
        return decode_workload("c4", seed=4 if seed is None else seed, num_seqs=8, num_q_heads=64, fixed_ctx=32768,
                               pool_pages=4096, bits=4)
    raise KeyError(name)
