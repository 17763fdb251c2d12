"""Host-side conversions between the MLX-style logical affine KV layout and pages.

Logical layout (what ``mlx.core.quantize`` of a ``[tokens, Hkv, D]`` K/V
tensor gives, scattered into ``[num_blocks, block_size, ...]`` like the
reference's dense cache ``lib/python/easymlx/caching/paged/cache.py:790-791``):

    codes  uint32 [nb, bs, Hkv, D*bits/32]
    scales fp16   [nb, bs, Hkv, D/gs]        (biases likewise)

Page layout used by the kernels (see ``include/emx_attn.h``):

    key codes    uint32 [nb, Hkv, bs, D*bits/32]   token-major
    value codes  uint32 [nb, Hkv, bs/T, D, T*bits/32]   T = min(bs, 256/bits) tokens per tile,
                                                     dim-major inside a tile (tokens packed along a word)
    scales       fp16   [nb, Hkv, D/gs, bs]         (biases likewise)

NumPy only; used to build pages from host data and to read pages back.
"""

from __future__ import annotations

import numpy as np


def _unpack(words: np.ndarray, bits: int) -> np.ndarray:
    per = 32 // bits
    sh = (np.arange(per, dtype=np.uint32) * np.uint32(bits)).astype(np.uint32)
    q = (words.astype(np.uint32)[..., None] >> sh) & np.uint32((1 << bits) - 1)
    return q.reshape(*words.shape[:-1], words.shape[-1] * per)


def _pack(q: np.ndarray, bits: int) -> np.ndarray:
    per = 32 // bits
    q = q.astype(np.uint32).reshape(*q.shape[:-1], q.shape[-1] // per, per)
    sh = (np.arange(per, dtype=np.uint32) * np.uint32(bits)).astype(np.uint32)
    return np.bitwise_or.reduce(q << sh, axis=-1).astype(np.uint32)


def key_pages_from_logical(codes: np.ndarray) -> np.ndarray:
    """``[nb, bs, Hkv, W]`` -> ``[nb, Hkv, bs, W]``."""
    return np.ascontiguousarray(np.asarray(codes, dtype=np.uint32).transpose(0, 2, 1, 3))


def key_logical_from_pages(pages: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(pages).view(np.uint32).transpose(0, 2, 1, 3))


def value_tile(block_size: int, bits: int) -> int:
    """Tokens per value tile: ``min(block_size, 256 // bits)``."""
    return min(block_size, 256 // bits)


# 4-bit value words interleave their eight tokens: token k sits at nibble
# (k >> 1) | ((k & 1) << 2), i.e. nibble n holds token _V4_TOKEN_AT[n].
_V4_TOKEN_AT = np.array([0, 2, 4, 6, 1, 3, 5, 7])
_V4_NIBBLE_OF = np.array([0, 4, 1, 5, 2, 6, 3, 7])


def value_pages_from_logical(codes: np.ndarray, bits: int) -> np.ndarray:
    """``[nb, bs, Hkv, W]`` -> ``[nb, Hkv, bs/T, D, T*bits/32]`` (tokens packed per word;
    4-bit words in the interleaved token order above, 8-bit words in byte order)."""
    q = _unpack(np.asarray(codes, dtype=np.uint32), bits)  # [nb, bs, Hkv, D]
    nb, bs, hkv, d = q.shape
    t = value_tile(bs, bits)
    q = q.reshape(nb, bs // t, t, hkv, d).transpose(0, 3, 1, 4, 2)  # [nb, Hkv, bs/T, D, T]
    if bits == 4:
        q = q.reshape(*q.shape[:-1], t // 8, 8)[..., _V4_TOKEN_AT].reshape(q.shape)
    return np.ascontiguousarray(_pack(q, bits))


def value_logical_from_pages(pages: np.ndarray, bits: int) -> np.ndarray:
    q = _unpack(np.asarray(pages).view(np.uint32), bits)  # [nb, Hkv, bs/T, D, T]
    nb, hkv, nt, d, t = q.shape
    if bits == 4:
        q = q.reshape(*q.shape[:-1], t // 8, 8)[..., _V4_NIBBLE_OF].reshape(q.shape)
    q = q.transpose(0, 2, 4, 1, 3).reshape(nb, nt * t, hkv, d)  # [nb, bs, Hkv, D]
    return np.ascontiguousarray(_pack(q, bits))


def params_pages_from_logical(p: np.ndarray) -> np.ndarray:
    """scales/biases ``[nb, bs, Hkv, G]`` -> ``[nb, Hkv, G, bs]``."""
    return np.ascontiguousarray(np.asarray(p).transpose(0, 2, 3, 1))


def params_logical_from_pages(p: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(p).transpose(0, 3, 1, 2))
