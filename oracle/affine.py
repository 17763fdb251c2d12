"""Restatement of MLX's affine quantize / dequantize (TEST INFRASTRUCTURE ONLY).

Third-party dependency: ``mlx`` (Apple, MIT), pinned ``mlx==0.31.1`` by the
reference (``uv.lock:319-320``).  The reference calls it as
``mx.quantize(w, group_size=g, bits=b)`` / ``mx.dequantize(w, scales, biases,
group_size=g, bits=b)`` (``lib/python/easymlx/infra/mixins/bridge.py:304,361``,
``lib/python/easymlx/layers/linears/_linear_moe.py:113,297``; format described
in ``lib/python/easymlx/infra/etils.py:74-94``).

Algorithm (MLX CPU backend, per group of ``g`` contiguous elements along the
last axis, all arithmetic in IEEE fp32, ``rint`` = round-half-to-even)::

    w_max, w_min   = max/min of the group (fp32)
    n_bins         = 2**bits - 1
    mask           = |w_min| > |w_max|
    scale          = max((w_max - w_min) / n_bins, 1e-7)
    scale          = mask ? scale : -scale
    edge           = mask ? w_min : w_max
    q0             = rint(edge / scale)
    if q0 != 0:      scale = edge / q0 ; bias = edge
    else:            bias  = 0
    code_i         = clip(rint((w_i - bias) / scale), 0, n_bins)
    scales, biases = cast(scale / bias -> input dtype)      # after quantizing

Codes are packed little-endian into uint32: element ``j`` of a word occupies
bits ``[j*bits, (j+1)*bits)`` (8 per word at 4-bit, 4 at 8-bit).

Parity status: **unpinned against a real MLX install** (not importable in this
environment).  Pinned instead by the invariant tests in
``tests/test_oracle_affine.py`` and by agreement with the independent C
restatement ``oracle/c/oracle.c``.
"""

from __future__ import annotations

import numpy as np

_EPS = np.float32(1e-7)


def _check(d: int, group_size: int, bits: int) -> None:
    if bits not in (4, 8):
        raise ValueError(f"bits must be 4 or 8, got {bits}")
    if group_size <= 0 or d % group_size != 0:
        raise ValueError(f"last dim {d} must be a multiple of group_size {group_size}")
    if (d * bits) % 32 != 0:
        raise ValueError("last dim * bits must be a multiple of 32")


def affine_quantize(w: np.ndarray, group_size: int = 64, bits: int = 4):
    """``mx.quantize(w, group_size, bits, mode="affine")`` restated.

    Args:
        w: ``[..., D]`` float16 / float32 array.

    Returns:
        ``(codes uint32 [..., D*bits/32], scales [..., D/g], biases [..., D/g])``
        with scales/biases in ``w.dtype``.
    """
    w = np.asarray(w)
    d = w.shape[-1]
    _check(d, group_size, bits)
    lead = w.shape[:-1]
    wf = w.astype(np.float32).reshape(-1, d // group_size, group_size)
    n_bins = np.float32((1 << bits) - 1)

    w_max = wf.max(axis=-1)
    w_min = wf.min(axis=-1)
    mask = np.abs(w_min) > np.abs(w_max)
    scale = np.maximum((w_max - w_min) / n_bins, _EPS).astype(np.float32)
    scale = np.where(mask, scale, -scale).astype(np.float32)
    edge = np.where(mask, w_min, w_max).astype(np.float32)
    q0 = np.rint(edge / scale).astype(np.float32)
    nz = q0 != 0
    safe_q0 = np.where(nz, q0, np.float32(1)).astype(np.float32)
    scale = np.where(nz, edge / safe_q0, scale).astype(np.float32)
    bias = np.where(nz, edge, np.float32(0)).astype(np.float32)

    q = np.rint((wf - bias[..., None]) / scale[..., None]).astype(np.float32)
    q = np.clip(q, np.float32(0), n_bins).astype(np.uint32)

    per_word = 32 // bits
    q = q.reshape(q.shape[0], -1, per_word)
    shifts = (np.arange(per_word, dtype=np.uint32) * np.uint32(bits)).astype(np.uint32)
    codes = np.bitwise_or.reduce(q << shifts, axis=-1).astype(np.uint32)

    codes = codes.reshape(*lead, d * bits // 32)
    scales = scale.astype(w.dtype).reshape(*lead, d // group_size)
    biases = bias.astype(w.dtype).reshape(*lead, d // group_size)
    return codes, scales, biases


def unpack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """Unpack little-endian uint32 words into integer codes ``[..., W*32/bits]``."""
    codes = np.asarray(codes, dtype=np.uint32)
    per_word = 32 // bits
    shifts = (np.arange(per_word, dtype=np.uint32) * np.uint32(bits)).astype(np.uint32)
    mask = np.uint32((1 << bits) - 1)
    q = (codes[..., None] >> shifts) & mask
    return q.reshape(*codes.shape[:-1], codes.shape[-1] * per_word)


def affine_dequantize(codes, scales, biases, group_size: int = 64, bits: int = 4, *, round_to_fp16: bool = True):
    """``mx.dequantize`` restated: ``w = scale * q + bias`` per group.

    MLX returns the dequantized array in the scales' dtype (fp16 here), so by
    default the fp32 value ``scale*q + bias`` is rounded once to fp16, as the
    reference composition (dequantize, then attention in fp32) would see it.
    """
    q = unpack_codes(codes, bits).astype(np.float32)
    s = np.asarray(scales).astype(np.float32)
    b = np.asarray(biases).astype(np.float32)
    d = q.shape[-1]
    q = q.reshape(*q.shape[:-1], d // group_size, group_size)
    w = q * s[..., None] + b[..., None]
    w = w.reshape(*w.shape[:-2], d)
    if round_to_fp16:
        w = w.astype(np.float16)
    return w
