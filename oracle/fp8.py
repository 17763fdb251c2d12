"""CPU restatement of the reference's FP8 (E4M3) KV cache -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU baseline use
this module, as the checker; the product path never imports it.

Follows:

* decode  ``fp8_e4m3_to_float``  lib/python/easymlx/operations/kernels/unified_attention.py:1275-1285
  (no NaN code: exponent 15 / mantissa 7 decodes as 480);
* encode  ``float_to_fp8_e4m3`` + ``detail::fp32_to_fp8<4,3,7>``
  lib/python/easymlx/operations/kernels/_metal_header.py:339-419 (round to
  nearest even on normals, round half up in the subnormal branch, |x| > 448 and
  infinities saturate to 448, NaN -> 0x7F);
* the write of ``PageCacheView.concatenate_to_cache`` for an FP8 cache
  lib/python/easymlx/caching/paged/cache.py:1171-1184: one scale per call,
  ``max|x| / 240`` over the written keys (values) (``_KV_SCALE_UPDATE_SOURCE``
  :195-239, ``compute_kv_scales`` :430-463), codes ``enc(x / max(scale, 1e-12))``
  (``_fp8_quantize`` :466-478), and the per-page scale raised to
  ``max(page_scale, scale)`` without requantizing the page's earlier codes;
* dequantization ``dec(code) * scale[page]`` (kernels :892-939, ``_fp8_dequantize`` :481-497).

The reference's unified write calls ``mlx.core.to_fp8`` (MLX 0.31.1, absent
here) where its paged write uses the encoder above; this restatement, and the
build, use the reference's own encoder.

Pinned by tests/test_oracle_fp8.py: known codes of the E4M3 format, a
brute-force nearest-code search for normal inputs, the exhaustive decode /
encode round trip, and the write's scale and page-scale rules on small inputs.
"""

from __future__ import annotations

import numpy as np

FP8_DIV = 240.0  # _KV_SCALE_UPDATE_SOURCE: scale = max|x| / 240
FP8_MIN_SCALE = 1e-12


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """uint8 E4M3 codes -> float32 (unified_attention.py:1275-1285)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.uint32)
    s = c >> 7
    e = (c >> 3) & 0xF
    m = (c & 0x7).astype(np.float64)
    sign = np.where(s == 1, -1.0, 1.0)
    sub = sign * (m / 8.0) * 2.0 ** -6
    nrm = sign * (1.0 + m / 8.0) * np.exp2(e.astype(np.float64) - 7.0)
    out = np.where(e == 0, sub, nrm)
    out = np.where((e == 0) & (m == 0), np.where(s == 1, -0.0, 0.0), out)
    return out.astype(np.float32)


def _encode_one(f: np.float32) -> int:
    bits = int(np.float32(f).view(np.uint32))
    s = bits >> 31
    ab = bits & 0x7FFFFFFF
    if ab > 0x7F800000:  # NaN
        return 0x7F
    if ab == 0x7F800000 or abs(float(f)) > 448.0:
        return (s << 7) | (0xF << 3) | 0x6
    e = ((ab >> 23) & 0xFF) - 127
    m = ab & 0x7FFFFF
    e8 = e + 7
    if 1 <= e8 <= 14:  # EXP_MAX = (1 << 4) - 2
        shift = 20
        mant = m >> shift
        lsb = mant & 1
        rnd = (m >> (shift - 1)) & 1
        sticky = int((m & ((1 << (shift - 1)) - 1)) != 0)
        mant += rnd & (sticky | lsb)
        if mant >> 3:
            mant = 0
            e8 += 1
            if e8 > 14:
                r = (s << 7) | (0xF << 3)  # the template's "infinity" (exp 15, mantissa 0)
                return _nan_guard(r, s)
        return _nan_guard((s << 7) | (e8 << 3) | (mant & 0x7), s)
    if e8 < 1 - 3:
        return s << 7
    rshift = (1 - e8) + 20
    mant = 0x800000 | m
    rounded = (mant + (1 << (rshift - 1))) >> rshift
    if rounded == 0:
        return s << 7
    return _nan_guard((s << 7) | (rounded & 0x7), s)


def _nan_guard(r: int, s: int) -> int:
    if ((r >> 3) & 0xF) == 0xF and (r & 0x7) == 0x7:
        return (s << 7) | (0xF << 3) | 0x6
    return r


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> uint8 E4M3 codes (_metal_header.py:391-419), vectorised.

    Same steps as ``_encode_one`` (the scalar restatement the tests compare it
    with) on whole arrays.
    """
    x = np.asarray(x, dtype=np.float32)
    bits = x.view(np.uint32).astype(np.int64)
    s = bits >> 31
    ab = bits & 0x7FFFFFFF
    e8 = ((ab >> 23) & 0xFF) - 127 + 7
    m = ab & 0x7FFFFF
    # normal path: exponent 1..14, round to nearest even
    mant = m >> 20
    rnd = (m >> 19) & 1
    sticky = ((m & 0x7FFFF) != 0).astype(np.int64)
    mant = mant + (rnd & (sticky | (mant & 1)))
    over = (mant >> 3) != 0
    ee = np.where(over, e8 + 1, e8)
    mant = np.where(over, 0, mant)
    normal = (s << 7) | (np.clip(ee, 0, 15) << 3) | (mant & 7)
    normal = np.where(over & (ee > 14), (s << 7) | (0xF << 3), normal)
    # sub-normal branch (also 240 < |x| <= 448): round half up, low mantissa bits kept
    rshift = np.clip((1 - e8) + 20, 1, 62)
    rounded = ((0x800000 | m) + (np.int64(1) << (rshift - 1))) >> rshift
    sub = np.where(rounded == 0, s << 7, (s << 7) | (rounded & 7))
    sub = np.where(e8 < -2, s << 7, sub)
    r = np.where((e8 >= 1) & (e8 <= 14), normal, sub)
    nanlike = (((r >> 3) & 0xF) == 0xF) & ((r & 7) == 7)
    r = np.where(nanlike, (s << 7) | 0x7E, r)
    sat = (ab == 0x7F800000) | (np.abs(x.astype(np.float64)) > 448.0)
    r = np.where(sat, (s << 7) | 0x7E, r)
    r = np.where(ab > 0x7F800000, 0x7F, r)
    return r.astype(np.uint8)


def e4m3_encode_scalar(x: np.ndarray) -> np.ndarray:
    """The scalar restatement, element by element (small inputs)."""
    x = np.asarray(x, dtype=np.float32)
    flat = x.reshape(-1)
    out = np.fromiter((_encode_one(v) for v in flat), dtype=np.uint8, count=flat.size)
    return out.reshape(x.shape)


def fp8_scale(x: np.ndarray) -> np.float32:
    """One call's scale: max|x| / 240 in fp32 (cache.py:195-239, :430-463); 0 for no elements."""
    x = np.asarray(x, dtype=np.float32)
    if x.size == 0:
        return np.float32(0.0)
    return np.float32(np.max(np.abs(x)) / np.float32(FP8_DIV))


def fp8_quantize(x: np.ndarray, scale: np.float32) -> np.ndarray:
    """``_fp8_quantize`` (cache.py:466-478): enc(x / max(scale, 1e-12)) in fp32."""
    safe = np.maximum(np.float32(scale), np.float32(FP8_MIN_SCALE))
    return e4m3_encode(np.asarray(x, dtype=np.float32) / safe)


def fp8_write(keys, values, slot_mapping, key_cache, value_cache, k_scales, v_scales):
    """FP8 cache write (cache.py:1171-1184), in place.

    keys/values [T, Hkv, D] (any float dtype); slot_mapping [T] int (block * bs
    + offset, -1 or a page outside the pool skips the token); key_cache/value_cache uint8 [nb, bs, Hkv, D];
    k_scales/v_scales float32 [nb].  The call's scale covers the written tokens.
    """
    slot_mapping = np.asarray(slot_mapping, dtype=np.int64)
    bs = key_cache.shape[1]
    # -1 skips a token; so does a page outside the pool (the kernels' bounds rule, cache.py:859-861)
    live = (slot_mapping >= 0) & (slot_mapping // bs < key_cache.shape[0])
    k = np.asarray(keys, dtype=np.float32)[live]
    v = np.asarray(values, dtype=np.float32)[live]
    slots = slot_mapping[live]
    if slots.size == 0:
        return
    ks, vs = fp8_scale(k), fp8_scale(v)
    blk, off = slots // bs, slots % bs
    key_cache[blk, off] = fp8_quantize(k, ks)
    value_cache[blk, off] = fp8_quantize(v, vs)
    for b in np.unique(blk):
        k_scales[b] = max(np.float32(k_scales[b]), ks)
        v_scales[b] = max(np.float32(v_scales[b]), vs)


def fp8_dequant_cache(cache: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """dec(code) * scale[page] -> float32 [nb, bs, Hkv, D] (kernels :892-939)."""
    return e4m3_decode(cache) * np.asarray(scales, dtype=np.float32)[:, None, None, None]
