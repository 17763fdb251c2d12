"""Pins of the affine quantize restatement (``oracle/affine.py``, ``oracle/c/oracle.c``).

MLX itself cannot be imported here, so the restatement is pinned by what the
mathematics of the affine format fixes:

* hand-computed known answers (a 0..15 ramp whose codes and packed words can
  be written down by hand, a half-way value that pins round-half-to-even);
* invariants: codes in range, the group edge reconstructs exactly, every
  element within half a step, nearest-code selection by brute force;
* special cases: constant groups, exact zeros, all-zero groups;
* agreement with the independent C restatement on random inputs.

A dropped term (bias), a sign slip (the ``mask`` branch), a transposed pack
order or round-half-away-from-zero each fails at least one of these.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np
import pytest

from oracle.affine import affine_dequantize, affine_quantize, unpack_codes

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def c_oracle():
    path = os.path.join(ROOT, "oracle", "c", "liboracle.so")
    if not os.path.exists(path):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle", "c")], check=True)
    lib = ctypes.CDLL(path)
    P = ctypes.c_void_p
    lib.oracle_affine_quantize.argtypes = [P, ctypes.c_long, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P]
    lib.oracle_affine_quantize.restype = None
    return lib


def test_ramp_known_answer_4bit():
    # w = 0..15: min 0, max 15 -> |min| <= |max| -> scale = -(15/15) = -1, edge = max = 15,
    # q0 = rint(15 / -1) = -15 -> scale = 15 / -15 = -1, bias = 15; code_i = rint((i - 15) / -1) = 15 - i.
    w = np.arange(16, dtype=np.float32)[None]
    codes, scales, biases = affine_quantize(w, group_size=16, bits=4)
    assert scales.tolist() == [[-1.0]] and biases.tolist() == [[15.0]]
    assert unpack_codes(codes, 4).tolist() == [[15 - i for i in range(16)]]
    word0 = sum((15 - j) << (4 * j) for j in range(8))
    word1 = sum((15 - 8 - j) << (4 * j) for j in range(8))
    assert codes.tolist() == [[word0, word1]]


def test_ramp_known_answer_8bit_negative_side():
    # w = -255..0 step 1 (x4 groups of 64 along a 256-wide row): |min| > |max| -> positive scale.
    w = -np.arange(256, dtype=np.float32)[::-1].copy()[None]  # -255 .. 0
    codes, scales, biases = affine_quantize(w, group_size=64, bits=8)
    q = unpack_codes(codes, 8).reshape(4, 64)
    for g in range(4):
        grp = w[0, 64 * g:64 * (g + 1)]
        lo, hi = grp.min(), grp.max()
        if abs(lo) > abs(hi):  # edge = min, code(min) = 0
            assert biases[0, g] == lo
            assert q[g, 0] == 0
        else:  # edge = max (the last group ends at 0: max = 0 -> q0 = 0 -> bias 0)
            assert biases[0, g] == 0.0
    # first byte of the first word is element 0 (little-endian packing)
    assert (codes[0, 0] & 0xFF) == q[0, 0] and (codes[0, 0] >> 24) == q[0, 3]


def test_round_half_to_even():
    # same ramp as above with element 8 replaced by 7.5: (7.5 - 15) / -1 = 7.5 -> rint -> 8 (even);
    # half-away-from-zero would also give 8, so also place 6.5 -> 8.5 -> 8 (even; away would give 9).
    w = np.arange(16, dtype=np.float32)
    w[8] = 7.5
    w[9] = 6.5
    c, _, _ = affine_quantize(w[None], group_size=16, bits=4)
    q = unpack_codes(c, 4)[0]
    assert q[8] == 8 and q[9] == 8


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_invariants_random(bits, gs):
    rng = np.random.default_rng(100 + bits + gs)
    d = 256
    w = (rng.standard_normal((300, d)) * rng.uniform(0.5, 4, d)).astype(np.float16)
    codes, scales, biases = affine_quantize(w, gs, bits)
    assert codes.dtype == np.uint32 and codes.shape == (300, d * bits // 32)
    assert scales.dtype == np.float16 and scales.shape == (300, d // gs)
    q = unpack_codes(codes, bits)
    assert q.max() <= 2**bits - 1
    # unclipped codes reconstruct within half a step (+ the fp16 rounding of scale and bias); codes at
    # the far end may be clipped because the zero-point adjustment can shrink |scale| (the brute-force
    # test below covers those)
    wf = w.astype(np.float32).reshape(300, d // gs, gs)
    s = scales.astype(np.float32)[..., None]
    b = biases.astype(np.float32)[..., None]
    rec = q.reshape(300, d // gs, gs) * s + b
    err = np.abs(rec - wf)
    step = np.abs(s)
    fp16_slack = (2**bits) * np.abs(s) * 2**-10 + np.abs(b) * 2**-10
    inner = (q.reshape(err.shape) > 0) & (q.reshape(err.shape) < 2**bits - 1)
    assert ((err <= 0.5 * step + fp16_slack + 1e-6) | ~inner).all()
    assert inner.mean() > 0.5
    # the dequantized edge equals the edge in fp32 params: re-run on fp32 input for exact params
    c32, s32, b32 = affine_quantize(w.astype(np.float32), gs, bits)
    rec32 = unpack_codes(c32, bits).reshape(300, d // gs, gs) * s32[..., None] + b32[..., None]
    lo, hi = wf.min(-1), wf.max(-1)
    edge = np.where(np.abs(lo) > np.abs(hi), lo, hi)
    nz = np.rint(edge / np.where(np.abs(lo) > np.abs(hi), 1, -1) /
                 np.maximum((hi - lo) / (2**bits - 1), 1e-7)) != 0
    edge_rec = np.take_along_axis(rec32, np.argmax(wf == edge[..., None], -1)[..., None], -1)[..., 0]
    np.testing.assert_allclose(edge_rec[nz], edge[nz], rtol=2e-6, atol=0)


@pytest.mark.parametrize("bits", [4, 8])
def test_nearest_code_brute_force(bits):
    """Given the (fp32) scale/bias, every code is the nearest of all 2^b candidates."""
    rng = np.random.default_rng(7 + bits)
    w = rng.standard_normal((40, 64)).astype(np.float32)
    c, s, b = affine_quantize(w, 64, bits)
    q = unpack_codes(c, bits)
    cand = np.arange(2**bits, dtype=np.float32)[None, None, :] * s[:, :, None] + b[:, :, None]  # [40,1,K]
    dist = np.abs(w[:, :, None] - cand)
    best = dist.min(-1)
    got = np.take_along_axis(dist, q[:, :, None].astype(np.int64), -1)[..., 0]
    assert (got <= best + 1e-6 * np.abs(w)).all()


@pytest.mark.parametrize("bits", [4, 8])
def test_constant_and_zero_groups(bits):
    w = np.zeros((4, 64), np.float32)
    w[1] = 3.25
    w[2] = -0.5
    w[3, :32] = 0.0
    w[3, 32:] = 2.0
    c, s, b = affine_quantize(w, 64, bits)
    rec = affine_dequantize(c, s, b, 64, bits, round_to_fp16=False)
    # all-zero group: q0 = 0 -> bias 0, reconstruction exactly 0
    assert b[0, 0] == 0.0 and (rec[0] == 0).all()
    # constant groups reconstruct exactly (bias = the constant, code 0)
    assert (rec[1] == 3.25).all() and (rec[2] == -0.5).all()
    # a group whose min is exactly 0 keeps zero exactly representable
    assert (rec[3, :32] == 0).all()


def test_dequantize_fp16_rounding():
    rng = np.random.default_rng(3)
    w = rng.standard_normal((8, 128)).astype(np.float16)
    c, s, b = affine_quantize(w, 64, 4)
    a32 = affine_dequantize(c, s, b, 64, 4, round_to_fp16=False)
    a16 = affine_dequantize(c, s, b, 64, 4)
    assert a16.dtype == np.float16
    np.testing.assert_array_equal(a16, a32.astype(np.float16))


def test_rejects_bad_shapes():
    with pytest.raises(ValueError):
        affine_quantize(np.zeros((2, 100), np.float32), 64, 4)
    with pytest.raises(ValueError):
        affine_quantize(np.zeros((2, 64), np.float32), 64, 3)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_numpy_matches_c_restatement(c_oracle, bits, gs):
    rng = np.random.default_rng(1000 * bits + gs)
    rows, d = 2048, 128
    w = (rng.standard_normal((rows, d)) * rng.uniform(0.5, 4, d)).astype(np.float16)
    w[:4] = 0
    w[4, :] = 1.5
    w[5, : d // 2] = 0
    codes, scales, biases = affine_quantize(w, gs, bits)
    cc = np.zeros_like(codes)
    cs = np.zeros(scales.shape, np.uint16)
    cb = np.zeros(biases.shape, np.uint16)
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    c_oracle.oracle_affine_quantize(P(w.view(np.uint16)), rows, d, gs, bits, P(cc), P(cs), P(cb))
    np.testing.assert_array_equal(cc, codes)
    np.testing.assert_array_equal(cs, scales.view(np.uint16))
    np.testing.assert_array_equal(cb, biases.view(np.uint16))
