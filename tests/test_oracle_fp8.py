"""Pins the FP8 (E4M3) oracle: known codes, brute-force nearest code, round trips, write rules."""

import numpy as np

from oracle import fp8


def test_decode_known_codes():
    d = fp8.e4m3_decode(np.array([0x38, 0xB8, 0x7E, 0x77, 0x08, 0x01, 0x07, 0x00, 0x80, 0x7F], np.uint8))
    assert d[0] == 1.0 and d[1] == -1.0
    assert d[2] == 448.0 and d[3] == 240.0
    assert d[4] == 2.0 ** -6 and d[5] == 2.0 ** -9 and d[6] == 7 * 2.0 ** -9
    assert d[7] == 0.0 and d[8] == 0.0 and np.signbit(d[8])
    # the reference decoder has no NaN code: exponent 15, mantissa 7 is (1 + 7/8) * 2^8
    assert d[9] == 480.0


def test_encode_known_values():
    x = np.array([1.0, -1.0, 240.0, 2.0 ** -9, 0.0, np.nan, np.inf, 1000.0, -1000.0, 0.5, 3.0], np.float32)
    e = fp8.e4m3_encode(x)
    assert list(e) == [0x38, 0xB8, 0x77, 0x01, 0x00, 0x7F, 0x7E, 0x7E, 0xFE, 0x30, 0x44]


def test_encode_round_to_nearest_even():
    # 1.0625 lies halfway between 1.0 (mantissa 0) and 1.125 (mantissa 1): even wins
    # 1.1875 lies halfway between 1.125 (mantissa 1) and 1.25 (mantissa 2): even wins
    e = fp8.e4m3_encode(np.array([1.0625, 1.1875, 1.0626, 1.1874], np.float32))
    assert list(e) == [0x38, 0x3A, 0x39, 0x39]


def test_encode_matches_brute_force_nearest_on_normals():
    rng = np.random.default_rng(5)
    x = np.exp2(rng.uniform(-6.0, np.log2(240.0), 4000)).astype(np.float32) * rng.choice([-1, 1], 4000)
    codes = np.arange(256, dtype=np.uint8)
    vals = fp8.e4m3_decode(codes).astype(np.float64)
    exp = (codes >> 3) & 0xF
    normal = (exp >= 1) & (exp <= 14)
    cand, cvals = codes[normal], vals[normal]
    got = fp8.e4m3_encode(x)
    for xi, gi in zip(x.astype(np.float64), got):
        dist = np.abs(cvals - xi)
        best = cand[dist == dist.min()]
        if best.size > 1:  # a tie: the even mantissa
            best = best[(best & 1) == 0]
        assert gi == best[0], (xi, gi, best)


def test_round_trip_every_finite_code():
    codes = np.arange(256, dtype=np.uint8)
    exp = (codes >> 3) & 0xF
    keep = exp <= 14  # exponent 15 lies outside the encoder's normal range (|x| > 240)
    back = fp8.e4m3_encode(fp8.e4m3_decode(codes[keep]))
    assert np.array_equal(back, codes[keep])


def test_write_scale_and_page_scale_rules():
    nb, bs, hkv, d = 2, 4, 1, 8
    kc = np.zeros((nb, bs, hkv, d), np.uint8)
    vc = np.zeros_like(kc)
    ks = np.zeros(nb, np.float32)
    vs = np.zeros(nb, np.float32)
    k1 = np.full((2, hkv, d), 2.0, np.float32)
    fp8.fp8_write(k1, -k1, [0, 1], kc, vc, ks, vs)
    assert ks[0] == np.float32(2.0 / 240.0) and vs[0] == ks[0] and ks[1] == 0.0
    assert np.all(kc[0, :2] == 0x77) and np.all(vc[0, :2] == 0xF7)  # +-240 after scaling
    # a later, smaller write to the same page: its codes use its own scale, the
    # page keeps the larger one, and the earlier codes are not requantized
    k2 = np.full((1, hkv, d), 0.5, np.float32)
    fp8.fp8_write(k2, k2, [2], kc, vc, ks, vs)
    assert ks[0] == np.float32(2.0 / 240.0)
    assert np.all(kc[0, 2] == 0x77) and np.all(kc[0, :2] == 0x77)
    # a skipped slot (-1) writes nothing and does not enter the scale
    fp8.fp8_write(np.full((1, hkv, d), 100.0, np.float32), k2, [-1], kc, vc, ks, vs)
    assert ks[0] == np.float32(2.0 / 240.0)
    # so does a slot whose page lies outside the pool
    before = kc.copy()
    fp8.fp8_write(np.full((2, hkv, d), 100.0, np.float32), np.full((2, hkv, d), 100.0, np.float32),
                  [nb * kc.shape[1] + 3, 3], kc, vc, ks, vs)
    assert np.array_equal(kc[1:], before[1:])
    assert ks[0] == np.float32(100.0 / 240.0) and ks[0] == vs[0]  # only the in-pool token (slot 3) counts
    fp8.fp8_write(np.full((1, hkv, d), 1e4, np.float32), k2, [nb * kc.shape[1]], kc, vc, ks, vs)
    assert ks[0] == np.float32(100.0 / 240.0) and np.all(ks[1:] == 0)
    ks[0] = vs[0] = np.float32(2.0 / 240.0)
    kc[0, 3] = vc[0, 3] = 0
    deq = fp8.fp8_dequant_cache(kc, ks)
    assert np.allclose(deq[0, :2], 2.0)


def test_vectorised_encoder_matches_scalar_restatement():
    rng = np.random.default_rng(9)
    x = np.concatenate([
        rng.standard_normal(3000).astype(np.float32) * np.exp2(rng.uniform(-12, 10, 3000)).astype(np.float32),
        np.array([0.0, -0.0, 240.0, 241.0, 300.0, 448.0, 449.0, -447.9, 2.0 ** -10, 2.0 ** -9, 7.5 * 2.0 ** -9,
                  np.inf, -np.inf, np.nan, 1e-40], np.float32),
    ])
    assert np.array_equal(fp8.e4m3_encode(x), fp8.e4m3_encode_scalar(x))
