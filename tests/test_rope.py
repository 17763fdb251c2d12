"""RotaryEmbedding (host side): the torch rotation vs a float64 NumPy restatement, Llama-3 periods vs the
reference's construction (lib/python/easymlx/layers/rotary/_rotary.py:175-190), call conventions."""

import math

import numpy as np
import pytest
import torch

from easymlx_amd import RotaryEmbedding


def np_rope(x, pos, inv, dims, traditional):
    """Float64 rotation of x [..., seq, D] at positions pos [..., seq]."""
    x = np.asarray(x, np.float64).copy()
    th = np.asarray(pos, np.float64)[..., None] * np.asarray(inv, np.float64)
    c, s = np.cos(th), np.sin(th)
    half = dims // 2
    if traditional:
        x0, x1 = x[..., 0:dims:2].copy(), x[..., 1:dims:2].copy()
        x[..., 0:dims:2], x[..., 1:dims:2] = x0 * c - x1 * s, x0 * s + x1 * c
    else:
        x0, x1 = x[..., :half].copy(), x[..., half:dims].copy()
        x[..., :half], x[..., half:dims] = x0 * c - x1 * s, x0 * s + x1 * c
    return x


@pytest.mark.parametrize("traditional", [False, True])
@pytest.mark.parametrize("dims", [128, 64])
def test_rotation_matches_float64(traditional, dims):
    rng = np.random.default_rng(3)
    rope = RotaryEmbedding(dims, traditional=traditional, base=500000.0)
    x = rng.standard_normal((2, 4, 7, 128)).astype(np.float32)
    got = rope(torch.from_numpy(x), offset=1000).numpy()
    inv = rope.inv_freq_cpu.numpy()
    exp = np_rope(x, np.arange(1000, 1007), inv, dims, traditional)
    np.testing.assert_allclose(got, exp, atol=2e-3, rtol=1e-4)  # fp32 angles at positions ~1e3
    assert np.array_equal(got[..., dims:], x[..., dims:])  # dims beyond `dims` pass through


def test_default_inverse_frequencies():
    rope = RotaryEmbedding(128, base=10000.0, scale=0.5)
    i = np.arange(0, 128, 2)
    np.testing.assert_allclose(rope.inv_freq_cpu.numpy(), 0.5 * 10000.0 ** (-i / 128), rtol=1e-6)


def test_llama3_periods():
    """Piecewise periods: high frequencies unscaled, low frequencies x factor, the middle band smoothed."""
    dims, base, factor, lo, hi, old = 128, 500000.0, 8.0, 1.0, 4.0, 8192
    rope = RotaryEmbedding.llama3(dims, base=base, factor=factor, low_freq_factor=lo, high_freq_factor=hi,
                                  original_max_position_embeddings=old)
    freqs = base ** (np.arange(0, dims, 2) / dims)
    wl = 2 * math.pi * freqs
    exp = np.where(wl > old / lo, freqs * factor, freqs)
    mid = (wl > old / hi) & (wl < old / lo)
    sm = (old / wl - lo) / (hi - lo)
    exp = np.where(mid, exp / ((1 - sm) / factor + sm), exp)
    np.testing.assert_allclose(1.0 / rope.inv_freq_cpu.numpy(), exp, rtol=1e-5)
    assert 1.0 / rope.inv_freq_cpu[0] == 1.0  # highest frequency untouched
    assert np.isclose(1.0 / rope.inv_freq_cpu[-1].item(), freqs[-1] * factor, rtol=1e-5)


def test_per_row_offsets_like_a_decode_batch():
    """rope(x [B, H, 1, D], offset=[B]) -- the reference's single-token decode call (cache.py:1161-1166)."""
    rng = np.random.default_rng(4)
    rope = RotaryEmbedding(128)
    x = rng.standard_normal((3, 2, 1, 128)).astype(np.float32)
    offs = np.array([5, 900, 17])
    got = rope(torch.from_numpy(x), offset=torch.from_numpy(offs)).numpy()
    for b in range(3):
        exp = np_rope(x[b], np.array([offs[b]]), rope.inv_freq_cpu.numpy(), 128, False)
        np.testing.assert_allclose(got[b], exp, atol=1e-4, rtol=1e-5)


def test_rejects_bad_dims_and_freqs():
    with pytest.raises(ValueError):
        RotaryEmbedding(7)
    with pytest.raises(ValueError):
        RotaryEmbedding(8, base=None, freqs=[1.0, 2.0])
