"""Pins of the attention oracle (``oracle/paged_attention.py``, ``oracle/c/oracle.c``).

* The reference tests' seeded cases (regenerated bit-exactly in
  ``tests/golden``) against ``torch.nn.functional.scaled_dot_product_attention``
  over sequences gathered by independent code here -- a second implementation
  of the same closed form.
* Closed forms: one visible key returns its value; equal keys average the
  values; a query of zeros averages the visible values.
* Semantics the reference kernels fix: causal limit for ragged chunks,
  sliding window, GQA head mapping, invalid pages (skip vs zero), empty rows.
* Split-K: merging partitions equals the unpartitioned result
  (``page_attention.py:2006-2059``).
* The C restatement's decode and its fp16 conversions.
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess

import numpy as np
import pytest
import torch

from oracle.affine import affine_dequantize, affine_quantize
from oracle.paged_attention import causal_single_sequence, gather_sequence, merge_partials, paged_attention

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")


def _sdpa_reference(q, kc, vc, tables, kv_lens, qsl, scale):
    """Independent computation: explicit gather + torch SDPA with a bottom-right causal mask."""
    out = torch.zeros(q.shape, dtype=torch.float64)
    hq, hkv = q.shape[1], kc.shape[2]
    bs = kc.shape[1]
    for s in range(tables.shape[0]):
        a, b = int(qsl[s]), int(qsl[s + 1])
        L = int(kv_lens[s])
        if b <= a or L <= 0:
            continue
        ks = np.stack([kc[tables[s, p // bs], p % bs] for p in range(L)])  # [L, Hkv, D]
        vs = np.stack([vc[tables[s, p // bs], p % bs] for p in range(L)])
        k = torch.from_numpy(ks).double().repeat_interleave(hq // hkv, dim=1).permute(1, 0, 2)
        v = torch.from_numpy(vs).double().repeat_interleave(hq // hkv, dim=1).permute(1, 0, 2)
        qq = torch.from_numpy(np.asarray(q[a:b])).double().permute(1, 0, 2)
        n = b - a
        mask = torch.arange(L)[None, :] <= (L - n + torch.arange(n))[:, None]
        o = torch.nn.functional.scaled_dot_product_attention(qq, k, v, attn_mask=mask, scale=scale)
        out[a:b] = o.permute(1, 0, 2)
    return out.numpy()


@pytest.mark.parametrize("name", ["attn_rng0", "attn_rng1", "attn_rng11"])
def test_golden_cases_match_sdpa(name):
    z = np.load(os.path.join(GOLDEN, name + ".npz"))
    args = (z["queries"], z["key_cache"], z["value_cache"], z["block_tables"], z["kv_lens"], z["query_start_loc"])
    ref = _sdpa_reference(*args, float(z["softmax_scale"]))
    got = paged_attention(*[a.astype(np.float64) if a.dtype == np.float32 else a for a in args],
                          softmax_scale=float(z["softmax_scale"]), compute_dtype=np.float64, out_dtype=np.float64)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
    # the committed expectations are the same numbers (fixture integrity)
    np.testing.assert_allclose(z["expected"], ref, rtol=1e-12, atol=1e-12)
    # the reference tests compare at atol=rtol=1e-5 in fp32: the fp32 oracle passes that bar too
    got32 = paged_attention(*args, softmax_scale=float(z["softmax_scale"]))
    np.testing.assert_allclose(got32, ref, rtol=1e-5, atol=1e-5)


def _single_seq(q, k, v, bs=4):
    """Lay one sequence's keys/values into consecutive pages; returns oracle args."""
    L, hkv, d = k.shape
    nb = max(1, math.ceil(L / bs))
    kc = np.zeros((nb, bs, hkv, d))
    vc = np.zeros((nb, bs, hkv, d))
    for p in range(L):
        kc[p // bs, p % bs] = k[p]
        vc[p // bs, p % bs] = v[p]
    tables = np.arange(nb, dtype=np.int32)[None]
    return q, kc, vc, tables, np.array([L], np.int32), np.array([0, q.shape[0]], np.int32)


def test_closed_forms():
    rng = np.random.default_rng(5)
    d, hq, hkv = 8, 4, 2
    v = rng.standard_normal((9, hkv, d))
    # one key -> the output is that key's value
    q = rng.standard_normal((1, hq, d))
    k = rng.standard_normal((1, hkv, d))
    o = paged_attention(*_single_seq(q, k, v[:1]), compute_dtype=np.float64)
    np.testing.assert_allclose(o[0], np.repeat(v[0], hq // hkv, axis=0), rtol=1e-12)
    # identical keys -> uniform weights -> mean of the values
    k = np.repeat(rng.standard_normal((1, hkv, d)), 9, axis=0)
    o = paged_attention(*_single_seq(q, k, v), compute_dtype=np.float64)
    np.testing.assert_allclose(o[0], np.repeat(v.mean(0), hq // hkv, axis=0), rtol=1e-12)
    # zero query -> mean of the visible values, with causal limit for a 3-token chunk
    q = np.zeros((3, hq, d))
    k = rng.standard_normal((9, hkv, d))
    o = paged_attention(*_single_seq(q, k, v), compute_dtype=np.float64)
    for i in range(3):
        np.testing.assert_allclose(o[i], np.repeat(v[: 9 - 3 + i + 1].mean(0), hq // hkv, axis=0), rtol=1e-12)


def test_sliding_window_equals_truncated_context():
    rng = np.random.default_rng(6)
    d, hq, hkv, L, w = 8, 2, 1, 11, 4
    q = rng.standard_normal((1, hq, d))
    k = rng.standard_normal((L, hkv, d))
    v = rng.standard_normal((L, hkv, d))
    o = paged_attention(*_single_seq(q, k, v), sliding_window=w, compute_dtype=np.float64)
    o_trunc = paged_attention(*_single_seq(q, k[-w:], v[-w:]), compute_dtype=np.float64)
    np.testing.assert_allclose(o, o_trunc, rtol=1e-12)


def test_gqa_mapping():
    # kv head j holds constant value j+1: query head h must read kv head h // (Hq/Hkv)
    d, hq, hkv, L = 4, 6, 3, 5
    k = np.zeros((L, hkv, d))
    v = np.broadcast_to(np.arange(1, hkv + 1, dtype=np.float64)[None, :, None], (L, hkv, d)).copy()
    q = np.ones((1, hq, d))
    o = paged_attention(*_single_seq(q, k, v), compute_dtype=np.float64)
    assert o[0, :, 0].tolist() == [1, 1, 2, 2, 3, 3]


def test_invalid_pages_and_empty_rows():
    rng = np.random.default_rng(8)
    d, hq, hkv, bs = 4, 2, 1, 4
    kc = rng.standard_normal((3, bs, hkv, d))
    vc = rng.standard_normal((3, bs, hkv, d))
    tables = np.array([[0, -1, 2], [1, 2, 0], [0, 0, 0]], np.int32)
    kv_lens = np.array([10, 0, 5], np.int32)
    q = rng.standard_normal((3, hq, d))
    qsl = np.array([0, 1, 2, 3], np.int32)
    o_skip = paged_attention(q, kc, vc, tables, kv_lens, qsl, compute_dtype=np.float64)
    o_zero = paged_attention(q, kc, vc, tables, kv_lens, qsl, invalid_block="zero", compute_dtype=np.float64)
    # skip == attention over the valid positions only
    pos = [p for p in range(10) if tables[0, p // bs] >= 0]
    kk = np.stack([kc[tables[0, p // bs], p % bs] for p in pos])
    vv = np.stack([vc[tables[0, p // bs], p % bs] for p in pos])
    o_valid = paged_attention(*_single_seq(q[:1], kk, vv), compute_dtype=np.float64)
    np.testing.assert_allclose(o_skip[0], o_valid[0], rtol=1e-12)
    # zero == the invalid positions count as zero keys/values (scores 0, weight e^0 each)
    assert not np.allclose(o_zero[0], o_skip[0])
    # a sequence with kv_len 0 produces zeros
    assert (o_skip[1] == 0).all() and (o_zero[1] == 0).all()
    g, valid = gather_sequence(kc, tables[0], 10)
    assert valid.tolist() == [True] * 4 + [False] * 4 + [True] * 2 and (g[4:8] == 0).all()


def test_split_k_merge_equals_whole():
    rng = np.random.default_rng(9)
    L, hq, d = 37, 3, 8
    q = rng.standard_normal((hq, d))
    k = rng.standard_normal((L, hq, d))
    v = rng.standard_normal((L, hq, d))
    s = np.einsum("hd,lhd->hl", q, k)
    p = np.exp(s - s.max(-1, keepdims=True))
    whole = np.einsum("hl,lhd->hd", p, v) / p.sum(-1)[:, None]
    cuts = [0, 5, 5, 20, 37]  # includes an empty partition
    ms, ls, os_ = [], [], []
    for a, b in zip(cuts[:-1], cuts[1:]):
        if a == b:
            ms.append(np.full(hq, -np.inf))
            ls.append(np.zeros(hq))
            os_.append(np.zeros((hq, d)))
            continue
        m = s[:, a:b].max(-1)
        e = np.exp(s[:, a:b] - m[:, None])
        ms.append(m)
        ls.append(e.sum(-1))
        os_.append(np.einsum("hl,lhd->hd", e, v[a:b]))
    np.testing.assert_allclose(merge_partials(np.stack(ms), np.stack(ls), np.stack(os_)), whole, rtol=1e-12)
    # all partitions empty -> zeros
    z = merge_partials(np.full((2, hq), -np.inf), np.zeros((2, hq)), np.zeros((2, hq, d)))
    assert (z == 0).all()


def test_causal_single_sequence_matches_paged():
    rng = np.random.default_rng(10)
    d, hq, hkv, past, n = 8, 4, 2, 6, 3
    k = rng.standard_normal((past + n, hkv, d))
    v = rng.standard_normal((past + n, hkv, d))
    q = rng.standard_normal((n, hq, d))
    a = causal_single_sequence(q, k, v, past)
    b = paged_attention(*_single_seq(q, k, v), compute_dtype=np.float64)
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-6)  # the single-sequence path computes in fp32


# ---------------------------------------------------------------- C restatement
@pytest.fixture(scope="module")
def c_oracle():
    path = os.path.join(ROOT, "oracle", "c", "liboracle.so")
    if not os.path.exists(path):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle", "c")], check=True)
    lib = ctypes.CDLL(path)
    lib.oracle_f2h.argtypes = [ctypes.c_float]
    lib.oracle_f2h.restype = ctypes.c_uint16
    lib.oracle_h2f.argtypes = [ctypes.c_uint16]
    lib.oracle_h2f.restype = ctypes.c_float
    P = ctypes.c_void_p
    lib.oracle_decode_affine.argtypes = [P] * 9 + [ctypes.c_int] * 9 + [ctypes.c_float, P]
    lib.oracle_decode_affine.restype = None
    return lib


def test_c_fp16_conversions(c_oracle):
    # every fp16 bit pattern (NaNs compared as NaN)
    for h in list(range(0, 0x7C01, 97)) + [0x0001, 0x03FF, 0x0400, 0x7BFF, 0x7C00, 0xFC00, 0x8001, 0xFBFF]:
        ref = np.array([h], np.uint16).view(np.float16).astype(np.float32)[0]
        assert c_oracle.oracle_h2f(h) == ref
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.standard_normal(2000) * 10.0 ** rng.integers(-8, 5, 2000),
                         [0.0, -0.0, 65504.0, 65520.0, 1e9, 2.0**-24, 2.0**-25, 3 * 2.0**-26, 5.96e-8]]).astype(np.float32)
    with np.errstate(over="ignore"):
        refs = xs.astype(np.float16).view(np.uint16)
    for x, ref in zip(xs, refs):
        assert c_oracle.oracle_f2h(float(x)) == ref, x


@pytest.mark.parametrize("bits", [4, 8])
def test_c_decode_matches_numpy(c_oracle, bits):
    rng = np.random.default_rng(20 + bits)
    S, hq, hkv, d, bs, gs = 3, 8, 2, 128, 16, 64
    lens = np.array([1, 37, 70], np.int32)
    max_blocks = 5
    nb = 16
    tables = rng.permutation(nb)[: S * max_blocks].reshape(S, max_blocks).astype(np.int32)
    kf = np.zeros((nb, bs, hkv, d), np.float16)
    vf = np.zeros_like(kf)
    for s in range(S):
        for p in range(lens[s]):
            kf[tables[s, p // bs], p % bs] = rng.standard_normal((hkv, d))
            vf[tables[s, p // bs], p % bs] = rng.standard_normal((hkv, d))
    kc, ks, kb = affine_quantize(kf, gs, bits)
    vc, vs, vb = affine_quantize(vf, gs, bits)
    q = rng.standard_normal((S, hq, d)).astype(np.float16)
    out = np.zeros((S, hq, d), np.float32)
    P = lambda a: np.ascontiguousarray(a).ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    keep = [q.view(np.uint16), kc, ks.view(np.uint16), kb.view(np.uint16), vc, vs.view(np.uint16), vb.view(np.uint16),
            tables, lens]
    c_oracle.oracle_decode_affine(*[P(a) for a in keep], S, hq, hkv, d, bs, nb, max_blocks, bits, gs,
                                  ctypes.c_float(1 / math.sqrt(d)), P(out))
    kd = affine_dequantize(kc, ks, kb, gs, bits)  # fp16-rounded dequant, as the C restatement does
    vd = affine_dequantize(vc, vs, vb, gs, bits)
    exp = paged_attention(q, kd, vd, tables, lens, np.arange(S + 1, dtype=np.int32), compute_dtype=np.float64,
                          out_dtype=np.float64)
    np.testing.assert_allclose(out, exp, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("bits,gs,fp16", [(4, 64, False), (8, 32, True), (4, 32, True), (8, 64, False)])
@pytest.mark.parametrize("window", [0, 5, 40])
def test_c_unified_matches_numpy(bits, gs, fp16, window):
    """The C ragged/causal restatement (full-size checker) against the numpy oracle."""
    from easymlx_amd.workloads import unified_workload
    from helpers import c_oracle_expected, oracle_expected

    wl = unified_workload("cpin", seed=bits + gs + window, num_prefill=2, chunk=37, prior_range=(0, 90),
                          num_decode=3, decode_ctx=(1, 120), num_q_heads=8, num_kv_heads=2, head_dim=64,
                          block_size=16, bits=bits, group_size=gs)
    tables = wl.block_tables.copy()
    lens = wl.kv_lens.copy()
    tables[1, 0] = -1              # skipped page
    tables[2, -1] = wl.num_blocks  # out-of-range page
    lens[-1] = 0                   # empty decode row
    exp = oracle_expected(wl, sliding_window=window, block_tables=tables, kv_lens=lens, fp16_dequant=fp16)
    got = c_oracle_expected(wl, sliding_window=window, block_tables=tables, kv_lens=lens, fp16_dequant=fp16)
    np.testing.assert_allclose(got, exp, rtol=1e-9, atol=1e-12)
    assert np.all(got[wl.query_start_loc[-2]:] == 0)
