"""Shared test helpers: build GPU pages from a workload, compute oracle outputs."""

from __future__ import annotations

import numpy as np
import torch

from easymlx_amd.caching import affine_pool
from easymlx_amd.caching import layout
from easymlx_amd.workloads import Workload
from oracle.affine import affine_dequantize, affine_quantize
from oracle.paged_attention import paged_attention as oracle_attention

# Attention tolerance stated by the north star for fp16 outputs vs the reference.
ATOL = 2e-3
RTOL = 1e-2


def gpu_cache(wl: Workload, device):
    """Quantize-on-write every token of the workload into a fresh GPU page pool."""
    view = affine_pool(
        num_blocks=wl.num_blocks,
        num_kv_heads=wl.num_kv_heads,
        head_dim=wl.head_dim,
        block_size=wl.block_size,
        bits=wl.bits,
        group_size=wl.group_size,
        block_tables=torch.from_numpy(wl.block_tables).to(device),
        kv_lens=torch.from_numpy(wl.kv_lens).to(device),
    )
    view.write_slots(
        torch.from_numpy(wl.k).to(device),
        torch.from_numpy(wl.v).to(device),
        torch.from_numpy(wl.slot.astype(np.int32)).to(device),
    )
    return view


def oracle_logical_pages(wl: Workload):
    """Oracle-quantized logical pages: codes/scales/biases ``[nb, bs, Hkv, ...]`` for K and V."""
    out = {}
    b, o = wl.slot // wl.block_size, wl.slot % wl.block_size
    for name, x in (("k", wl.k), ("v", wl.v)):
        c, s, bi = affine_quantize(x, wl.group_size, wl.bits)
        C = np.zeros((wl.num_blocks, wl.block_size) + c.shape[1:], np.uint32)
        S = np.zeros((wl.num_blocks, wl.block_size) + s.shape[1:], np.float16)
        B = np.zeros_like(S)
        C[b, o], S[b, o], B[b, o] = c, s, bi
        out[name] = (C, S, B)
    return out


def oracle_expected(wl: Workload, *, sliding_window: int = 0, block_tables=None, kv_lens=None,
                    fp16_dequant: bool = False):
    """Oracle attention over the oracle-quantized cache (float64).

    ``fp16_dequant=False`` (default): the affine values ``scale * code + bias``
    enter attention exactly (fp32), which is the attention the quantized cache
    defines.  ``True``: each dequantized element is first rounded to fp16, as a
    materialised ``mx.dequantize`` output would be; with per-channel gains up to
    4 that rounding alone moves outputs by up to ~4e-3, so it is not the
    parity target (see tests/test_oracle_attention.py).
    """
    kc = np.zeros((wl.num_blocks, wl.block_size, wl.num_kv_heads, wl.head_dim), np.float32)
    vc = np.zeros_like(kc)
    b, o = wl.slot // wl.block_size, wl.slot % wl.block_size
    if wl.bits is None:
        kc[b, o], vc[b, o] = wl.k, wl.v
    else:
        for src, dst in ((wl.k, kc), (wl.v, vc)):
            c, s, bi = affine_quantize(src, wl.group_size, wl.bits)
            dst[b, o] = affine_dequantize(c, s, bi, wl.group_size, wl.bits, round_to_fp16=fp16_dequant)
    return oracle_attention(
        wl.q, kc, vc,
        wl.block_tables if block_tables is None else block_tables,
        wl.kv_lens if kv_lens is None else kv_lens,
        wl.query_start_loc,
        softmax_scale=1.0 / np.sqrt(wl.head_dim),
        sliding_window=sliding_window,
        compute_dtype=np.float64,
        out_dtype=np.float64,
    )


def gpu_pages_to_logical(view):
    """Read GPU pages back in the logical MLX layout (numpy)."""
    kc = layout.key_logical_from_pages(view.k_codes.cpu().numpy())
    vc = layout.value_logical_from_pages(view.v_codes.cpu().numpy(), view.bits)
    ks = layout.params_logical_from_pages(view.k_scales.cpu().numpy())
    kb = layout.params_logical_from_pages(view.k_biases.cpu().numpy())
    vs = layout.params_logical_from_pages(view.v_scales.cpu().numpy())
    vb = layout.params_logical_from_pages(view.v_biases.cpu().numpy())
    return {"k": (kc, ks, kb), "v": (vc, vs, vb)}


def assert_attention_close(actual: np.ndarray, expected: np.ndarray, what: str = ""):
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, (a.shape, e.shape)
    assert np.isfinite(a).all(), f"{what}: non-finite outputs"
    err = np.abs(a - e)
    bad = err > ATOL + RTOL * np.abs(e)
    assert not bad.any(), (
        f"{what}: {int(bad.sum())} of {bad.size} outside atol={ATOL} rtol={RTOL}; "
        f"max abs err {err.max():.3e} at {np.unravel_index(err.argmax(), err.shape)}"
    )


# ---------------------------------------------------------------- C oracle (full sizes)
_C_ORACLE = None


def c_oracle_lib():
    """The C restatement ``oracle/c/liboracle.so`` (built by ``make -C oracle/c``)."""
    global _C_ORACLE
    if _C_ORACLE is None:
        import ctypes
        import os
        import subprocess

        root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
        path = os.path.join(root, "oracle", "c", "liboracle.so")
        if not os.path.exists(path):
            subprocess.run(["make", "-s", "-C", os.path.dirname(path)], check=True)
        lib = ctypes.CDLL(path)
        P, I = ctypes.c_void_p, ctypes.c_int
        lib.oracle_affine_quantize.argtypes = [P, ctypes.c_long, I, I, I, P, P, P]
        lib.oracle_affine_quantize.restype = None
        lib.oracle_attention_affine.argtypes = [P] * 10 + [I] * 9 + [ctypes.c_double, I, I, P]
        lib.oracle_attention_affine.restype = None
        _C_ORACLE = lib
    return _C_ORACLE


def _ptr(a):
    import ctypes

    return a.ctypes.data_as(ctypes.c_void_p)


def c_quantize(x: np.ndarray, group_size: int, bits: int):
    """``oracle_affine_quantize`` over the last axis of fp16 ``x`` (bit-identical to oracle.affine)."""
    x = np.ascontiguousarray(x, dtype=np.float16)
    d = x.shape[-1]
    rows = x.size // d
    codes = np.zeros(x.shape[:-1] + (d * bits // 32,), np.uint32)
    sc = np.zeros(x.shape[:-1] + (d // group_size,), np.float16)
    bi = np.zeros_like(sc)
    c_oracle_lib().oracle_affine_quantize(_ptr(x.view(np.uint16)), rows, d, group_size, bits, _ptr(codes),
                                          _ptr(sc.view(np.uint16)), _ptr(bi.view(np.uint16)))
    return codes, sc, bi


def c_oracle_expected(wl: Workload, *, sliding_window: int = 0, block_tables=None, kv_lens=None,
                      fp16_dequant: bool = False) -> np.ndarray:
    """``oracle_expected`` computed by the C restatement (double precision), for full-size workloads.

    Same semantics as :func:`oracle_expected` (pinned against it in
    ``tests/test_oracle_attention.py``); quantizes with the C quantizer, which
    is bit-identical to ``oracle.affine.affine_quantize``.
    """
    assert wl.bits is not None
    b, o = wl.slot // wl.block_size, wl.slot % wl.block_size
    pages = []
    for x in (wl.k, wl.v):
        c, s, bi = c_quantize(x, wl.group_size, wl.bits)
        C = np.zeros((wl.num_blocks, wl.block_size) + c.shape[1:], np.uint32)
        S = np.zeros((wl.num_blocks, wl.block_size) + s.shape[1:], np.float16)
        B = np.zeros_like(S)
        C[b, o], S[b, o], B[b, o] = c, s, bi
        pages.append((C, S, B))
    bt = np.ascontiguousarray(wl.block_tables if block_tables is None else block_tables, dtype=np.int32)
    kl = np.ascontiguousarray(wl.kv_lens if kv_lens is None else kv_lens, dtype=np.int32)
    qsl = np.ascontiguousarray(wl.query_start_loc, dtype=np.int32)
    q = np.ascontiguousarray(wl.q, dtype=np.float16)
    out = np.zeros(q.shape, np.float64)
    (kc, ks, kb), (vc, vs, vb) = pages
    c_oracle_lib().oracle_attention_affine(
        _ptr(q.view(np.uint16)), _ptr(kc), _ptr(ks.view(np.uint16)), _ptr(kb.view(np.uint16)), _ptr(vc),
        _ptr(vs.view(np.uint16)), _ptr(vb.view(np.uint16)), _ptr(bt), _ptr(kl), _ptr(qsl), int(kl.shape[0]),
        wl.num_q_heads, wl.num_kv_heads, wl.head_dim, wl.block_size, wl.num_blocks, int(bt.shape[1]), wl.bits,
        wl.group_size, 1.0 / np.sqrt(wl.head_dim), int(sliding_window), int(fp16_dequant), _ptr(out))
    return out
