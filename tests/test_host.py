"""Host-side logic, checked on the CPU: write-position arithmetic against the
reference tests' own assertions, the page-layout conversions, the operator
plugin surface, input validation, workloads, the C ABI's exports and its
argument errors (no kernel is launched here)."""

from __future__ import annotations

import ctypes
import math
import os
import re
import subprocess
import sys

import numpy as np
import pytest
import torch

from easymlx_amd.caching import layout
from easymlx_amd.caching.paged import PageCacheView, PageMetadata, build_query_start_loc
from oracle.affine import affine_quantize
from oracle.cache_write import build_query_start_loc as oracle_qsl
from oracle.cache_write import write_positions

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")


# ---------------------------------------------------------------- write positions
@pytest.mark.parametrize("name,initial,qlens", [("write_rng2", [1, 0, 2], [2, 0, 3]), ("write_rng7", [2, 1, 3], [1, 1, 1])])
def test_write_goldens(name, initial, qlens):
    """``tests/operations/test_unified_attention.py:268-415``: kv_lens += q_len, token j of a slot lands at
    ``[table[pos // bs], pos % bs]`` with ``pos = initial_len + j``."""
    z = np.load(os.path.join(GOLDEN, name + ".npz"))
    bs = z["key_cache"].shape[1]
    assert z["kv_lens"].tolist() == initial
    assert z["query_start_loc"].tolist() == oracle_qsl(qlens).tolist()
    assert z["expected_kv_lens"].tolist() == [a + b for a, b in zip(initial, qlens)]
    # the slot mapping written from first principles (tables are consecutive per sequence)
    exp = []
    for s, n in enumerate(qlens):
        for j in range(n):
            pos = initial[s] + j
            exp.append(int(z["block_tables"][s, pos // bs]) * bs + pos % bs)
    assert z["slot_mapping"].tolist() == exp
    sm, lens = write_positions(z["block_tables"], z["kv_lens"], z["query_start_loc"], [0, 1, 2], bs)
    assert sm.tolist() == exp and lens.tolist() == z["expected_kv_lens"].tolist()

    # the cache views perform the same write on the GPU: tests/test_gpu_write.py


def test_slot_mapping_out_of_table_and_negative_blocks():
    # seq 0: pos 3 -> block 3 off 3; pos 4 -> block -1 -> skipped.  seq 1: pos 7 -> block 1 off 3
    tables = np.array([[3, -1], [0, 1]], dtype=np.int32)
    exp, lens = write_positions(tables, [3, 7], [0, 2, 4], [0, 1], 4)
    assert exp.tolist()[:3] == [15, -1, 7] and lens.tolist() == [5, 9]


def test_cache_writes_refuse_host_tensors():
    """No host fallback: a view over CPU tensors refuses to write."""
    view = PageCacheView(key_cache=torch.zeros(4, 4, 1, 2), value_cache=torch.zeros(4, 4, 1, 2),
                         block_tables=torch.zeros(1, 4, dtype=torch.int32), kv_lens=torch.zeros(1, dtype=torch.int32),
                         block_size=4, num_kv_heads=1, head_dim=2)
    with pytest.raises(RuntimeError, match="GPU"):
        view.concatenate_to_cache(torch.zeros(1, 2, 2), torch.zeros(1, 1, 2), torch.zeros(1, 1, 2),
                                  cache_metadata=PageMetadata(query_start_loc=[0, 1]), slot_ids=[0])


def test_build_query_start_loc():
    assert build_query_start_loc([2, 0, 3]).tolist() == [0, 2, 2, 5]
    assert build_query_start_loc([]).tolist() == [0]


# ---------------------------------------------------------------- page layout
@pytest.mark.parametrize("bits", [4, 8])
def test_layout_round_trips(bits):
    rng = np.random.default_rng(bits)
    nb, bs, hkv, d, gs = 3, 128, 2, 128, 64
    x = rng.standard_normal((nb, bs, hkv, d)).astype(np.float16)
    c, s, b = affine_quantize(x, gs, bits)
    kp = layout.key_pages_from_logical(c)
    assert kp.shape == (nb, hkv, bs, d * bits // 32)
    np.testing.assert_array_equal(layout.key_logical_from_pages(kp), c)
    vp = layout.value_pages_from_logical(c, bits)
    t = min(bs, 256 // bits)
    assert vp.shape == (nb, hkv, bs // t, d, t * bits // 32)
    np.testing.assert_array_equal(layout.value_logical_from_pages(vp, bits), c)
    # value tile word w of dim j holds tokens w*per .. w*per+per-1 of that tile and dim:
    # 8-bit in byte order, 4-bit with token k at nibble (k >> 1) | ((k & 1) << 2)
    per = 32 // bits
    from oracle.affine import unpack_codes

    q = unpack_codes(c, bits)  # [nb, bs, hkv, d]
    shift = (lambda k: 4 * ((k >> 1) | ((k & 1) << 2))) if bits == 4 else (lambda k: 8 * k)
    m = (1 << bits) - 1
    for k in range(per):
        assert (int(vp[1, 1, 0, 5, 0]) >> shift(k)) & m == q[1, k, 1, 5]
    if bits == 4:
        assert (int(vp[1, 1, 0, 5, 0]) >> 4) & m == q[1, 2, 1, 5]   # nibble 1 holds token 2
        assert (int(vp[1, 1, 0, 5, 0]) >> 16) & m == q[1, 1, 1, 5]  # nibble 4 holds token 1
    if bs // t > 1:
        assert (vp[2, 0, 1, 7, 1] & m) == q[2, t + per, 0, 7]
    sp = layout.params_pages_from_logical(s)
    assert sp.shape == (nb, hkv, d // gs, bs) and sp[2, 1, 1, 7] == s[2, 7, 1, 1]
    np.testing.assert_array_equal(layout.params_logical_from_pages(sp), s)


# ---------------------------------------------------------------- operator plugin surface
def test_registry_and_requirements():
    from easymlx_amd.operations import OperationRegistry, UnifiedAttention
    from easymlx_amd.operations._base_operation import MetadataField

    for name in ("unified_attention", "unified", "paged", "full_attention", "linear_attention"):
        assert OperationRegistry.get(name) is UnifiedAttention
    with pytest.raises(KeyError):
        OperationRegistry.get("no_such_op")
    req = UnifiedAttention.get_requirements()
    for f in (MetadataField.QUERY_START_LOC, MetadataField.BLOCK_TABLES, MetadataField.KV_LENS,
              MetadataField.BLOCK_SIZE):
        assert f in req.required_metadata
    assert MetadataField.SLIDING_WINDOW in req.optional_metadata
    op = OperationRegistry.create("unified_attention")
    with pytest.raises(ValueError, match="requires cache_metadata"):
        op(query=torch.zeros(1, 2, 4), key=None, value=None, cache_metadata=None)
    with pytest.raises(ValueError, match="must be resolved"):
        op(query=torch.zeros(1, 2, 4), key=None, value=None, cache_metadata=PageMetadata(query_start_loc=[0, 1]))


def _dense_args(T=2, hq=4, hkv=2, d=8, nb=3, bs=4, S=2):
    return (torch.zeros(T, hq, d), torch.zeros(nb, bs, hkv, d), torch.zeros(nb, bs, hkv, d),
            torch.zeros(S, 2, dtype=torch.int32), torch.ones(S, dtype=torch.int32),
            torch.arange(S + 1, dtype=torch.int32))


def test_validation_messages():
    from easymlx_amd import paged_attention

    q, k, v, bt, kl, qsl = _dense_args()
    with pytest.raises(ValueError, match="queries must be rank-3"):
        paged_attention(q[0], k, v, bt, kl, qsl)
    with pytest.raises(ValueError, match="rank-4"):
        paged_attention(q, k[0], v, bt, kl, qsl)
    with pytest.raises(ValueError, match="same shape"):
        paged_attention(q, k, v[:2], bt, kl, qsl)
    with pytest.raises(ValueError, match="head_dim must match"):
        paged_attention(q[..., :4], k, v, bt, kl, qsl)
    with pytest.raises(ValueError, match="divisible by num_kv_heads"):
        paged_attention(q[:, :3], k, v, bt, kl, qsl)
    with pytest.raises(ValueError, match="block_tables must be rank-2"):
        paged_attention(q, k, v, bt[0], kl, qsl)
    with pytest.raises(ValueError, match="length num_seqs"):
        paged_attention(q, k, v, bt, kl, qsl[:-1])
    with pytest.raises(ValueError, match="affine caches need"):
        paged_attention(q, k, v, bt, kl, qsl, k_scales=torch.zeros(1))
    # affine codes in the logical (mlx.core.quantize) layout are converted on the device: no CPU path
    z = torch.zeros(1)
    with pytest.raises(RuntimeError, match="GPU only"):
        paged_attention(q, k.int(), v.int(), bt, kl, qsl, k_scales=z, k_biases=z, v_scales=z, v_biases=z, bits=4,
                        group_size=8)
    # zero tokens -> zeros without touching a device (unified_attention.py:1425-1426)
    out = paged_attention(torch.ones(0, 4, 8), k, v, bt, kl, torch.zeros(3, dtype=torch.int32))
    assert out.shape == (0, 4, 8)
    # no CPU fallback: a CPU tensor is refused loudly
    with pytest.raises(RuntimeError, match="GPU only"):
        paged_attention(q, k, v, bt, kl, qsl)


def test_single_token_decode_detection():
    from easymlx_amd.operations.unified_attention import _is_single_token_decode

    assert _is_single_token_decode(torch.tensor([0, 1, 2, 3]), 3)
    assert not _is_single_token_decode(torch.tensor([0, 2, 3]), 3)
    assert not _is_single_token_decode(torch.tensor([0, 1]), 0)
    assert not _is_single_token_decode(torch.tensor([1, 2, 3]), 2)


# ---------------------------------------------------------------- workloads
def test_workload_bytes_and_determinism():
    from easymlx_amd.workloads import config

    c2 = config("c2")
    assert (c2.num_seqs, c2.num_q_heads, c2.num_kv_heads, c2.head_dim, c2.block_size, c2.bits, c2.group_size) == \
        (32, 32, 8, 128, 128, 4, 64)
    assert c2.kv_lens.min() >= 512 and c2.kv_lens.max() <= 4096
    assert c2.kv_bytes() == int(c2.kv_lens.sum()) * 8 * 144  # 4-bit: 64 B codes + 8 B params, K and V
    c1 = config("c1")
    assert c1.bits == 8 and c1.kv_bytes() == int(c1.kv_lens.sum()) * 8 * 272
    again = config("c2")
    np.testing.assert_array_equal(again.kv_lens, c2.kv_lens)
    np.testing.assert_array_equal(again.block_tables, c2.block_tables)
    # every live token has its own slot (no two tokens share a page slot)
    assert len(np.unique(c2.slot)) == len(c2.slot) == int(c2.kv_lens.sum())


# ---------------------------------------------------------------- C ABI
def _header_functions():
    text = open(os.path.join(ROOT, "include", "emx_attn.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:int|size_t|const char\*)\s+(emx_\w+)\s*\(", text, flags=re.M)


@pytest.fixture(scope="module")
def lib():
    from easymlx_amd import _native

    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("libemx_attn.so not built (run __graft_entry__.build())")
    return _native.load()


def test_abi_exports_every_declared_symbol(lib):
    from easymlx_amd import _native

    names = _header_functions()
    assert set(names) == set(_native.SIGNATURES), (names, list(_native.SIGNATURES))
    for n in names:
        assert hasattr(lib, n), n
    assert lib.emx_version() >= 100


def test_abi_argument_errors(lib):
    from easymlx_amd import _native

    assert lib.emx_affine_quantize(None, 4, 128, 64, 3, None, None, None, None) == _native.EMX_ERR_UNSUPPORTED
    assert b"bits" in lib.emx_last_error()
    assert lib.emx_affine_quantize(None, 4, 100, 64, 4, None, None, None, None) == _native.EMX_ERR_INVALID
    assert lib.emx_affine_quantize(None, 0, 128, 64, 4, None, None, None, None) == _native.EMX_OK
    assert lib.emx_affine_quantize(None, 4, 128, 64, 4, None, None, None, None) == _native.EMX_ERR_INVALID
    with pytest.raises(ValueError):
        _native.check(_native.EMX_ERR_INVALID)
    with pytest.raises(NotImplementedError):
        _native.check(_native.EMX_ERR_UNSUPPORTED)
    with pytest.raises(RuntimeError):
        _native.check(_native.EMX_ERR_HIP)
    # decode workspace size is pure host arithmetic; 0 where neither the MFMA decode nor the split-K
    # path applies (head_dim not a multiple of 32, or pages not a multiple of 8 tokens)
    assert lib.emx_paged_workspace_bytes(32, 32, 8, 128, 32, 128) > 0
    assert lib.emx_paged_workspace_bytes(32, 32, 8, 64, 32, 128) > 0  # split-K
    assert lib.emx_paged_workspace_bytes(32, 32, 8, 48, 32, 128) == 0
    assert lib.emx_paged_workspace_bytes(32, 32, 8, 64, 32, 12) == 0


def test_abi_rope_and_prefill_split_arguments(lib):
    """Argument checks of the RoPE and key-split entry points run on the host (no device work)."""
    from easymlx_amd import _native

    err = _native.EMX_ERR_INVALID
    one = ctypes.c_int32(0)
    inv = ctypes.c_float(1.0)
    p_one, p_inv = ctypes.addressof(one), ctypes.addressof(inv)
    # rope_rows: zero rows is a no-op; odd or oversized rot_dims and missing tables are errors
    assert lib.emx_rope_rows(None, 0, 8, 128, None, None, 128, 0, None) == _native.EMX_OK
    assert lib.emx_rope_rows(p_one, 4, 8, 128, p_one, p_inv, 127, 0, None) == err
    assert lib.emx_rope_rows(p_one, 4, 8, 128, p_one, p_inv, 130, 0, None) == err
    assert lib.emx_rope_rows(p_one, 4, 8, 128, None, p_inv, 128, 0, None) == err
    assert b"rope" in lib.emx_last_error()
    # fused writes: the same checks before any pointer is touched; FP8 needs rot_dims % 8 (4 if traditional)
    args = [p_one, p_one, p_one, 4, 8, 128, 64, 4, 128, 16] + [p_one] * 6
    assert lib.emx_affine_cache_write_rope(*args, None, p_inv, 128, 0, None, None, 0, None) == err
    assert lib.emx_affine_cache_write_rope(*args, p_one, p_inv, 0, 0, None, None, 0, None) == err
    assert lib.emx_affine_cache_write_rope(*args, p_one, p_inv, 128, 0, None, p_one, 0, None) == err  # no q heads
    assert lib.emx_affine_cache_write_rope(*args, p_one, p_inv, 128, 0, p_one, None, 8, None) == err  # in, no out
    fargs = [p_one, p_one, _native.DTYPE_F16, p_one, 4, 8, 128, 128, 16, p_one, p_one, p_one, p_one, p_one, 2048]
    assert lib.emx_fp8_cache_write_rope(*fargs, p_one, p_inv, 12, 0, None, None, 0, None) == err
    assert lib.emx_fp8_cache_write_rope(*fargs, p_one, p_inv, 10, 1, None, None, 0, None) == err
    assert lib.emx_fp8_cache_write_rope(*fargs, p_one, p_inv, 128, 0, None, p_one, 0, None) == err  # no q heads
    assert lib.emx_fp8_cache_write_rope(*fargs, p_one, p_inv, 128, 0, p_one, None, 8, None) == err  # in, no out
    # FP8 writes index words with 32 bits: more than 2^33 values per tensor are refused before any launch
    big = list(fargs)
    big[4] = 1 << 24  # 2^24 tokens x 8 heads x 128 dims = 2^34 values
    assert lib.emx_fp8_cache_write(*big, None) == _native.EMX_ERR_UNSUPPORTED
    # prefill key-split workspace: host arithmetic, 0 where the split cannot apply, growing with the tokens
    c3 = lib.emx_paged_prefill_workspace_bytes(2076, 32, 32, 8, 128)
    assert c3 > 0 and c3 % 4 == 0
    assert lib.emx_paged_prefill_workspace_bytes(4152, 32, 32, 8, 128) > c3
    assert lib.emx_paged_prefill_workspace_bytes(2076, 32, 32, 8, 64) == 0    # head_dim 64: no MFMA prefill
    assert lib.emx_paged_prefill_workspace_bytes(2076, 32, 24, 8, 128) == 0   # GQA 3
    assert lib.emx_paged_prefill_workspace_bytes(0, 32, 32, 8, 128) == 0
    assert lib.emx_paged_prefill_workspace_bytes(10 ** 7, 32, 32, 8, 128) == 0  # counters would not fit


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 2 and "one GPU" in r.stdout


# ---------------------------------------------------------------- page lifecycle (host side)
def test_oracle_copy_and_zero_known_answers():
    from oracle.cache_write import copy_blocks, zero_pages

    a = np.arange(5 * 3, dtype=np.int32).reshape(5, 3)
    b = np.arange(5 * 2, dtype=np.float32).reshape(5, 2) + 100
    copy_blocks([a, b], [[0, 4], [2, 1], [7, 3], [3, 3]])  # (7, 3) skipped: past the pool; (3, 3) a no-op
    assert a.tolist() == [[0, 1, 2], [6, 7, 8], [6, 7, 8], [9, 10, 11], [0, 1, 2]]
    assert b[4].tolist() == [100, 101] and b[1].tolist() == [104, 105]
    # reads come from the arrays as they were: swapping two blocks in one call
    c = np.array([[1], [2]])
    copy_blocks([c], [[0, 1], [1, 0]])
    assert c.ravel().tolist() == [2, 1]
    zero_pages([a, b], [1, -1, 9, 4])
    assert a[1].tolist() == [0, 0, 0] and a[4].tolist() == [0, 0, 0] and a[2].tolist() == [6, 7, 8]
    assert b[1].tolist() == [0, 0] and b[0].tolist() == [100, 101]


def test_cache_dtype_validation_and_config():
    from easymlx_amd.caching.pagecache import CacheConfigError, PageCacheConfig, resolve_cache_dtype, validate_cache_dtype

    for ok in (None, "auto", "float16", "bfloat16", "float32", "fp8", "affine4", "affine8"):
        validate_cache_dtype(ok)
    for bad in ("int4", "fp16", "affine2", "q4"):
        with pytest.raises(CacheConfigError, match="Unsupported cache_dtype"):
            validate_cache_dtype(bad)
    with pytest.raises(CacheConfigError, match="TurboQuant"):
        validate_cache_dtype("turboquant3")
    with pytest.raises(CacheConfigError, match="contradicts"):
        validate_cache_dtype("affine4", cache_bits=8)
    assert resolve_cache_dtype("affine8") == ("affine", 8)
    assert resolve_cache_dtype("fp8") == ("fp8", None)
    assert resolve_cache_dtype(None) == ("float", None)
    cfg = PageCacheConfig.create(num_hidden_layers=2, num_kv_heads=8, head_dim=128, page_size=128, max_num_reqs=3,
                                 max_model_length=1000, cache_dtype="affine4")
    assert cfg.num_pages == 8 * 3  # ceil(1000 / 128) pages per request (cache.py:1358-1362)
    with pytest.raises(CacheConfigError):
        PageCacheConfig(num_hidden_layers=1, num_kv_heads=1, head_dim=64, cache_dtype="int8")


def test_block_mapping_checks():
    from easymlx_amd.caching.paged import block_mapping_on_device

    with pytest.raises(ValueError, match="rank-2"):
        block_mapping_on_device([1, 2, 3], "cpu")
    # chained / swapped pairs are valid (the kernel stages every source block before writing)
    assert block_mapping_on_device([[0, 1], [1, 2], [2, 0]], "cpu").tolist() == [[0, 1], [1, 2], [2, 0]]
    assert block_mapping_on_device([[0, 1], [2, 3], [4, 4]], "cpu").dtype == torch.int32


def test_copy_blocks_oracle_simultaneous_semantics():
    """The oracle reads every source as it was before the call (the reference kernel's separate outputs)."""
    from oracle import cache_write as ocw

    a = np.arange(5)[:, None].repeat(3, 1).astype(np.int32)
    ocw.copy_blocks([a], [[0, 1], [1, 0], [2, 3], [3, 4], [4, 2], [1, 4]])
    # swap 0<->1; 2->3, 3->4 then 1->4 (the later pair wins), 4->2: all from the old contents
    np.testing.assert_array_equal(a[:, 0], [1, 0, 4, 2, 1])
