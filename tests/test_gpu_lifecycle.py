"""Cache allocation and page lifecycle on the GPU: PageCacheConfig / PageCache.init_cache for every cache_dtype,
copy-on-write block copies and page zeroing (bit-exact against oracle.cache_write over every array of the cache),
reset / clear, and attention over copied pages."""

import numpy as np
import pytest
import torch

from easymlx_amd import (AffinePageCacheView, Fp8PageCacheView, PageCache, PageCacheConfig, PageCacheView,
                         PageMetadata, paged_attention)
from oracle import cache_write as ocw

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cache_dtype,cls", [(None, PageCacheView), ("bfloat16", PageCacheView),
                                             ("fp8", Fp8PageCacheView), ("affine4", AffinePageCacheView),
                                             ("affine8", AffinePageCacheView)])
def test_init_cache_per_layer(cuda, cache_dtype, cls):
    print(f"[init_cache {cache_dtype}]", flush=True)
    cfg = PageCacheConfig(num_hidden_layers=3, num_kv_heads=4, head_dim=128, page_size=64, max_num_reqs=5,
                          max_model_length=300, cache_dtype=cache_dtype, device=cuda)
    cache = PageCache.init_cache(cfg)
    assert len(cache) == 3 and all(type(v) is cls for v in cache)
    v = cache[0]
    assert v.num_blocks == cfg.num_pages == 5 * 5
    assert v.block_tables.tolist() == np.arange(25).reshape(5, 5).tolist()  # contiguous tables (cache.py:779-786)
    assert v.kv_lens.tolist() == [0] * 5
    assert all(not t.any() for t in v.page_arrays())
    if cls is AffinePageCacheView:
        assert v.bits == int(cache_dtype[-1]) and v.group_size == 64
    if cache_dtype == "bfloat16":
        assert v.key_cache.dtype == torch.bfloat16
    assert cache[0].key_cache.data_ptr() != cache[1].key_cache.data_ptr()


def _filled(kind, cuda, rng):
    S, hkv, d, bs = 4, 2, 128, 64
    if kind == "dense":
        v = PageCacheView.init(num_seqs=S, max_seq_len=4 * bs, num_kv_heads=hkv, head_dim=d, block_size=bs,
                               device=cuda)
    elif kind == "fp8":
        v = Fp8PageCacheView.init(num_seqs=S, max_seq_len=4 * bs, num_kv_heads=hkv, head_dim=d, block_size=bs,
                                  device=cuda)
    else:
        v = AffinePageCacheView.init(num_seqs=S, max_seq_len=4 * bs, num_kv_heads=hkv, head_dim=d, block_size=bs,
                                     bits=int(kind[-1]), group_size=64, device=cuda)
    for s in range(S):  # fill every page with distinct data through the write path
        n = 4 * bs
        k = torch.from_numpy(rng.standard_normal((n, hkv, d)).astype(np.float16)).to(cuda)
        val = torch.from_numpy(rng.standard_normal((n, hkv, d)).astype(np.float16)).to(cuda)
        v.append(s, k, val)
    torch.cuda.synchronize()
    return v


@pytest.mark.parametrize("kind", ["dense", "fp8", "affine4", "affine8"])
def test_copy_blocks_and_zero_pages_match_oracle(cuda, kind):
    print(f"[copy / zero {kind}]", flush=True)
    rng = np.random.default_rng(len(kind))
    view = _filled(kind, cuda, rng)
    arrays = [t.cpu().numpy() for t in view.page_arrays()]
    mapping = [[0, 9], [3, 12], [15, 2], [4, 4], [1, 99]]  # a no-op pair and one past the pool
    view.copy_blocks(mapping)
    ocw.copy_blocks(arrays, mapping)
    torch.cuda.synchronize()
    for t, a in zip(view.page_arrays(), arrays):
        np.testing.assert_array_equal(t.cpu().numpy(), a)
    # a device mapping takes the same path without host checks
    dm = torch.tensor([[5, 6], [7, 8]], dtype=torch.int32, device=cuda)
    view.copy_blocks(dm)
    ocw.copy_blocks(arrays, dm.cpu().numpy())
    pages = [9, -1, 13, 200, 0]
    view.zero_pages(pages)
    ocw.zero_pages(arrays, pages)
    torch.cuda.synchronize()
    for t, a in zip(view.page_arrays(), arrays):
        np.testing.assert_array_equal(t.cpu().numpy(), a)


@pytest.mark.parametrize("kind", ["dense", "fp8", "affine4"])
def test_copy_blocks_swaps_and_chains(cuda, kind):
    """Swapped, chained and repeated destinations: every destination gets its source as it was before the call
    (cache.py:95-136 reads its inputs); of two pairs with one destination the later counts."""
    print(f"[copy swaps / chains {kind}]", flush=True)
    rng = np.random.default_rng(40 + len(kind))
    view = _filled(kind, cuda, rng)
    arrays = [t.cpu().numpy() for t in view.page_arrays()]
    for mapping in ([[0, 1], [1, 0]],                      # swap
                    [[2, 3], [3, 4], [4, 5], [5, 2]],      # a 4-cycle
                    [[6, 7], [7, 8], [8, 9]],              # a chain
                    [[10, 11], [12, 11], [11, 13], [1, 99], [-1, 3]]):  # repeated destination, skipped ids
        view.copy_blocks(mapping)
        ocw.copy_blocks(arrays, mapping)
        torch.cuda.synchronize()
        for t, a in zip(view.page_arrays(), arrays):
            np.testing.assert_array_equal(t.cpu().numpy(), a, err_msg=str(mapping))
        dm = torch.tensor(mapping[::-1], dtype=torch.int32, device=cuda)  # and as a device tensor
        view.copy_blocks(dm)
        ocw.copy_blocks(arrays, mapping[::-1])
        torch.cuda.synchronize()
        for t, a in zip(view.page_arrays(), arrays):
            np.testing.assert_array_equal(t.cpu().numpy(), a, err_msg=f"device {mapping[::-1]}")


@pytest.mark.parametrize("kind", ["dense", "affine4"])
def test_reset_and_clear(cuda, kind):
    print(f"[reset / clear {kind}]", flush=True)
    rng = np.random.default_rng(9)
    view = _filled(kind, cuda, rng)
    arrays = [t.cpu().numpy() for t in view.page_arrays()]
    view.block_tables[2, 1] = -1  # an unassigned page in the row is skipped
    tables = view.block_tables.cpu().numpy()
    view.reset(2)
    ocw.zero_pages(arrays, tables[2])
    torch.cuda.synchronize()
    assert view.kv_lens.tolist() == [256, 256, 0, 256]
    for t, a in zip(view.page_arrays(), arrays):
        np.testing.assert_array_equal(t.cpu().numpy(), a)
    view.reset_batch([0, 3])
    assert view.kv_lens.tolist() == [0, 256, 0, 0]
    view.clear()
    torch.cuda.synchronize()
    assert view.kv_lens.tolist() == [0] * 4 and all(not t.any() for t in view.page_arrays())


@pytest.mark.parametrize("kind", ["affine4", "fp8"])
def test_attention_over_copied_pages(cuda, kind):
    """Copy-on-write: a second sequence whose table points at copies of the first's pages attends exactly as the
    first does (its copies are bit-identical), through the registered op's kernels."""
    print(f"[cow attention {kind}]", flush=True)
    rng = np.random.default_rng(3)
    view = _filled(kind, cuda, rng)
    src = view.block_tables[0].tolist()
    dst = view.block_tables[1].tolist()
    view.copy_blocks([[a, b] for a, b in zip(src, dst)])
    q = torch.from_numpy(rng.standard_normal((1, 8, 128)).astype(np.float16)).to(cuda)
    qq = torch.cat([q, q])
    qsl = torch.tensor([0, 1, 2], dtype=torch.int32, device=cuda)
    tables, lens = view.block_tables[:2].contiguous(), view.kv_lens[:2].contiguous()
    if kind == "fp8":
        out = paged_attention(qq, view.key_cache, view.value_cache, tables, lens, qsl, k_scale=view.k_scales,
                              v_scale=view.v_scales, single_token_decode=True)
    else:
        out = paged_attention(qq, view.key_cache, view.value_cache, tables, lens, qsl, k_scales=view.k_scales,
                              k_biases=view.k_biases, v_scales=view.v_scales, v_biases=view.v_biases, bits=4,
                              group_size=64, single_token_decode=True)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all() and out.abs().sum() > 0
    assert torch.equal(out[0], out[1])


@pytest.mark.parametrize("kind", ["dense", "fp8", "affine4", "affine8"])
def test_gather_kv_cache_matches_oracle(cuda, kind):
    """gather_kv_cache (cache.py:974-1027) against the oracle's dequantized logical pages."""
    from oracle.affine import affine_dequantize
    from oracle.fp8 import fp8_dequant_cache
    from tests.helpers import gpu_pages_to_logical

    print(f"[gather {kind}]", flush=True)
    rng = np.random.default_rng(11)
    view = _filled(kind, cuda, rng)
    S, bs = view.num_seqs, view.block_size
    lens = [200, 0, 256, 37]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    bt = view.block_tables.cpu().numpy().copy()
    bt[3, 0] = -1  # an unassigned page gathers zeros
    k, v = view.gather_kv_cache(torch.from_numpy(bt), torch.from_numpy(cu), out_dtype=torch.float32)
    torch.cuda.synchronize()
    if kind == "dense":
        lk, lv = view.key_cache.float().cpu().numpy(), view.value_cache.float().cpu().numpy()
    elif kind == "fp8":
        lk = fp8_dequant_cache(view.key_cache.cpu().numpy(), view.k_scales.cpu().numpy())
        lv = fp8_dequant_cache(view.value_cache.cpu().numpy(), view.v_scales.cpu().numpy())
    else:
        pages = gpu_pages_to_logical(view)
        lk = affine_dequantize(*pages["k"], view.group_size, view.bits, round_to_fp16=False)
        lv = affine_dequantize(*pages["v"], view.group_size, view.bits, round_to_fp16=False)
    exp_k = np.zeros((cu[-1],) + lk.shape[2:], np.float32)
    exp_v = np.zeros_like(exp_k)
    for b in range(S):
        for j in range(lens[b]):
            blk = bt[b, j // bs]
            if blk >= 0:
                exp_k[cu[b] + j] = lk[blk, j % bs]
                exp_v[cu[b] + j] = lv[blk, j % bs]
    np.testing.assert_array_equal(k.cpu().numpy(), exp_k)
    np.testing.assert_array_equal(v.cpu().numpy(), exp_v)
    assert view.gather_kv_cache(torch.from_numpy(bt), torch.from_numpy(cu))[0].dtype == (
        torch.float16 if kind != "dense" else view.key_cache.dtype)
