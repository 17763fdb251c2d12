"""FP8 (E4M3) cache: GPU write bit-exact vs the oracle; attention over it vs the oracle."""

import numpy as np
import pytest
import torch

from easymlx_amd import Fp8PageCacheView, UnifiedAttention, paged_attention
from easymlx_amd.caching.paged import PageMetadata
from easymlx_amd.workloads import decode_workload, unified_workload
from oracle import fp8
from oracle.paged_attention import paged_attention as oracle_attention
from tests.helpers import assert_attention_close

pytestmark = pytest.mark.gpu


def _view(wl, device):
    nb = wl.num_blocks
    shape = (nb, wl.block_size, wl.num_kv_heads, wl.head_dim)
    return Fp8PageCacheView(
        key_cache=torch.zeros(shape, dtype=torch.uint8, device=device),
        value_cache=torch.zeros(shape, dtype=torch.uint8, device=device),
        k_scales=torch.zeros((nb,), dtype=torch.float32, device=device),
        v_scales=torch.zeros((nb,), dtype=torch.float32, device=device),
        block_tables=torch.from_numpy(wl.block_tables).to(device),
        kv_lens=torch.from_numpy(wl.kv_lens).to(device),
        block_size=wl.block_size,
        num_kv_heads=wl.num_kv_heads,
        head_dim=wl.head_dim,
    )


def _write_per_sequence(wl, view, dtype, hold_last: bool):
    """One write call per sequence (each its own scale); the oracle replays the same calls.

    hold_last: the last token of every sequence is held back and written in one
    final call for all sequences (a decode step), which raises page scales.
    """
    shape = (wl.num_blocks, wl.block_size, wl.num_kv_heads, wl.head_dim)
    kc, vc = np.zeros(shape, np.uint8), np.zeros(shape, np.uint8)
    ks, vs = np.zeros(wl.num_blocks, np.float32), np.zeros(wl.num_blocks, np.float32)
    bounds = np.concatenate([[0], np.cumsum(wl.kv_lens)])
    last = []
    dev = view.key_cache.device
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[dtype]

    def call(idx):
        k = torch.from_numpy(wl.k[idx]).to(dev).to(tdt)
        v = torch.from_numpy(wl.v[idx]).to(dev).to(tdt)
        slot = wl.slot[idx].astype(np.int32)
        view.write_slots(k, v, torch.from_numpy(slot).to(dev))
        # the oracle sees exactly the values the GPU converted
        fp8.fp8_write(k.float().cpu().numpy(), v.float().cpu().numpy(), slot, kc, vc, ks, vs)

    for s in range(len(wl.kv_lens)):
        lo, hi = int(bounds[s]), int(bounds[s + 1])
        if hi == lo:
            continue
        if hold_last:
            last.append(hi - 1)
            hi -= 1
        if hi > lo:
            call(np.arange(lo, hi))
    if last:
        call(np.array(last))
    return kc, vc, ks, vs


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
def test_fp8_write_bit_exact(cuda, dtype):
    print(f"[fp8 write {dtype}]", flush=True)
    wl = decode_workload(seed=21, num_seqs=6, num_q_heads=8, num_kv_heads=2, head_dim=64, ctx_range=(5, 300),
                         block_size=32, bits=None)
    view = _view(wl, cuda)
    kc, vc, ks, vs = _write_per_sequence(wl, view, dtype, hold_last=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(view.key_cache.cpu().numpy(), kc)
    np.testing.assert_array_equal(view.value_cache.cpu().numpy(), vc)
    np.testing.assert_array_equal(view.k_scales.cpu().numpy(), ks)
    np.testing.assert_array_equal(view.v_scales.cpu().numpy(), vs)


@pytest.mark.parametrize("t", [4096, 32])
def test_fp8_write_skips_and_large_batch(cuda, t):
    """A 4096-token write (several workgroups in the max pass) and a 32-token one-launch write, with skipped
    slots: -1 and pages outside the pool (large values there must not enter the call's scale)."""
    print(f"[fp8 write skips t={t}]", flush=True)
    rng = np.random.default_rng(3)
    nb, bs, hkv, d = 64, 128, 4, 128
    k = (rng.standard_normal((t, hkv, d)) * rng.uniform(0.1, 8.0, (1, hkv, d))).astype(np.float16)
    v = rng.standard_normal((t, hkv, d)).astype(np.float16)
    slot = rng.permutation(nb * bs)[:t].astype(np.int32)
    slot[rng.random(t) < 0.1] = -1
    out_of_pool = rng.random(t) < 0.05
    out_of_pool[0] = True
    slot[out_of_pool] = nb * bs + rng.integers(0, 5 * bs, int(out_of_pool.sum()))
    k[out_of_pool] = 3000.0
    v[out_of_pool] = -3000.0
    shape = (nb, bs, hkv, d)
    view = Fp8PageCacheView(key_cache=torch.zeros(shape, dtype=torch.uint8, device=cuda),
                            value_cache=torch.zeros(shape, dtype=torch.uint8, device=cuda),
                            k_scales=torch.zeros(nb, device=cuda), v_scales=torch.zeros(nb, device=cuda),
                            block_tables=torch.zeros((1, 1), dtype=torch.int32, device=cuda),
                            kv_lens=torch.zeros(1, dtype=torch.int32, device=cuda), block_size=bs,
                            num_kv_heads=hkv, head_dim=d)
    view.write_slots(torch.from_numpy(k).to(cuda), torch.from_numpy(v).to(cuda), torch.from_numpy(slot).to(cuda))
    kc, vc = np.zeros(shape, np.uint8), np.zeros(shape, np.uint8)
    ks, vs = np.zeros(nb, np.float32), np.zeros(nb, np.float32)
    fp8.fp8_write(k.astype(np.float32), v.astype(np.float32), slot, kc, vc, ks, vs)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(view.key_cache.cpu().numpy(), kc)
    np.testing.assert_array_equal(view.value_cache.cpu().numpy(), vc)
    np.testing.assert_array_equal(view.k_scales.cpu().numpy(), ks)
    np.testing.assert_array_equal(view.v_scales.cpu().numpy(), vs)


def _attention_case(cuda, wl, hold_last, sliding_window=0):
    view = _view(wl, cuda)
    kc, vc, ks, vs = _write_per_sequence(wl, view, "f16", hold_last=hold_last)
    q = torch.from_numpy(wl.q).to(cuda)
    out = paged_attention(q, view.key_cache, view.value_cache, view.block_tables, view.kv_lens,
                          torch.from_numpy(wl.query_start_loc).to(cuda), k_scale=view.k_scales,
                          v_scale=view.v_scales, sliding_window=sliding_window or None)
    torch.cuda.synchronize()
    exp = oracle_attention(wl.q.astype(np.float32), fp8.fp8_dequant_cache(kc, ks), fp8.fp8_dequant_cache(vc, vs),
                           wl.block_tables, wl.kv_lens, wl.query_start_loc, sliding_window=sliding_window,
                           compute_dtype=np.float64)
    return out, exp, view


def test_fp8_decode_vs_oracle(cuda):
    print("[fp8 decode]", flush=True)
    wl = decode_workload(seed=22, num_seqs=16, ctx_range=(1, 1500), bits=None)
    out, exp, _ = _attention_case(cuda, wl, hold_last=True)
    assert_attention_close(out.float().cpu().numpy(), exp, "fp8 decode")


@pytest.mark.parametrize("seed,hq", [(501, 32), (502, 64)])
def test_fp8_decode_short_contexts_stress(cuda, seed, hq):
    """Many short contexts over channels with gains up to 4: outputs near zero from large values of both
    signs (P in fp16 against fp32 values; max err / tol 0.51 and 0.44 when added)."""
    print(f"[fp8 decode short stress seed={seed} hq={hq}]", flush=True)
    wl = decode_workload(seed=seed, num_seqs=300, ctx_range=(1, 256), bits=None, num_q_heads=hq)
    out, exp, _ = _attention_case(cuda, wl, hold_last=True)
    assert_attention_close(out.float().cpu().numpy(), exp, "fp8 short stress")


def test_fp8_unified_vs_oracle(cuda):
    print("[fp8 unified]", flush=True)
    wl = unified_workload("fp8u", seed=23, num_prefill=2, chunk=96, prior_range=(0, 300), num_decode=5,
                          decode_ctx=(1, 700), bits=None)
    out, exp, _ = _attention_case(cuda, wl, hold_last=False)
    assert_attention_close(out.float().cpu().numpy(), exp, "fp8 unified")
    out, exp, _ = _attention_case(cuda, wl, hold_last=False, sliding_window=64)
    assert_attention_close(out.float().cpu().numpy(), exp, "fp8 unified window")
    # long contexts: prefill tiles split over workgroups and merged in-kernel
    wl = unified_workload("fp8long", seed=26, num_prefill=2, chunk=100, prior_range=(1500, 2500), num_decode=3,
                          decode_ctx=(1, 2000), bits=None)
    out, exp, _ = _attention_case(cuda, wl, hold_last=False)
    assert_attention_close(out.float().cpu().numpy(), exp, "fp8 unified long")


def test_fp8_registered_op(cuda):
    """UnifiedAttention routes an FP8 cache view to the per-page scales (unified_attention.py:1633-1656)."""
    print("[fp8 op]", flush=True)
    wl = decode_workload(seed=24, num_seqs=8, ctx_range=(16, 900), bits=None)
    out_ref, exp, view = _attention_case(cuda, wl, hold_last=True)
    md = PageMetadata(query_start_loc=torch.from_numpy(wl.query_start_loc).to(cuda), block_tables=view.block_tables,
                      kv_lens=view.kv_lens, block_size=wl.block_size, is_single_token_decode=True)
    res = UnifiedAttention().forward_native(query=torch.from_numpy(wl.q).to(cuda), key=view.key_cache,
                                            value=view.value_cache, cache_metadata=md, cache_view=view)
    torch.cuda.synchronize()
    assert torch.equal(res.attention_outputs, out_ref)
    assert_attention_close(res.attention_outputs.float().cpu().numpy(), exp, "fp8 op")


@pytest.mark.parametrize("hq,hkv,bs", [(8, 8, 32), (16, 8, 64), (64, 8, 128), (32, 2, 32)])
def test_fp8_decode_gqa_and_page_sizes(cuda, hq, hkv, bs):
    """Split-K FP8 decode over GQA 1/2/8/16 and pages of 32/64/128 tokens."""
    print(f"[fp8 decode hq={hq} hkv={hkv} bs={bs}]", flush=True)
    wl = decode_workload(seed=25 + hq + bs, num_seqs=7, num_q_heads=hq, num_kv_heads=hkv, block_size=bs,
                         ctx_range=(1, 900), bits=None)
    out, exp, _ = _attention_case(cuda, wl, hold_last=True)
    assert_attention_close(out.float().cpu().numpy(), exp, f"fp8 decode {hq}/{hkv} bs {bs}")


def test_fp8_decode_window_and_long_context(cuda):
    """40,000-token contexts: more than 16 pieces per unit (two-level merge); then a sliding window."""
    print("[fp8 decode long]", flush=True)
    wl = decode_workload(seed=31, num_seqs=2, fixed_ctx=40000, bits=None)
    out, exp, _ = _attention_case(cuda, wl, hold_last=True)
    assert_attention_close(out.float().cpu().numpy(), exp, "fp8 decode long")
    wl = decode_workload(seed=32, num_seqs=9, ctx_range=(1, 2000), bits=None)
    out, exp, _ = _attention_case(cuda, wl, hold_last=True, sliding_window=200)
    assert_attention_close(out.float().cpu().numpy(), exp, "fp8 decode window")


def test_fp8_decode_edge_lengths_and_invalid_pages(cuda):
    """kv_len 0 -> zeros; block id -1 / out-of-range pages are skipped like the reference's Metal kernel."""
    print("[fp8 decode edges]", flush=True)
    wl = decode_workload(seed=27, num_seqs=5, ctx_range=(300, 1200), bits=None)
    view = _view(wl, cuda)
    kc, vc, ks, vs = _write_per_sequence(wl, view, "f16", hold_last=True)
    lens = wl.kv_lens.copy()
    lens[1] = 0
    tables = wl.block_tables.copy()
    tables[2, 1] = -1
    tables[3, 0] = wl.num_blocks + 7
    bt = torch.from_numpy(tables).to(cuda)
    kl = torch.from_numpy(lens).to(cuda)
    out = paged_attention(torch.from_numpy(wl.q).to(cuda), view.key_cache, view.value_cache, bt, kl,
                          torch.from_numpy(wl.query_start_loc).to(cuda), k_scale=view.k_scales,
                          v_scale=view.v_scales).float().cpu().numpy()
    exp = oracle_attention(wl.q.astype(np.float32), fp8.fp8_dequant_cache(kc, ks), fp8.fp8_dequant_cache(vc, vs),
                           tables, lens, wl.query_start_loc, compute_dtype=np.float64)
    assert_attention_close(out, exp, "fp8 edges")
    assert np.all(out[1] == 0)


@pytest.mark.parametrize("qdtype,hq,hkv,d", [("bf16", 32, 8, 128), ("f32", 12, 4, 64), ("f16", 24, 8, 128)],
                         ids=["bf16-queries", "f32-d64", "gqa3"])
def test_fp8_generic_shapes_vs_oracle(cuda, qdtype, hq, hkv, d):
    """Shapes outside the MFMA paths (bf16 / fp32 queries, head_dim 64, GQA 3) on the generic kernel's FP8
    loader: a ragged batch of prefill chunks and decode rows vs the oracle."""
    print(f"[fp8 generic {qdtype} {hq}/{hkv} d={d}]", flush=True)
    wl = unified_workload("fp8g", seed=28 + hq, num_prefill=2, chunk=40, prior_range=(0, 200), num_decode=4,
                          decode_ctx=(1, 600), num_q_heads=hq, num_kv_heads=hkv, head_dim=d, bits=None)
    view = _view(wl, cuda)
    kc, vc, ks, vs = _write_per_sequence(wl, view, "f16", hold_last=False)
    tdt = {"bf16": torch.bfloat16, "f32": torch.float32, "f16": torch.float16}[qdtype]
    q = torch.from_numpy(wl.q).to(cuda).to(tdt)
    out = paged_attention(q, view.key_cache, view.value_cache, view.block_tables, view.kv_lens,
                          torch.from_numpy(wl.query_start_loc).to(cuda), k_scale=view.k_scales, v_scale=view.v_scales)
    torch.cuda.synchronize()
    assert out.dtype == tdt
    exp = oracle_attention(q.float().cpu().numpy(), fp8.fp8_dequant_cache(kc, ks), fp8.fp8_dequant_cache(vc, vs),
                           wl.block_tables, wl.kv_lens, wl.query_start_loc, compute_dtype=np.float64)
    assert_attention_close(out.float().cpu().numpy(), exp, f"fp8 generic {qdtype}")
