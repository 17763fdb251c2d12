"""Decode attention over affine pages on the GPU vs the oracle (max-abs 2e-3 / rel 1e-2)."""

import numpy as np
import pytest
import torch

from easymlx_amd import paged_attention
from easymlx_amd.workloads import config, decode_workload
from tests.helpers import assert_attention_close, c_oracle_expected, gpu_cache, oracle_expected

pytestmark = pytest.mark.gpu


def _run(wl, view, cuda, **kw):
    q = torch.from_numpy(wl.q).to(cuda)
    out = paged_attention(
        q, view.k_codes, view.v_codes, view.block_tables, view.kv_lens,
        torch.from_numpy(wl.query_start_loc).to(cuda),
        k_scales=view.k_scales, k_biases=view.k_biases, v_scales=view.v_scales, v_biases=view.v_biases,
        bits=wl.bits, group_size=wl.group_size, single_token_decode=wl.single_token_decode, **kw,
    )
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


CASES = [
    # (bits, group, Hq, Hkv, ctx range, seqs)
    (4, 64, 32, 8, (512, 4096), 8),
    (8, 64, 32, 8, (512, 4096), 8),
    (4, 32, 16, 4, (1, 900), 5),
    (4, 128, 64, 4, (100, 2000), 3),
    (8, 128, 16, 16, (1, 300), 4),
    (4, 64, 64, 8, (3000, 5000), 2),
    (8, 32, 8, 2, (129, 129), 3),
    # 4-bit on the 4x4x4 kernel: GQA 1, 2, 16 and groups 64 / 128
    (4, 64, 8, 8, (1, 700), 4),
    (4, 128, 16, 8, (60, 3000), 5),
    (4, 64, 64, 4, (200, 2500), 3),
    # many short sequences: workgroup ranges spanning many whole units
    (4, 64, 32, 8, (1, 300), 96),
]


@pytest.mark.parametrize("case", CASES, ids=[f"b{c[0]}g{c[1]}hq{c[2]}hkv{c[3]}" for c in CASES])
def test_decode_matches_oracle(cuda, case):
    bits, gs, hq, hkv, ctx, seqs = case
    print(f"[decode {case}]", flush=True)
    wl = decode_workload(seed=hash(case) % 1000, num_seqs=seqs, num_q_heads=hq, num_kv_heads=hkv,
                         ctx_range=ctx, bits=bits, group_size=gs)
    view = gpu_cache(wl, cuda)
    assert_attention_close(_run(wl, view, cuda), oracle_expected(wl), str(case))


def test_decode_c2_full(cuda):
    """The north-star configuration at full size (batch 32, 4-bit, contexts 512..4096)."""
    print("[decode c2 full]", flush=True)
    wl = config("c2")
    view = gpu_cache(wl, cuda)
    assert_attention_close(_run(wl, view, cuda), oracle_expected(wl), "c2")


@pytest.mark.xfail(reason="MLX-style fp16 dequantization is not the parity target: rounding each dequantized "
                          "K/V element to fp16 moves c2 outputs by up to 4.5e-3 (2-3 of 131072 elements beyond "
                          "2e-3 + 1e-2|exp|); the kernels dequantize in fp32", strict=False)
def test_decode_c2_vs_fp16_dequant_target(cuda):
    """c2 against the oracle with each dequantized element rounded to fp16 (recorded, not required)."""
    print("[decode c2 vs fp16-dequant oracle]", flush=True)
    wl = config("c2")
    view = gpu_cache(wl, cuda)
    assert_attention_close(_run(wl, view, cuda), c_oracle_expected(wl, fp16_dequant=True), "c2 fp16-dequant")


@pytest.mark.timeout(400)
def test_decode_c4_full(cuda):
    """The c4 configuration exactly as bench.py times it: 8 x 32k tokens, Hq 64 / Hkv 8, 4096-page pool."""
    print("[decode c4 full]", flush=True)
    wl = config("c4")
    view = gpu_cache(wl, cuda)
    got = _run(wl, view, cuda)
    del view
    assert_attention_close(got, c_oracle_expected(wl), "c4")


def test_decode_c1_full(cuda):
    print("[decode c1 full]", flush=True)
    wl = config("c1")
    view = gpu_cache(wl, cuda)
    assert_attention_close(_run(wl, view, cuda), oracle_expected(wl), "c1")


def test_decode_long_context_split(cuda):
    """C4 shape (Hq 64 / Hkv 8, 32k context) on 2 sequences: many split-K partitions."""
    print("[decode c4-shape 2 seqs]", flush=True)
    wl = decode_workload("c4s", seed=4, num_seqs=2, num_q_heads=64, fixed_ctx=32768, pool_pages=600, bits=4)
    view = gpu_cache(wl, cuda)
    assert_attention_close(_run(wl, view, cuda), oracle_expected(wl), "c4-shape")


@pytest.mark.parametrize("seqs,ctx", [(64, (64, 512)), (40, (257, 512)), (300, (1, 256))],
                         ids=["short64", "two-item-units", "one-item-units"])
def test_decode_short_units_whole_ranges(cuda, seqs, ctx):
    """4-bit decode where every unit is at most two items: ranges end on unit starts (some empty), so no
    unit is split between workgroups."""
    print(f"[decode short units seqs={seqs} ctx={ctx}]", flush=True)
    wl = decode_workload(seed=31 + seqs, num_seqs=seqs, ctx_range=ctx, bits=4)
    view = gpu_cache(wl, cuda)
    got = _run(wl, view, cuda)
    assert_attention_close(got, oracle_expected(wl), f"short units {seqs}")
    assert np.array_equal(_run(wl, view, cuda), got), "repeat differs"


@pytest.mark.parametrize("seed,bits,hq,gs,seqs,ctx", [(331, 8, 32, 64, 300, (1, 256)), (332, 4, 64, 64, 300, (1, 256)),
                                                       (333, 8, 32, 32, 200, (1, 600)), (334, 4, 32, 64, 300, (1, 256))],
                         ids=["8bit", "4bit-gqa8", "8bit-g32", "4bit"])
def test_decode_bias_cancellation(cuda, seed, bits, hq, gs, seqs, ctx):
    """Short contexts over channels with large biases: outputs near zero come from sum P' * code cancelling
    sum p * v_bias, so P' = p * v_scale must enter the matrix core with more than fp16's 11 bits (these cases
    had 6 (4bit-gqa8) and 1 (4bit) elements outside the tolerance with a single fp16 P'; max err / tol is now
    0.05 - 0.31)."""
    print(f"[decode bias cancellation bits={bits} hq={hq} gs={gs}]", flush=True)
    wl = decode_workload(seed=seed, num_seqs=seqs, ctx_range=ctx, bits=bits, num_q_heads=hq, group_size=gs)
    view = gpu_cache(wl, cuda)
    assert_attention_close(_run(wl, view, cuda), oracle_expected(wl), f"bias cancellation {bits}/{hq}/{gs}")


def test_decode_sliding_window(cuda):
    print("[decode sliding window]", flush=True)
    wl = decode_workload(seed=8, num_seqs=6, ctx_range=(10, 2000), bits=4)
    view = gpu_cache(wl, cuda)
    for window in (1, 100, 700, 5000):
        got = _run(wl, view, cuda, sliding_window=window)
        assert_attention_close(got, oracle_expected(wl, sliding_window=window), f"window {window}")


def test_decode_edge_lengths_and_invalid_pages(cuda):
    """kv_len 0 -> zeros; block id -1 / out of range pages are skipped like the Metal kernel."""
    print("[decode edge lengths]", flush=True)
    wl = decode_workload(seed=13, num_seqs=5, ctx_range=(300, 1200), bits=4)
    view = gpu_cache(wl, cuda)
    lens = wl.kv_lens.copy()
    lens[1] = 0
    tables = wl.block_tables.copy()
    tables[2, 1] = -1
    tables[3, 0] = wl.num_blocks + 7
    view.kv_lens.copy_(torch.from_numpy(lens))
    view.block_tables.copy_(torch.from_numpy(tables))
    got = _run(wl, view, cuda)
    exp = oracle_expected(wl, block_tables=tables, kv_lens=lens)
    assert_attention_close(got, exp, "edges")
    assert np.all(got[1] == 0)


def test_decode_repeat_reuses_workspace(cuda):
    """Split-K tickets return to zero: repeated launches give identical results."""
    print("[decode repeat]", flush=True)
    wl = decode_workload(seed=17, num_seqs=4, ctx_range=(2000, 4096), bits=4)
    view = gpu_cache(wl, cuda)
    first = _run(wl, view, cuda)
    for _ in range(3):
        np.testing.assert_array_equal(_run(wl, view, cuda), first)


SMALL_PAGE_CASES = [
    # (page, Hq, Hkv, ctx range, seqs, window)
    (16, 32, 8, (512, 4096), 32, 0),   # the c2 batch at the reference's default page size
    (16, 8, 8, (1, 700), 9, 0),        # GQA 1, lengths not a multiple of the page
    (32, 16, 8, (60, 3000), 6, 0),     # GQA 2
    (64, 64, 4, (200, 2500), 4, 0),    # GQA 16
    (16, 32, 8, (100, 2000), 7, 333),  # sliding window inside a page
    (32, 32, 8, (1, 300), 80, 0),      # many one-item units
]


@pytest.mark.parametrize("case", SMALL_PAGE_CASES, ids=[f"p{c[0]}hq{c[1]}hkv{c[2]}w{c[5]}" for c in SMALL_PAGE_CASES])
def test_decode_small_pages(cuda, case):
    """4-bit decode over pages of 16 / 32 / 64 tokens (a 64-token slice spans several pages) vs the oracle,
    and a repeat on the cached plan bit for bit."""
    bs, hq, hkv, ctx, seqs, window = case
    print(f"[decode small pages {case}]", flush=True)
    wl = decode_workload(seed=600 + bs + seqs, num_seqs=seqs, num_q_heads=hq, num_kv_heads=hkv, ctx_range=ctx,
                         bits=4, group_size=64, block_size=bs)
    view = gpu_cache(wl, cuda)
    kw = {"sliding_window": window} if window else {}
    got = _run(wl, view, cuda, **kw)
    assert_attention_close(got, oracle_expected(wl, sliding_window=window), f"small pages {case}")
    assert np.array_equal(_run(wl, view, cuda, **kw), got), "repeat differs"


def test_decode_small_pages_invalid_pages(cuda):
    """Page 16: an unassigned page (-1) and one past the pool inside a slice are skipped, as the Metal kernel
    skips block < 0; kv_len 0 gives zeros."""
    print("[decode small pages invalid]", flush=True)
    wl = decode_workload(seed=77, num_seqs=5, ctx_range=(300, 1200), bits=4, block_size=16)
    view = gpu_cache(wl, cuda)
    lens = wl.kv_lens.copy()
    lens[1] = 0
    tables = wl.block_tables.copy()
    tables[2, 3] = -1
    tables[3, 5] = wl.num_blocks + 7
    view.kv_lens.copy_(torch.from_numpy(lens))
    view.block_tables.copy_(torch.from_numpy(tables))
    got = _run(wl, view, cuda)
    exp = oracle_expected(wl, block_tables=tables, kv_lens=lens)
    assert_attention_close(got, exp, "small pages invalid")
    assert not got[1].any()
