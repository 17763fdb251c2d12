"""Multi-token (prefill) and mixed batches on the MFMA paths vs the oracle.

Ragged batches are split on the device: rows of sequences with more than one
query token go to the prefill kernel, single-token rows to the split-K decode
kernel.  Expected values: the float64 oracle over the oracle-quantized cache
(``tests/helpers.py``), tolerance max-abs 2e-3 + rel 1e-2.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from easymlx_amd import paged_attention
from easymlx_amd.workloads import config, unified_workload
from helpers import assert_attention_close, c_oracle_expected, gpu_cache, oracle_expected

pytestmark = pytest.mark.gpu


def _run(wl, view, device, *, sliding_window=0, kv_lens=None):
    q = torch.from_numpy(wl.q).to(device)
    out = paged_attention(q, view.k_codes, view.v_codes, view.block_tables,
                          view.kv_lens if kv_lens is None else kv_lens,
                          torch.from_numpy(wl.query_start_loc).to(device), k_scales=view.k_scales,
                          k_biases=view.k_biases, v_scales=view.v_scales, v_biases=view.v_biases, bits=wl.bits,
                          group_size=wl.group_size, single_token_decode=False, sliding_window=sliding_window)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def test_c3_slice_full_chunks(cuda):
    """C3 structure with full 512-token chunks: 2 prefill chunks (prior 0..2048) + 6 decode rows."""
    print("[prefill c3 slice]", flush=True)
    wl = unified_workload("c3s", seed=3, num_prefill=2, chunk=512, prior_range=(0, 2048), num_decode=6,
                          decode_ctx=(256, 4096), bits=4)
    view = gpu_cache(wl, cuda)
    assert_attention_close(_run(wl, view, cuda), oracle_expected(wl), "c3 slice")


@pytest.mark.timeout(300)
def test_c3_full(cuda):
    """The c3 configuration exactly as bench.py times it (4 x 512-token chunks + 28 decode rows), with the
    prefill key split on (bench-sized workspace), against the C oracle."""
    print("[prefill c3 full]", flush=True)
    wl = config("c3")
    view = gpu_cache(wl, cuda)
    assert_attention_close(_run(wl, view, cuda), c_oracle_expected(wl), "c3 full")


@pytest.mark.parametrize("window", [0, 1, 77, 600])
def test_single_sequence_prefill(cuda, window):
    """One sequence, no prior context (the reference's single-sequence causal path), with windows."""
    print(f"[prefill single window={window}]", flush=True)
    wl = unified_workload("single", seed=11, num_prefill=1, chunk=300, prior_range=(0, 0), num_decode=0, bits=4)
    view = gpu_cache(wl, cuda)
    assert_attention_close(_run(wl, view, cuda, sliding_window=window),
                           oracle_expected(wl, sliding_window=window), f"single w{window}")


@pytest.mark.parametrize("hq,hkv,gs,bits", [(8, 8, 64, 4), (16, 8, 128, 4), (64, 8, 64, 4), (32, 8, 32, 4),
                                           (32, 8, 64, 8), (16, 2, 32, 8)],
                         ids=["gqa1", "gqa2-g128", "gqa8", "g32", "8bit", "8bit-gqa8-g32"])
def test_prefill_shapes(cuda, hq, hkv, gs, bits):
    print(f"[prefill shape hq={hq} hkv={hkv} gs={gs} bits={bits}]", flush=True)
    wl = unified_workload("shape", seed=hq + hkv + gs + bits, num_prefill=3, chunk=133, prior_range=(0, 400),
                          num_decode=3, decode_ctx=(1, 500), num_q_heads=hq, num_kv_heads=hkv, bits=bits,
                          group_size=gs)
    view = gpu_cache(wl, cuda)
    assert_attention_close(_run(wl, view, cuda), oracle_expected(wl), f"shape {hq}/{hkv}/{gs}/{bits}")


@pytest.mark.parametrize("bits,hq", [(4, 32), (8, 32), (4, 64)], ids=["4bit", "8bit", "4bit-gqa8"])
def test_mixed_decode_heavy(cuda, bits, hq):
    """Mostly decode rows beside one short prefill chunk: the single launch gives the decode rows their
    largest workgroup count (ranges split over every decode workgroup)."""
    print(f"[mixed decode-heavy bits={bits} hq={hq}]", flush=True)
    wl = unified_workload("dheavy", seed=70 + bits + hq, num_prefill=1, chunk=40, prior_range=(0, 300),
                          num_decode=60, decode_ctx=(1, 2000), num_q_heads=hq, bits=bits)
    view = gpu_cache(wl, cuda)
    assert_attention_close(_run(wl, view, cuda), oracle_expected(wl), f"decode-heavy {bits}/{hq}")


def test_kv_shorter_than_query_rows(cuda):
    """kv_len < q_len: early query rows see no key (zeros, like the reference's max_k < 0 rows)."""
    print("[prefill short kv]", flush=True)
    wl = unified_workload("short", seed=21, num_prefill=2, chunk=200, prior_range=(0, 100), num_decode=2,
                          decode_ctx=(10, 300), bits=4)
    view = gpu_cache(wl, cuda)
    lens = wl.kv_lens.copy()
    lens[0] = 120  # 200 query rows, 120 keys: rows 0..79 see nothing
    lens[2] = 0    # a decode row with no context
    got = _run(wl, view, cuda, kv_lens=torch.from_numpy(lens).to(cuda))
    exp = oracle_expected(wl, kv_lens=lens)
    assert_attention_close(got, exp, "short kv")
    assert np.all(got[:80] == 0)
    assert np.all(got[int(wl.query_start_loc[2])] == 0)


@pytest.mark.parametrize("bits,window", [(4, 0), (8, 0), (4, 1000)])
def test_prefill_key_split(cuda, bits, window):
    """Tiles of long contexts split over up to three workgroups (merged in-kernel) vs the oracle and vs one
    workgroup per tile (a workspace without room for the split); a repeat reuses the cleared counters."""
    from easymlx_amd import _native

    print(f"[prefill key split bits={bits} window={window}]", flush=True)
    wl = unified_workload("split", seed=50 + bits, num_prefill=3, chunk=160, prior_range=(1500, 3000),
                          num_decode=4, decode_ctx=(100, 3000), bits=bits)
    view = gpu_cache(wl, cuda)
    exp = oracle_expected(wl, sliding_window=window)
    split = _run(wl, view, cuda, sliding_window=window)
    assert_attention_close(split, exp, "split")
    assert np.array_equal(_run(wl, view, cuda, sliding_window=window), split), "repeat differs"
    lib = _native.load()
    S, mb = wl.block_tables.shape
    ws = torch.zeros(lib.emx_paged_workspace_bytes(S, wl.num_q_heads, wl.num_kv_heads, wl.head_dim, mb,
                                                   wl.block_size), dtype=torch.uint8, device=cuda)
    q = torch.from_numpy(wl.q).to(cuda)
    whole = paged_attention(q, view.k_codes, view.v_codes, view.block_tables, view.kv_lens,
                            torch.from_numpy(wl.query_start_loc).to(cuda), k_scales=view.k_scales,
                            k_biases=view.k_biases, v_scales=view.v_scales, v_biases=view.v_biases, bits=wl.bits,
                            group_size=wl.group_size, single_token_decode=False, sliding_window=window,
                            workspace=ws).float().cpu().numpy()
    assert_attention_close(whole, exp, "unsplit")
    assert np.abs(whole - split).max() < 2e-3
