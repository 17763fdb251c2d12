"""Ragged / unified attention, dense caches and odd shapes (generic HIP kernel) vs the oracle."""

import os

import numpy as np
import pytest
import torch

from easymlx_amd import paged_attention
from easymlx_amd.workloads import config, decode_workload, unified_workload
from tests.helpers import assert_attention_close, gpu_cache, oracle_expected

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.mark.parametrize("name", ["attn_rng0.npz", "attn_rng1.npz", "attn_rng11.npz"])
def test_reference_seeded_cases_dense_fp32(cuda, name):
    """The reference tests' own seeded inputs, fp32 cache, tolerance 1e-5 as in those tests."""
    print(f"[golden {name}]", flush=True)
    g = np.load(os.path.join(GOLDEN, name))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)  # noqa: E731
    out = paged_attention(
        t(g["queries"]), t(g["key_cache"]), t(g["value_cache"]), t(g["block_tables"]), t(g["kv_lens"]),
        t(g["query_start_loc"]), softmax_scale=float(g["softmax_scale"]), sliding_window=0,
    )
    torch.cuda.synchronize()
    np.testing.assert_allclose(out.cpu().numpy(), g["expected"], atol=1e-5, rtol=1e-5)


def test_c0_plumbing_fp16(cuda):
    print("[c0 fp16 dense]", flush=True)
    wl = config("c0")
    kc, vc = wl.logical_cache()
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)  # noqa: E731
    out = paged_attention(t(wl.q), t(kc), t(vc), t(wl.block_tables), t(wl.kv_lens), t(wl.query_start_loc),
                          single_token_decode=True)
    torch.cuda.synchronize()
    assert_attention_close(out.float().cpu().numpy(), oracle_expected(wl), "c0")


def test_dense_bf16_ragged(cuda):
    print("[bf16 ragged dense]", flush=True)
    wl = unified_workload("u", seed=31, num_prefill=2, chunk=37, prior_range=(0, 50), num_decode=3,
                          decode_ctx=(1, 90), num_q_heads=8, num_kv_heads=2, head_dim=64, block_size=16, bits=None)
    kc, vc = wl.logical_cache()
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)  # noqa: E731
    out = paged_attention(t(wl.q).bfloat16(), t(kc).bfloat16(), t(vc).bfloat16(), t(wl.block_tables),
                          t(wl.kv_lens), t(wl.query_start_loc))
    torch.cuda.synchronize()
    wl.q = wl.q.astype(np.float32)
    exp = oracle_expected(wl)
    np.testing.assert_allclose(out.float().cpu().numpy(), exp, atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("bits", [4, 8])
def test_unified_ragged_affine(cuda, bits):
    """C3 structure (prefill chunks + decode rows) at reduced size, causal inside chunks."""
    print(f"[unified ragged bits={bits}]", flush=True)
    wl = unified_workload("u", seed=40 + bits, num_prefill=2, chunk=96, prior_range=(0, 300), num_decode=5,
                          decode_ctx=(1, 700), bits=bits)
    view = gpu_cache(wl, cuda)
    q = torch.from_numpy(wl.q).to(cuda)
    out = paged_attention(q, view.k_codes, view.v_codes, view.block_tables, view.kv_lens,
                          torch.from_numpy(wl.query_start_loc).to(cuda), k_scales=view.k_scales,
                          k_biases=view.k_biases, v_scales=view.v_scales, v_biases=view.v_biases, bits=bits,
                          group_size=wl.group_size, single_token_decode=False, sliding_window=0)
    torch.cuda.synchronize()
    assert_attention_close(out.float().cpu().numpy(), oracle_expected(wl), f"unified b{bits}")


@pytest.mark.parametrize("shape", [(64, 16, 32), (96, 8, 32), (256, 32, 64)], ids=["d64bs16", "d96bs8", "d256bs32"])
def test_decode_odd_shapes_generic(cuda, shape):
    d, bs, gs = shape
    print(f"[odd shape {shape}]", flush=True)
    wl = decode_workload(seed=d + bs, num_seqs=4, num_q_heads=12, num_kv_heads=4, head_dim=d, block_size=bs,
                         ctx_range=(1, 300), bits=4, group_size=gs)
    view = gpu_cache(wl, cuda)
    q = torch.from_numpy(wl.q).to(cuda)
    out = paged_attention(q, view.k_codes, view.v_codes, view.block_tables, view.kv_lens,
                          torch.from_numpy(wl.query_start_loc).to(cuda), k_scales=view.k_scales,
                          k_biases=view.k_biases, v_scales=view.v_scales, v_biases=view.v_biases, bits=4,
                          group_size=gs, single_token_decode=True)
    torch.cuda.synchronize()
    assert_attention_close(out.float().cpu().numpy(), oracle_expected(wl), str(shape))


SPLIT_CASES = [
    # (kind, D, page, Hq, Hkv, bits, group, ctx, seqs, window)
    ("affine", 256, 128, 32, 8, 4, 64, (512, 4096), 6, 0),   # head-256 decode
    ("affine", 256, 16, 16, 8, 4, 64, (1, 1500), 7, 0),
    ("affine", 256, 64, 16, 4, 8, 128, (100, 2500), 4, 700),
    ("affine", 64, 8, 8, 2, 8, 32, (1, 900), 9, 0),
    ("affine", 96, 32, 24, 8, 4, 32, (60, 1200), 5, 0),      # GQA 3
    ("affine", 128, 128, 64, 2, 4, 64, (300, 2000), 3, 0),   # GQA 32: two head chunks per kv head
    ("affine", 64, 128, 8, 2, 4, 64, (16000, 30000), 3, 0),  # 60-120 chunks per row merged through LDS
    ("affine", 256, 64, 16, 4, 8, 64, (20000, 24000), 2, 5000),  # long rows under a window
    ("dense", 256, 16, 32, 8, None, 64, (1, 2000), 6, 0),
    ("dense", 96, 32, 12, 4, None, 64, (1, 700), 5, 99),
]


@pytest.mark.parametrize("case", SPLIT_CASES, ids=[f"{c[0]}d{c[1]}p{c[2]}hq{c[3]}hkv{c[4]}b{c[5]}g{c[6]}w{c[9]}"
                                                  for c in SPLIT_CASES])
def test_split_decode_shapes(cuda, case):
    """Single-token decode outside the MFMA kernels (head_dim 64..256, pages of 8..128 tokens, any GQA): the
    split-K kernel (chunks of 256 keys + a merge launch) against the oracle, and a repeat bit for bit."""
    kind, d, bs, hq, hkv, bits, gs, ctx, seqs, window = case
    print(f"[split decode {case}]", flush=True)
    wl = decode_workload(seed=900 + d + bs + seqs, num_seqs=seqs, num_q_heads=hq, num_kv_heads=hkv, head_dim=d,
                         block_size=bs, ctx_range=ctx, bits=bits, group_size=gs)
    q = torch.from_numpy(wl.q).to(cuda)
    qsl = torch.from_numpy(wl.query_start_loc).to(cuda)
    kw = {"sliding_window": window} if window else {}
    if kind == "affine":
        view = gpu_cache(wl, cuda)

        def run():
            return paged_attention(q, view.k_codes, view.v_codes, view.block_tables, view.kv_lens, qsl,
                                   k_scales=view.k_scales, k_biases=view.k_biases, v_scales=view.v_scales,
                                   v_biases=view.v_biases, bits=bits, group_size=gs, single_token_decode=True, **kw)
    else:
        kc, vc = wl.logical_cache()
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)  # noqa: E731
        kct, vct, bt, kl = t(kc), t(vc), t(wl.block_tables), t(wl.kv_lens)

        def run():
            return paged_attention(q, kct, vct, bt, kl, qsl, single_token_decode=True, **kw)
    got = run().float().cpu().numpy()
    torch.cuda.synchronize()
    assert_attention_close(got, oracle_expected(wl, sliding_window=window), f"split decode {case}")
    assert np.array_equal(run().float().cpu().numpy(), got), "repeat differs"


def test_split_decode_very_wide_table_takes_generic(cuda):
    """A block table wider than the split-K merge's LDS holds (5000 pages of 128 tokens: more
    than 2,500 chunks per row) sends the decode to the generic kernel; same results."""
    print("[split decode wide table]", flush=True)
    wl = decode_workload(seed=77, num_seqs=3, num_q_heads=8, num_kv_heads=2, head_dim=64, block_size=128,
                         ctx_range=(100, 900), bits=4, group_size=64)
    view = gpu_cache(wl, cuda)
    wide = np.full((wl.block_tables.shape[0], 5000), -1, np.int32)
    wide[:, :wl.block_tables.shape[1]] = wl.block_tables
    q = torch.from_numpy(wl.q).to(cuda)
    qsl = torch.from_numpy(wl.query_start_loc).to(cuda)
    out = paged_attention(q, view.k_codes, view.v_codes, torch.from_numpy(wide).to(cuda), view.kv_lens, qsl,
                          k_scales=view.k_scales, k_biases=view.k_biases, v_scales=view.v_scales,
                          v_biases=view.v_biases, bits=4, group_size=64, single_token_decode=True)
    assert_attention_close(out.float().cpu().numpy(), oracle_expected(wl), "wide table")
