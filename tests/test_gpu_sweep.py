"""Seeded sweep of random shapes through the public op vs the oracle: affine 4/8-bit (group 32/64/128) and
FP8 caches, GQA 1..16, page sizes 32..256, head_dim 64/128, ragged mixes of prefill chunks and decode rows,
sliding windows.  Each case is small; together they cross the kernel choices (4x4x4 / 16x16 / FP8 decode,
MFMA prefill with and without the key split, generic kernel)."""

import numpy as np
import pytest
import torch

from easymlx_amd import Fp8PageCacheView, paged_attention
from easymlx_amd.workloads import unified_workload
from oracle import fp8
from oracle.paged_attention import paged_attention as oracle_attention
from tests.helpers import assert_attention_close, gpu_cache, oracle_expected

pytestmark = pytest.mark.gpu


def _case(seed):
    rng = np.random.default_rng(1000 + seed)
    kind = ["q4", "q8", "fp8"][seed % 3]
    hkv = int(rng.choice([1, 2, 4, 8]))
    hg = int(rng.choice([1, 2, 4, 8, 16]))
    d = 128 if rng.random() < 0.8 else 64
    gs = int(rng.choice([32, 64, 128])) if d == 128 else 32
    if kind == "q4":
        bs = int(rng.choice([64, 128, 256]))
    else:
        bs = int(rng.choice([32, 64, 128, 256]))
    npf = int(rng.integers(0, 4))
    ndec = int(rng.integers(0 if npf else 1, 7))
    big = rng.random() < 0.3  # long priors: the prefill key split
    return dict(kind=kind, hkv=hkv, hq=hkv * hg, d=d, gs=gs, bs=bs, num_prefill=npf,
                chunk=int(rng.integers(2, 200)), prior=(0, 2500 if big else 400), num_decode=ndec,
                decode_ctx=(1, int(rng.integers(50, 3000))), window=int(rng.choice([0, 0, 0, 37, 700])))


@pytest.mark.parametrize("seed", range(36))
def test_random_shape_vs_oracle(cuda, seed):
    c = _case(seed)
    print(f"[sweep {seed}] {c}", flush=True)
    bits = {"q4": 4, "q8": 8, "fp8": None}[c["kind"]]
    wl = unified_workload("sweep", seed=2000 + seed, num_prefill=c["num_prefill"], chunk=c["chunk"],
                          prior_range=c["prior"], num_decode=c["num_decode"], decode_ctx=c["decode_ctx"],
                          num_q_heads=c["hq"], num_kv_heads=c["hkv"], head_dim=c["d"], block_size=c["bs"],
                          bits=bits, group_size=c["gs"])
    q = torch.from_numpy(wl.q).to(cuda)
    qsl = torch.from_numpy(wl.query_start_loc).to(cuda)
    w = c["window"] or None
    if bits is not None:
        view = gpu_cache(wl, cuda)
        out = paged_attention(q, view.k_codes, view.v_codes, view.block_tables, view.kv_lens, qsl,
                              k_scales=view.k_scales, k_biases=view.k_biases, v_scales=view.v_scales,
                              v_biases=view.v_biases, bits=bits, group_size=c["gs"], sliding_window=w)
        exp = oracle_expected(wl, sliding_window=c["window"])
    else:
        nb = wl.num_blocks
        shape = (nb, wl.block_size, wl.num_kv_heads, wl.head_dim)
        view = Fp8PageCacheView(key_cache=torch.zeros(shape, dtype=torch.uint8, device=cuda),
                                value_cache=torch.zeros(shape, dtype=torch.uint8, device=cuda),
                                k_scales=torch.zeros(nb, device=cuda), v_scales=torch.zeros(nb, device=cuda),
                                block_tables=torch.from_numpy(wl.block_tables).to(cuda),
                                kv_lens=torch.from_numpy(wl.kv_lens).to(cuda), block_size=wl.block_size,
                                num_kv_heads=wl.num_kv_heads, head_dim=wl.head_dim)
        kc, vc = np.zeros(shape, np.uint8), np.zeros(shape, np.uint8)
        ks, vs = np.zeros(nb, np.float32), np.zeros(nb, np.float32)
        k16, v16 = wl.k.astype(np.float16), wl.v.astype(np.float16)
        slot = wl.slot.astype(np.int32)
        view.write_slots(torch.from_numpy(k16).to(cuda), torch.from_numpy(v16).to(cuda),
                         torch.from_numpy(slot).to(cuda))
        fp8.fp8_write(k16.astype(np.float32), v16.astype(np.float32), slot, kc, vc, ks, vs)
        out = paged_attention(q, view.key_cache, view.value_cache, view.block_tables, view.kv_lens, qsl,
                              k_scale=view.k_scales, v_scale=view.v_scales, sliding_window=w)
        exp = oracle_attention(wl.q.astype(np.float32), fp8.fp8_dequant_cache(kc, ks), fp8.fp8_dequant_cache(vc, vs),
                               wl.block_tables, wl.kv_lens, wl.query_start_loc, sliding_window=c["window"],
                               compute_dtype=np.float64)
    torch.cuda.synchronize()
    assert_attention_close(out.float().cpu().numpy(), exp, f"sweep {seed}")
