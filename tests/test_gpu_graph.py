"""A decode step captured in a HIP graph (the counterpart of the reference's decode under mx.compile,
model_runner.py:139-189): quantize-on-write of the new tokens, then split-K paged attention.  Every replay,
with new inputs copied into the captured buffers and eager work between replays, matches the eager step."""

import numpy as np
import pytest
import torch

from easymlx_amd import _native, paged_attention
from easymlx_amd.caching.paged import affine_pool
from easymlx_amd.workloads import decode_workload

pytestmark = pytest.mark.gpu


def test_decode_step_graph_replays_match_eager(cuda):
    print("[graph decode step]", flush=True)
    rng = np.random.default_rng(12)
    wl = decode_workload(seed=12, num_seqs=16, ctx_range=(100, 1500), bits=4)
    S, hq, hkv, d, bs = wl.num_seqs, wl.num_q_heads, wl.num_kv_heads, wl.head_dim, wl.block_size
    tables = torch.from_numpy(wl.block_tables).to(cuda)
    lens = torch.from_numpy(wl.kv_lens).to(cuda)

    def pool():
        p = affine_pool(num_blocks=wl.num_blocks, num_kv_heads=hkv, head_dim=d, block_size=bs, bits=4, group_size=64,
                        block_tables=tables, kv_lens=lens)
        p.write_slots(torch.from_numpy(wl.k).to(cuda).half(), torch.from_numpy(wl.v).to(cuda).half(),
                      torch.from_numpy(wl.slot.astype(np.int32)).to(cuda))
        return p

    graph_pool, eager_pool = pool(), pool()
    # the step appends one token per sequence at its last position (kv_lens already count it)
    last = torch.from_numpy(((wl.block_tables[np.arange(S), (wl.kv_lens - 1) // bs]) * bs
                             + (wl.kv_lens - 1) % bs).astype(np.int32)).to(cuda)
    qsl = torch.arange(S + 1, dtype=torch.int32, device=cuda)
    lib = _native.load()
    ws = torch.zeros(lib.emx_paged_workspace_bytes(S, hq, hkv, d, wl.block_tables.shape[1], bs), dtype=torch.uint8,
                     device=cuda)
    q_buf = torch.zeros((S, hq, d), dtype=torch.float16, device=cuda)
    k_buf = torch.zeros((S, hkv, d), dtype=torch.float16, device=cuda)
    v_buf = torch.zeros((S, hkv, d), dtype=torch.float16, device=cuda)
    out_buf = torch.zeros((S, hq, d), dtype=torch.float16, device=cuda)

    def step(p, q, k, v, out):
        p.write_slots(k, v, last)
        paged_attention(q, p.k_codes, p.v_codes, tables, lens, qsl, k_scales=p.k_scales, k_biases=p.k_biases,
                        v_scales=p.v_scales, v_biases=p.v_biases, bits=4, group_size=64, single_token_decode=True,
                        workspace=ws, out=out)

    side = torch.cuda.Stream(cuda)
    side.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(side):  # warm the allocator / library on the capture stream
        step(graph_pool, q_buf, k_buf, v_buf, out_buf)
    torch.cuda.current_stream(cuda).wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step(graph_pool, q_buf, k_buf, v_buf, out_buf)
    for rep in range(4):
        q = torch.from_numpy(rng.standard_normal((S, hq, d)).astype(np.float16)).to(cuda)
        k = torch.from_numpy((rng.standard_normal((S, hkv, d)) * 2).astype(np.float16)).to(cuda)
        v = torch.from_numpy((rng.standard_normal((S, hkv, d)) * 2).astype(np.float16)).to(cuda)
        q_buf.copy_(q)
        k_buf.copy_(k)
        v_buf.copy_(v)
        g.replay()
        torch.cuda.synchronize()
        eager_out = torch.empty_like(out_buf)
        step(eager_pool, q, k, v, eager_out)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out_buf, eager_out), f"replay {rep}"
        for name in ("k_codes", "k_scales", "k_biases", "v_codes", "v_scales", "v_biases"):
            assert torch.equal(getattr(graph_pool, name), getattr(eager_pool, name)), (rep, name)
