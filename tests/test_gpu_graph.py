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


def _extended(wl, extra_pages=1):
    """The workload's tables with ``extra_pages`` fresh pages per sequence (room for appended tokens)."""
    S = wl.num_seqs
    ext = np.full((S, wl.block_tables.shape[1] + extra_pages), -1, np.int32)
    for s in range(S):
        used = -(-int(wl.kv_lens[s]) // wl.block_size)
        ext[s, :used] = wl.block_tables[s, :used]
        ext[s, used:used + extra_pages] = wl.num_blocks + s * extra_pages + np.arange(extra_pages)
    return ext, wl.num_blocks + S * extra_pages


def test_compiled_proxy_decode_graph_matches_oracle(cuda):
    """``CompiledPagedCacheProxy.concatenate_to_cache`` + ``UnifiedAttention.forward_native`` captured in one
    graph (the reference's compiled decode, model_runner.py:139-189): every replay appends one token per
    sequence on the device (kv_lens advance inside the graph) and its attention output matches the float64
    oracle over all tokens written so far."""
    from dataclasses import replace

    from easymlx_amd import CompiledPagedCacheProxy, PageMetadata, UnifiedAttention
    from tests.helpers import assert_attention_close, c_oracle_expected

    print("[graph compiled proxy vs oracle]", flush=True)
    rng = np.random.default_rng(21)
    wl = decode_workload(seed=21, num_seqs=12, ctx_range=(60, 1400), bits=4)
    S, hq, hkv, d, bs = wl.num_seqs, wl.num_q_heads, wl.num_kv_heads, wl.head_dim, wl.block_size
    tables_np, nb = _extended(wl)
    view = affine_pool(num_blocks=nb, num_kv_heads=hkv, head_dim=d, block_size=bs, bits=4, group_size=64,
                       block_tables=torch.from_numpy(tables_np).to(cuda),
                       kv_lens=torch.from_numpy(wl.kv_lens).to(cuda))
    view.write_slots(torch.from_numpy(wl.k).to(cuda), torch.from_numpy(wl.v).to(cuda),
                     torch.from_numpy(wl.slot.astype(np.int32)).to(cuda))
    proxy = CompiledPagedCacheProxy(view)
    op = UnifiedAttention()
    md0 = PageMetadata(query_start_loc=torch.arange(S + 1, dtype=torch.int32, device=cuda),
                       slot_ids=tuple(range(S)))
    q_buf = torch.zeros((S, hq, d), dtype=torch.float16, device=cuda)
    k_buf = torch.zeros((S, hkv, d), dtype=torch.float16, device=cuda)
    v_buf = torch.zeros((S, hkv, d), dtype=torch.float16, device=cuda)
    out_buf = torch.zeros((S, hq, d), dtype=torch.float16, device=cuda)

    def step():
        q2, kc, vc, md = proxy.concatenate_to_cache(q_buf, k_buf, v_buf, cache_metadata=md0)
        out = op.forward_native(query=q2, key=kc, value=vc, cache_metadata=md, cache_view=view).attention_outputs
        out_buf.copy_(out)

    # host record of every token written: (slot, k, v) per sequence, for the oracle
    toks_k = [wl.k[wl.query_start_loc[0]:0]]  # placeholder, replaced below
    offs = np.concatenate([[0], np.cumsum(wl.kv_lens)])
    seq_k = [wl.k[offs[s]:offs[s + 1]] for s in range(S)]
    seq_v = [wl.v[offs[s]:offs[s + 1]] for s in range(S)]
    lens = wl.kv_lens.astype(np.int64).copy()

    def feed():
        q = rng.standard_normal((S, hq, d)).astype(np.float16)
        k = (rng.standard_normal((S, hkv, d)) * 2).astype(np.float16)
        v = (rng.standard_normal((S, hkv, d)) * 2).astype(np.float16)
        q_buf.copy_(torch.from_numpy(q))
        k_buf.copy_(torch.from_numpy(k))
        v_buf.copy_(torch.from_numpy(v))
        for s in range(S):
            seq_k[s] = np.concatenate([seq_k[s], k[s:s + 1]])
            seq_v[s] = np.concatenate([seq_v[s], v[s:s + 1]])
        lens[:] += 1
        return q

    def expected(q):
        slot = np.concatenate([tables_np[s, np.arange(lens[s]) // bs].astype(np.int64) * bs + np.arange(lens[s]) % bs
                               for s in range(S)])
        w = replace(wl, q=q, k=np.concatenate(seq_k), v=np.concatenate(seq_v), slot=slot,
                    kv_lens=lens.astype(np.int32), block_tables=tables_np, num_blocks=nb)
        return c_oracle_expected(w)

    side = torch.cuda.Stream(cuda)
    side.wait_stream(torch.cuda.current_stream(cuda))
    q = feed()
    with torch.cuda.stream(side):  # the eager step: buffers, workspace and library made on the capture stream
        step()
    side.synchronize()
    assert_attention_close(out_buf.float().cpu().numpy(), expected(q), "eager step")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        step()
    for rep in range(4):
        q = feed()
        g.replay()
        torch.cuda.synchronize()
        # eager work between replays (a throwaway op on the default stream)
        torch.cuda.synchronize()
        assert np.array_equal(view.kv_lens.cpu().numpy(), lens), f"kv_lens after replay {rep}"
        assert_attention_close(out_buf.float().cpu().numpy(), expected(q), f"replay {rep}")
        (torch.ones(1024, device=cuda) * 2).sum().item()
    del toks_k


@pytest.mark.parametrize("kind", ["affine", "fp8", "dense"])
def test_compiled_proxy_rope_graph_matches_eager_views(cuda, kind):
    """The proxy with a fused RotaryEmbedding, captured, against the eager ``concatenate_to_cache`` of a second
    view of the same kind: rotated queries and every cache byte identical after each replay."""
    from easymlx_amd import CompiledPagedCacheProxy, Fp8PageCacheView, PageCacheView, PageMetadata, RotaryEmbedding

    print(f"[graph proxy rope {kind}]", flush=True)
    rng = np.random.default_rng(5)
    S, hq, hkv, d, bs = 6, 16, 4, 128, 32
    rope = RotaryEmbedding.llama3(d, base=500000.0)

    def make():
        if kind == "affine":
            v = affine_pool(num_blocks=S * 4, num_kv_heads=hkv, head_dim=d, block_size=bs, bits=4, group_size=64,
                            block_tables=torch.arange(S * 4, dtype=torch.int32, device=cuda).reshape(S, 4),
                            kv_lens=torch.from_numpy(rng.integers(0, 90, S).astype(np.int32)).to(cuda))
        elif kind == "fp8":
            v = Fp8PageCacheView.init(num_seqs=S, max_seq_len=4 * bs, num_kv_heads=hkv, head_dim=d, block_size=bs,
                                      device=cuda)
        else:
            v = PageCacheView.init(num_seqs=S, max_seq_len=4 * bs, num_kv_heads=hkv, head_dim=d, block_size=bs,
                                   device=cuda)
        return v

    a, b = make(), make()
    b.kv_lens.copy_(a.kv_lens)
    proxy = CompiledPagedCacheProxy(a)
    md0 = PageMetadata(query_start_loc=torch.arange(S + 1, dtype=torch.int32, device=cuda), slot_ids=tuple(range(S)))
    bufs = [torch.zeros((S, h, d), dtype=torch.float16, device=cuda) for h in (hq, hkv, hkv)]
    qo = torch.zeros((S, hq, d), dtype=torch.float16, device=cuda)

    def step():
        q2, _, _, _ = proxy.concatenate_to_cache(*bufs, cache_metadata=md0, rope=rope)
        qo.copy_(q2)

    side = torch.cuda.Stream(cuda)
    side.wait_stream(torch.cuda.current_stream(cuda))
    names = ("key_cache", "value_cache") + (("k_scales", "k_biases", "v_scales", "v_biases") if kind == "affine"
                                            else ("k_scales", "v_scales") if kind == "fp8" else ())
    for rep in range(4):
        xs = [torch.from_numpy(rng.standard_normal(tuple(t.shape)).astype(np.float16)).to(cuda) for t in bufs]
        for t, x in zip(bufs, xs):
            t.copy_(x)
        if rep == 0:
            with torch.cuda.stream(side):
                step()
            side.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                step()
        else:
            g.replay()
        torch.cuda.synchronize()
        q_ref, _, _, _ = b.concatenate_to_cache(*xs, cache_metadata=md0, rope=rope)
        torch.cuda.synchronize()
        assert torch.equal(qo, q_ref), f"{kind} replay {rep}: rotated queries"
        assert torch.equal(a.kv_lens, b.kv_lens), f"{kind} replay {rep}: kv_lens"
        for n in names:
            assert torch.equal(getattr(a, n), getattr(b, n)), f"{kind} replay {rep}: {n}"
