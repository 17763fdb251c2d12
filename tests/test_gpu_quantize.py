"""GPU quantize / quantize-on-write vs the oracle: codes, scales, biases bit-exact."""

import numpy as np
import pytest
import torch

from easymlx_amd import affine_quantize as gpu_quantize
from easymlx_amd.workloads import decode_workload
from oracle.affine import affine_quantize
from tests.helpers import gpu_cache, gpu_pages_to_logical, oracle_logical_pages

pytestmark = pytest.mark.gpu


def _edge_rows(rng, d):
    rows = [
        np.zeros(d),
        np.full(d, 3.0),
        np.full(d, -0.125),
        rng.integers(-8, 8, d).astype(np.float64),          # integer grid: many exact ties
        rng.integers(0, 16, d).astype(np.float64) * 0.5,     # one-sided positive
        -rng.integers(0, 16, d).astype(np.float64) * 0.25,   # one-sided negative
        rng.standard_normal(d) * 1e-4,                       # tiny range -> eps path
        np.clip(rng.standard_normal(d), -3, 3) * 2e4,        # near fp16 max
        np.linspace(-1, 1, d),
    ]
    return np.stack(rows).astype(np.float16)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_quantize_rows_bit_exact(cuda, bits, gs):
    print(f"[quantize rows bits={bits} gs={gs}]", flush=True)
    rng = np.random.default_rng(100 + bits * 7 + gs)
    d = 128
    x = (rng.standard_normal((2000, d)) * rng.uniform(0.01, 40.0, (2000, 1))).astype(np.float16)
    x = np.concatenate([x, _edge_rows(rng, d)])
    c, s, b = gpu_quantize(torch.from_numpy(x).to(cuda), group_size=gs, bits=bits)
    ec, es, eb = affine_quantize(x, gs, bits)
    np.testing.assert_array_equal(c.cpu().numpy().view(np.uint32), ec)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint16), es.view(np.uint16))
    np.testing.assert_array_equal(b.cpu().numpy().view(np.uint16), eb.view(np.uint16))


@pytest.mark.parametrize("bits", [4, 8])
def test_cache_write_bit_exact(cuda, bits):
    print(f"[cache write bits={bits}]", flush=True)
    wl = decode_workload(seed=21 + bits, num_seqs=6, ctx_range=(1, 700), bits=bits)
    view = gpu_cache(wl, cuda)
    torch.cuda.synchronize()
    got = gpu_pages_to_logical(view)
    exp = oracle_logical_pages(wl)
    live = np.zeros((wl.num_blocks, wl.block_size), bool)
    live[wl.slot // wl.block_size, wl.slot % wl.block_size] = True
    for name in ("k", "v"):
        for g, e in zip(got[name], exp[name]):
            g = g[live]
            e = e[live]
            if g.dtype == np.float16:
                g, e = g.view(np.uint16), e.view(np.uint16)
            np.testing.assert_array_equal(g, e, err_msg=f"{name} page contents differ")


def test_cache_write_overwrite_and_skip(cuda):
    """Rewriting a slot replaces its nibbles; slot -1 writes nothing; neighbours keep theirs."""
    print("[cache write overwrite/skip]", flush=True)
    wl = decode_workload(seed=5, num_seqs=2, ctx_range=(40, 40), bits=4)
    view = gpu_cache(wl, cuda)
    before = gpu_pages_to_logical(view)
    rng = np.random.default_rng(9)
    k2 = rng.standard_normal((3, wl.num_kv_heads, wl.head_dim)).astype(np.float16)
    v2 = rng.standard_normal((3, wl.num_kv_heads, wl.head_dim)).astype(np.float16)
    slots = np.array([wl.slot[5], -1, wl.slot[17]], np.int32)
    view.write_slots(torch.from_numpy(k2).to(cuda), torch.from_numpy(v2).to(cuda), torch.from_numpy(slots).to(cuda))
    after = gpu_pages_to_logical(view)
    for name, src in (("k", k2), ("v", v2)):
        ec, es, eb = affine_quantize(src, wl.group_size, wl.bits)
        for i, sl in ((0, wl.slot[5]), (2, wl.slot[17])):
            b, o = sl // wl.block_size, sl % wl.block_size
            np.testing.assert_array_equal(after[name][0][b, o], ec[i])
            np.testing.assert_array_equal(after[name][1][b, o].view(np.uint16), es[i].view(np.uint16))
            np.testing.assert_array_equal(after[name][2][b, o].view(np.uint16), eb[i].view(np.uint16))
        keep = np.ones((wl.num_blocks, wl.block_size), bool)
        for sl in (wl.slot[5], wl.slot[17]):
            keep[sl // wl.block_size, sl % wl.block_size] = False
        np.testing.assert_array_equal(after[name][0][keep], before[name][0][keep])


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("chunks", [(100, 29), (20,), ()], ids=["large-write", "small-shared", "appends-only"])
def test_cache_write_appends_and_unaligned_chunks(cuda, bits, chunks):
    """Decode appends (one token per sequence into a partly filled page) and prefill chunks that
    start mid-word: whole-word stores and per-token nibble updates must give the same bit-exact
    pages as the oracle, and leave every other slot untouched."""
    print(f"[cache write appends/chunks bits={bits} chunks={chunks}]", flush=True)
    wl = decode_workload(seed=31 + bits, num_seqs=5, ctx_range=(300, 600), bits=bits, pool_pages=32)
    view = gpu_cache(wl, cuda)
    before = gpu_pages_to_logical(view)
    rng = np.random.default_rng(77 + bits)
    bs = wl.block_size
    # slots: one append per sequence (the next free position), then a 100-token chunk starting at offset 5
    # of a fresh page, then a 29-token chunk at offset 37 of another page
    appends = [int(wl.block_tables[s, wl.kv_lens[s] // bs]) * bs + int(wl.kv_lens[s]) % bs
               for s in range(5) if wl.kv_lens[s] % bs]  # sequences whose last page has room
    free = sorted(set(range(wl.num_blocks)) - set(int(x) for x in (wl.slot // bs)))
    assert len(free) >= 2, "workload pool has no spare page"
    starts = (5, 37)
    chunk_slots = [free[c] * bs + starts[c] + i for c, n in enumerate(chunks) for i in range(n)]
    slots = np.array(appends + chunk_slots, np.int32)
    n = len(slots)
    k2 = (rng.standard_normal((n, wl.num_kv_heads, wl.head_dim)) * 3).astype(np.float16)
    v2 = (rng.standard_normal((n, wl.num_kv_heads, wl.head_dim)) * 3).astype(np.float16)
    view.write_slots(torch.from_numpy(k2).to(cuda), torch.from_numpy(v2).to(cuda), torch.from_numpy(slots).to(cuda))
    after = gpu_pages_to_logical(view)
    written = np.zeros((wl.num_blocks, bs), bool)
    written[slots // bs, slots % bs] = True
    for name, src in (("k", k2), ("v", v2)):
        ec, es, eb = affine_quantize(src, wl.group_size, bits)
        b, o = slots // bs, slots % bs
        np.testing.assert_array_equal(after[name][0][b, o], ec, err_msg=f"{name} codes")
        np.testing.assert_array_equal(after[name][1][b, o].view(np.uint16), es.view(np.uint16))
        np.testing.assert_array_equal(after[name][2][b, o].view(np.uint16), eb.view(np.uint16))
        for i in range(3):
            np.testing.assert_array_equal(after[name][i][~written], before[name][i][~written],
                                          err_msg=f"{name} array {i}: unwritten slots changed")
