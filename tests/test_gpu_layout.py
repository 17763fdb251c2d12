"""Device layout conversion of affine caches (``emx_affine_pages_from_logical`` / ``emx_affine_logical_from_pages``).

The logical layout is ``mlx.core.quantize`` of the reference's dense cache ``[nb, bs, Hkv, D]``
(``cache.py:790-791``).  Checks: bit-exact against the host restatement in ``caching/layout.py`` on random
words (4/8 bits, page sizes below and above one value tile, groups 32/64/128), exact round trip, and attention
over pages converted from the oracle's logical pages against the oracle."""

import numpy as np
import pytest
import torch

from easymlx_amd import AffinePageCacheView, paged_attention
from easymlx_amd.caching import layout
from easymlx_amd.workloads import decode_workload
from helpers import assert_attention_close, oracle_expected, oracle_logical_pages

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits,bs,gs", [(4, 128, 64), (4, 16, 32), (4, 64, 128), (8, 128, 64), (8, 16, 32),
                                        (8, 32, 128)])
def test_logical_pages_round_trip(cuda, bits, bs, gs):
    print(f"[layout bits={bits} bs={bs} gs={gs}]", flush=True)
    rng = np.random.default_rng(bits * 1000 + bs + gs)
    nb, hkv, d = 7, 3, 128
    w, G = d * bits // 32, d // gs
    kc = rng.integers(0, 2**32, (nb, bs, hkv, w), dtype=np.uint64).astype(np.uint32)
    vc = rng.integers(0, 2**32, (nb, bs, hkv, w), dtype=np.uint64).astype(np.uint32)
    par = [rng.standard_normal((nb, bs, hkv, G)).astype(np.float16) for _ in range(4)]
    t = lambda a: torch.from_numpy(a.view(np.int32) if a.dtype == np.uint32 else a).to(cuda)  # noqa: E731
    tables = torch.arange(nb, dtype=torch.int32, device=cuda).reshape(1, nb)
    lens = torch.tensor([nb * bs], dtype=torch.int32, device=cuda)
    view = AffinePageCacheView.from_logical(k_codes=t(kc), k_scales=t(par[0]), k_biases=t(par[1]), v_codes=t(vc),
                                            v_scales=t(par[2]), v_biases=t(par[3]), block_tables=tables,
                                            kv_lens=lens, bits=bits, group_size=gs)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(view.key_cache.cpu().numpy().view(np.uint32), layout.key_pages_from_logical(kc))
    np.testing.assert_array_equal(view.value_cache.cpu().numpy().view(np.uint32),
                                  layout.value_pages_from_logical(vc, bits))
    for got, want in zip((view.k_scales, view.k_biases, view.v_scales, view.v_biases), par):
        np.testing.assert_array_equal(got.cpu().numpy(), layout.params_pages_from_logical(want))
    back = view.to_logical()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(back["k_codes"].cpu().numpy().view(np.uint32), kc)
    np.testing.assert_array_equal(back["v_codes"].cpu().numpy().view(np.uint32), vc)
    for n, want in zip(("k_scales", "k_biases", "v_scales", "v_biases"), par):
        np.testing.assert_array_equal(back[n].cpu().numpy(), want)


@pytest.mark.parametrize("bits", [4, 8])
def test_attention_over_converted_pages(cuda, bits):
    """The oracle's own quantized logical pages, converted on the device, attended by the library."""
    print(f"[layout attention bits={bits}]", flush=True)
    wl = decode_workload("lay", seed=11 + bits, num_seqs=6, ctx_range=(40, 700), bits=bits)
    lp = oracle_logical_pages(wl)
    t = lambda a: torch.from_numpy(a.view(np.int32) if a.dtype == np.uint32 else a).to(cuda)  # noqa: E731
    view = AffinePageCacheView.from_logical(k_codes=t(lp["k"][0]), k_scales=t(lp["k"][1]), k_biases=t(lp["k"][2]),
                                            v_codes=t(lp["v"][0]), v_scales=t(lp["v"][1]), v_biases=t(lp["v"][2]),
                                            block_tables=torch.from_numpy(wl.block_tables),
                                            kv_lens=torch.from_numpy(wl.kv_lens), bits=bits,
                                            group_size=wl.group_size)
    out = paged_attention(torch.from_numpy(wl.q).to(cuda), view.key_cache, view.value_cache, view.block_tables,
                          view.kv_lens, torch.from_numpy(wl.query_start_loc).to(cuda), k_scales=view.k_scales,
                          k_biases=view.k_biases, v_scales=view.v_scales, v_biases=view.v_biases, bits=bits,
                          group_size=wl.group_size, single_token_decode=True)
    torch.cuda.synchronize()
    assert_attention_close(out.float().cpu().numpy(), oracle_expected(wl), f"converted pages, {bits}-bit")


@pytest.mark.parametrize("bits,decode", [(4, True), (8, True), (4, False)])
def test_op_takes_the_logical_layout(cuda, bits, decode):
    """``paged_attention`` given the reference's logical layout (rank-4 value codes) converts the pages for the
    call: the same bits as on pages converted once, and the oracle's attention."""
    print(f"[op logical layout bits={bits} decode={decode}]", flush=True)
    if decode:
        wl = decode_workload("lay", seed=21 + bits, num_seqs=5, ctx_range=(40, 900), bits=bits)
    else:
        from easymlx_amd.workloads import unified_workload
        wl = unified_workload("lay", seed=23, num_prefill=2, chunk=40, prior_range=(0, 300), num_decode=3,
                              decode_ctx=(50, 600), bits=bits)
    lp = oracle_logical_pages(wl)
    t = lambda a: torch.from_numpy(a.view(np.int32) if a.dtype == np.uint32 else a).to(cuda)  # noqa: E731
    logical = dict(k_codes=t(lp["k"][0]), k_scales=t(lp["k"][1]), k_biases=t(lp["k"][2]), v_codes=t(lp["v"][0]),
                   v_scales=t(lp["v"][1]), v_biases=t(lp["v"][2]))
    view = AffinePageCacheView.from_logical(**logical, block_tables=torch.from_numpy(wl.block_tables),
                                            kv_lens=torch.from_numpy(wl.kv_lens), bits=bits,
                                            group_size=wl.group_size)
    q = torch.from_numpy(wl.q).to(cuda)
    qsl = torch.from_numpy(wl.query_start_loc).to(cuda)
    a = paged_attention(q, view.key_cache, view.value_cache, view.block_tables, view.kv_lens, qsl,
                        k_scales=view.k_scales, k_biases=view.k_biases, v_scales=view.v_scales,
                        v_biases=view.v_biases, bits=bits, group_size=wl.group_size)
    b = paged_attention(q, logical["k_codes"], logical["v_codes"], view.block_tables, view.kv_lens, qsl,
                        k_scales=logical["k_scales"], k_biases=logical["k_biases"], v_scales=logical["v_scales"],
                        v_biases=logical["v_biases"], bits=bits, group_size=wl.group_size)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert_attention_close(b.float().cpu().numpy(), oracle_expected(wl), f"logical layout, {bits}-bit")
