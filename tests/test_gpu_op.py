"""End to end through the plugin boundary: concatenate_to_cache (quantize-on-write) then
UnifiedAttention.forward_native, prefill step followed by decode steps, vs the oracle."""

import numpy as np
import pytest
import torch

from easymlx_amd import AffinePageCacheView, OperationRegistry, PageMetadata, build_query_start_loc
from oracle.affine import affine_dequantize, affine_quantize
from oracle.paged_attention import paged_attention as oracle_attention
from tests.helpers import assert_attention_close

pytestmark = pytest.mark.gpu


def _oracle_step(tokens_k, tokens_v, queries, qlens, bits, gs, hkv, d):
    """Oracle over per-sequence token lists using a trivial contiguous page table."""
    bs = 16
    lens = [len(k) for k in tokens_k]
    max_blocks = max(-(-n // bs) for n in lens)
    nb = max_blocks * len(lens)
    kc = np.zeros((nb, bs, hkv, d), np.float32)
    vc = np.zeros_like(kc)
    tables = np.arange(nb, dtype=np.int32).reshape(len(lens), max_blocks)
    for s, (ks, vs) in enumerate(zip(tokens_k, tokens_v)):
        pos = np.arange(len(ks))
        kq = affine_dequantize(*affine_quantize(np.stack(ks), gs, bits), gs, bits, round_to_fp16=False)
        vq = affine_dequantize(*affine_quantize(np.stack(vs), gs, bits), gs, bits, round_to_fp16=False)
        kc[tables[s, pos // bs], pos % bs] = kq
        vc[tables[s, pos // bs], pos % bs] = vq
    qsl = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    return oracle_attention(queries, kc, vc, tables, np.array(lens, np.int32), qsl, compute_dtype=np.float64,
                            out_dtype=np.float64)


@pytest.mark.parametrize("bits", [4, 8])
def test_prefill_then_decode_through_operation(cuda, bits):
    print(f"[op prefill+decode bits={bits}]", flush=True)
    rng = np.random.default_rng(77 + bits)
    S, hq, hkv, d, gs = 3, 32, 8, 128, 64
    view = AffinePageCacheView.init(num_seqs=S, max_seq_len=1200, num_kv_heads=hkv, head_dim=d, block_size=128,
                                    bits=bits, group_size=gs, device=cuda)
    op = OperationRegistry.create("unified_attention")
    tk = [[] for _ in range(S)]
    tv = [[] for _ in range(S)]
    steps = [[300, 129, 1], [1, 1, 1], [1, 1, 1], [40, 1, 200]]
    for qlens in steps:
        T = sum(qlens)
        q = rng.standard_normal((T, hq, d)).astype(np.float16)
        k = (rng.standard_normal((T, hkv, d)) * 2).astype(np.float16)
        v = (rng.standard_normal((T, hkv, d)) * 2).astype(np.float16)
        md = PageMetadata(query_start_loc=build_query_start_loc(qlens, device=cuda), slot_ids=tuple(range(S)))
        qq, kcache, vcache, md = view.concatenate_to_cache(
            torch.from_numpy(q).to(cuda), torch.from_numpy(k).to(cuda), torch.from_numpy(v).to(cuda),
            cache_metadata=md)
        at = 0
        for s, n in enumerate(qlens):
            tk[s].extend(list(k[at:at + n]))
            tv[s].extend(list(v[at:at + n]))
            at += n
        res = op(query=qq, key=kcache, value=vcache, cache_metadata=md, cache_view=view, scale=d ** -0.5)
        torch.cuda.synchronize()
        exp = _oracle_step(tk, tv, q, qlens, bits, gs, hkv, d)
        assert_attention_close(res.attention_outputs.float().cpu().numpy(), exp, f"step {qlens}")
        assert view.kv_lens.cpu().tolist() == [len(x) for x in tk]
