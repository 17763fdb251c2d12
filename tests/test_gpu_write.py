"""Cache writes through the views on the GPU: the device slot arithmetic (emx_cache_slots) and the
unquantized scatter kernel, against the reference tests' write goldens and the oracle's write positions."""

import os

import numpy as np
import pytest
import torch

from easymlx_amd import PageCacheView, PageMetadata
from oracle.cache_write import build_query_start_loc as oracle_qsl
from oracle.cache_write import write_positions

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("name,qlens", [("write_rng2", [2, 0, 3]), ("write_rng7", [1, 1, 1])])
def test_view_write_goldens(cuda, name, qlens):
    """``tests/operations/test_unified_attention.py:268-415`` replayed through ``concatenate_to_cache``:
    kv_lens += q_len and token j of a slot lands at ``[table[pos // bs], pos % bs]``."""
    print(f"[view write {name}]", flush=True)
    z = np.load(os.path.join(GOLDEN, name + ".npz"))
    bs = z["key_cache"].shape[1]
    exp = z["slot_mapping"].tolist()
    view = PageCacheView(key_cache=torch.from_numpy(z["key_cache"].copy()).to(cuda),
                         value_cache=torch.from_numpy(z["value_cache"].copy()).to(cuda),
                         block_tables=torch.from_numpy(z["block_tables"].copy()).to(cuda),
                         kv_lens=torch.from_numpy(z["kv_lens"].copy()).to(cuda), block_size=bs,
                         num_kv_heads=z["key_cache"].shape[2], head_dim=z["key_cache"].shape[3])
    md = PageMetadata(query_start_loc=torch.from_numpy(z["query_start_loc"]).to(cuda))
    q, kc, vc, md2 = view.concatenate_to_cache(torch.from_numpy(z["queries"]).to(cuda),
                                               torch.from_numpy(z["keys"]).to(cuda),
                                               torch.from_numpy(z["values"]).to(cuda), cache_metadata=md,
                                               slot_ids=[0, 1, 2])
    torch.cuda.synchronize()
    assert view.kv_lens.tolist() == z["expected_kv_lens"].tolist()
    assert md2.kv_lens.tolist() == z["expected_kv_lens"].tolist()
    assert md2.is_single_token_decode == (name == "write_rng7")
    assert torch.equal(q.cpu(), torch.from_numpy(z["queries"]))
    flat_k = kc.reshape(-1, *kc.shape[2:]).cpu().numpy()
    flat_v = vc.reshape(-1, *vc.shape[2:]).cpu().numpy()
    np.testing.assert_array_equal(flat_k[exp], z["keys"])
    np.testing.assert_array_equal(flat_v[exp], z["values"])
    untouched = np.ones(flat_k.shape[0], bool)
    untouched[exp] = False
    np.testing.assert_array_equal(flat_k[untouched], z["key_cache"].reshape(flat_k.shape)[untouched])


def test_device_slot_arithmetic_matches_oracle(cuda):
    """emx_cache_slots through the view on a ragged write with skipped slots, empty sequences, negative block ids
    and positions past the table, against oracle.cache_write.write_positions; fp32 dense scatter."""
    print("[device slot arithmetic]", flush=True)
    rng = np.random.default_rng(4)
    S, width, bs, hkv, d = 9, 6, 8, 2, 16
    nb = S * width
    tables = rng.permutation(nb).astype(np.int32).reshape(S, width)
    tables[2, 3] = -1
    lens = rng.integers(0, 30, S).astype(np.int32)
    lens[5] = width * bs - 2  # two tokens fit, the third runs past the table
    slot_ids = [5, 0, 2, 7, 3, 1]
    qlens = [4, 0, 9, 1, 3, 17]
    T = sum(qlens)
    view = PageCacheView(key_cache=torch.zeros((nb, bs, hkv, d), device=cuda),
                         value_cache=torch.zeros((nb, bs, hkv, d), device=cuda),
                         block_tables=torch.from_numpy(tables).to(cuda), kv_lens=torch.from_numpy(lens).to(cuda),
                         block_size=bs, num_kv_heads=hkv, head_dim=d)
    keys = rng.standard_normal((T, hkv, d)).astype(np.float32)
    vals = rng.standard_normal((T, hkv, d)).astype(np.float32)
    md = PageMetadata(query_start_loc=oracle_qsl(qlens))
    view.concatenate_to_cache(torch.zeros((T, 4, d), device=cuda), torch.from_numpy(keys).to(cuda),
                              torch.from_numpy(vals).to(cuda), cache_metadata=md, slot_ids=slot_ids, query_lens=qlens)
    torch.cuda.synchronize()
    # the oracle over the same write (its tables indexed by slot id)
    exp_map, exp_lens = write_positions(tables, lens, oracle_qsl(qlens), slot_ids, bs)
    assert view.kv_lens.cpu().numpy().tolist() == exp_lens.tolist()
    kc = view.key_cache.reshape(-1, hkv, d).cpu().numpy()
    vc = view.value_cache.reshape(-1, hkv, d).cpu().numpy()
    live = np.asarray(exp_map) >= 0
    np.testing.assert_array_equal(kc[np.asarray(exp_map)[live]], keys[live])
    np.testing.assert_array_equal(vc[np.asarray(exp_map)[live]], vals[live])
    assert (~live).sum() >= 2  # the negative block and the run past the table were skipped
    untouched = np.ones(kc.shape[0], bool)
    untouched[np.asarray(exp_map)[live]] = False
    assert not kc[untouched].any() and not vc[untouched].any()
