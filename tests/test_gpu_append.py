"""One-launch decode append (``emx_affine_cache_append_rope``) against the two-launch path it folds together
(``emx_cache_slots`` then ``emx_affine_cache_write_rope``, both checked against the oracle elsewhere): every page
array, ``kv_lens`` and the turned queries bit for bit, on batches with slots in and out of order, invalid slot
ids, a full table, a negative page id, two sequences sharing a page (value words written by two tokens of the
call) and two calls in a row (the workgroup counter returns to zero)."""

import numpy as np
import pytest
import torch

from easymlx_amd import RotaryEmbedding, _native
from easymlx_amd.caching import affine_pool

pytestmark = pytest.mark.gpu


def _view(rng, cuda, nb, bs, hkv, d, bits, gs, tables, lens):
    v = affine_pool(num_blocks=nb, num_kv_heads=hkv, head_dim=d, block_size=bs, bits=bits, group_size=gs,
                    block_tables=torch.from_numpy(tables).to(cuda), kv_lens=torch.from_numpy(lens).to(cuda))
    for t in v.page_arrays():  # arbitrary prior contents: the write must leave the rest of every word alone
        if t.dtype == torch.float16:
            t.copy_(torch.from_numpy(rng.standard_normal(tuple(t.shape)).astype(np.float16)))
        else:
            t.copy_(torch.from_numpy(rng.integers(-2**31, 2**31, tuple(t.shape), dtype=np.int64).astype(np.int32)))
    return v


def _clone(v, cuda):
    w = affine_pool(num_blocks=v.num_blocks, num_kv_heads=v.num_kv_heads, head_dim=v.head_dim,
                    block_size=v.block_size, bits=v.bits, group_size=v.group_size,
                    block_tables=v.block_tables.clone(), kv_lens=v.kv_lens.clone())
    for a, b in zip(w.page_arrays(), v.page_arrays()):
        a.copy_(b)
    return w


def _two_launches(v, slots, k, val, q, rope, cuda):
    lib = _native.load()
    n = len(slots)
    meta = torch.tensor(list(slots) + list(range(n + 1)), dtype=torch.int32, device=cuda)
    mapping = torch.empty(n, dtype=torch.int32, device=cuda)
    pos = torch.empty(n, dtype=torch.int32, device=cuda)
    st = torch.cuda.current_stream(cuda).cuda_stream
    bt = v.block_tables
    _native.check(lib.emx_cache_slots(meta[:n].data_ptr(), meta[n:].data_ptr(), n, n, bt.data_ptr(), bt.shape[0],
                                      bt.shape[1], v.block_size, v.kv_lens.data_ptr(), mapping.data_ptr(),
                                      pos.data_ptr(), st))
    q_out = torch.empty_like(q)
    inv = rope.inv_freq(cuda)
    _native.check(lib.emx_affine_cache_write_rope(
        k.data_ptr(), val.data_ptr(), mapping.data_ptr(), n, v.num_kv_heads, v.head_dim, v.group_size, v.bits,
        v.block_size, v.num_blocks, v.key_cache.data_ptr(), v.k_scales.data_ptr(), v.k_biases.data_ptr(),
        v.value_cache.data_ptr(), v.v_scales.data_ptr(), v.v_biases.data_ptr(), pos.data_ptr(), inv.data_ptr(),
        rope.dims, int(rope.traditional), q.data_ptr(), q_out.data_ptr(), q.shape[1], st))
    return q_out


def _one_launch(v, slots, k, val, q, rope, cuda, counter):
    lib = _native.load()
    s = torch.tensor(slots, dtype=torch.int32, device=cuda)
    q_out = torch.empty_like(q)
    bt = v.block_tables
    _native.check(lib.emx_affine_cache_append_rope(
        k.data_ptr(), val.data_ptr(), s.data_ptr(), len(slots), bt.data_ptr(), bt.shape[0], bt.shape[1],
        v.kv_lens.data_ptr(), counter.data_ptr(), v.num_kv_heads, v.head_dim, v.group_size, v.bits, v.block_size,
        v.num_blocks, v.key_cache.data_ptr(), v.k_scales.data_ptr(), v.k_biases.data_ptr(), v.value_cache.data_ptr(),
        v.v_scales.data_ptr(), v.v_biases.data_ptr(), rope.inv_freq(cuda).data_ptr(), rope.dims,
        int(rope.traditional), q.data_ptr(), q_out.data_ptr(), q.shape[1], torch.cuda.current_stream(cuda).cuda_stream))
    return q_out


@pytest.mark.parametrize("bits,bs,gs,trad", [(4, 128, 64, False), (8, 128, 64, False), (4, 16, 32, True),
                                             (8, 32, 32, False)])
def test_append_matches_the_two_launch_write(cuda, bits, bs, gs, trad):
    print(f"[append bits={bits} bs={bs} gs={gs} traditional={trad}]", flush=True)
    rng = np.random.default_rng(bits * 100 + bs + gs)
    S, hkv, hq, d, mb = 12, 4, 16, 128, 5
    nb = S * mb + 3
    tables = rng.permutation(nb)[:S * mb].astype(np.int32).reshape(S, mb)
    lens = rng.integers(0, mb * bs, S).astype(np.int32)
    lens[0] = bs - 1          # the last slot of a page
    lens[1] = bs              # the first slot of a new page
    lens[2] = mb * bs         # the table is full: not written, kv_lens still advances
    tables[3, lens[3] // bs] = -1  # a negative page id where the token goes
    tables[5] = tables[4]     # two sequences share their pages ...
    lens[5] = lens[4] + 1     # ... and the neighbouring slots of one value word
    rope = RotaryEmbedding(d, traditional=trad, base=10000.0)
    base = _view(rng, cuda, nb, bs, hkv, d, bits, gs, tables, lens)
    counter = torch.zeros(_native.APPEND_COUNTER_INTS, dtype=torch.int32, device=cuda)
    for slots in (tuple(range(S)), (7, 3, 11, 4, 5, 0, 2, 1), (6, -1, 9, S + 2, 10)):
        a, b = _clone(base, cuda), _clone(base, cuda)
        for rep in range(2):  # two calls in a row: the counter is back at zero
            n = len(slots)
            k = torch.from_numpy(rng.standard_normal((n, hkv, d)).astype(np.float16) * 3).to(cuda)
            val = torch.from_numpy(rng.standard_normal((n, hkv, d)).astype(np.float16) * 3).to(cuda)
            q = torch.from_numpy(rng.standard_normal((n, hq, d)).astype(np.float16)).to(cuda)
            qa = _two_launches(a, slots, k, val, q, rope, cuda)
            qb = _one_launch(b, slots, k, val, q, rope, cuda, counter)
            torch.cuda.synchronize()
            assert torch.equal(qa, qb), (slots, rep)
            assert torch.equal(a.kv_lens, b.kv_lens), (slots, rep)
            for x, y in zip(a.page_arrays(), b.page_arrays()):
                assert torch.equal(x, y), (slots, rep)
            assert not counter.any()


def test_append_rejects_unsupported_geometry(cuda):
    lib = _native.load()
    z = torch.zeros(64, dtype=torch.int32, device=cuda)
    p = z.data_ptr()
    rc = lib.emx_affine_cache_append_rope(p, p, p, 1, p, 1, 1, p, p, 1, 128, 128, 4, 128, 1, p, p, p, p, p, p, p,
                                          128, 0, None, None, 0, None)
    assert rc == _native.EMX_ERR_UNSUPPORTED


@pytest.mark.parametrize("bs,trad,S,hkv,dt,rot", [(128, False, 12, 4, "f16", 128), (16, True, 12, 4, "f16", 128),
                                                  (128, False, 80, 1, "f16", 128), (16, True, 80, 1, "f16", 128),
                                                  (128, False, 12, 4, "bf16", 64), (16, True, 12, 4, "f32", 64),
                                                  (32, False, 12, 2, "f32", 128), (128, True, 12, 4, "bf16", 32)])
def test_fp8_append_matches_the_two_launch_write(cuda, bs, trad, S, hkv, dt, rot):
    """``emx_fp8_cache_append_rope`` against ``emx_cache_slots`` + ``emx_fp8_cache_write_rope``: codes, page
    scales, kv_lens and the turned queries bit for bit.  80 one-head tokens: more (token, pair) angles than
    the one-launch write's LDS table holds (each value turned with its own sincosf)."""
    print(f"[fp8 append bs={bs} traditional={trad} S={S} hkv={hkv} dtype={dt} rot={rot}]", flush=True)
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[dt]
    code = {"f16": _native.DTYPE_F16, "bf16": _native.DTYPE_BF16, "f32": _native.DTYPE_F32}[dt]
    from easymlx_amd import Fp8PageCacheView

    rng = np.random.default_rng(500 + bs + S)
    hq, d, mb = 16, 128, 5
    nb = S * mb + 3
    tables = rng.permutation(nb)[:S * mb].astype(np.int32).reshape(S, mb)
    lens = rng.integers(0, mb * bs, S).astype(np.int32)
    lens[1] = bs
    lens[2] = mb * bs
    tables[3, lens[3] // bs] = -1
    rope = RotaryEmbedding(rot, traditional=trad, base=10000.0)
    lib = _native.load()
    st = torch.cuda.current_stream(cuda).cuda_stream

    def view():
        kc = torch.from_numpy(rng.integers(0, 256, (nb, bs, hkv, d), dtype=np.uint8)).to(cuda)
        return Fp8PageCacheView(key_cache=kc, value_cache=kc.clone(),
                                k_scales=torch.from_numpy(rng.random(nb, dtype=np.float32)).to(cuda),
                                v_scales=torch.from_numpy(rng.random(nb, dtype=np.float32)).to(cuda),
                                block_tables=torch.from_numpy(tables).to(cuda),
                                kv_lens=torch.from_numpy(lens).to(cuda), block_size=bs, num_kv_heads=hkv,
                                head_dim=d)

    base = view()
    counter = torch.zeros(_native.APPEND_COUNTER_INTS, dtype=torch.int32, device=cuda)
    ws = torch.empty(int(lib.emx_fp8_write_workspace_bytes()), dtype=torch.uint8, device=cuda)
    inv = rope.inv_freq(cuda)
    for slots in (tuple(range(S)), (7, 3, 11, 4, 0, 2), (6, -1, 9, S + 2, 10)):
        a = [t.clone() for t in (base.key_cache, base.value_cache, base.k_scales, base.v_scales, base.kv_lens)]
        b = [t.clone() for t in a]
        bt = base.block_tables
        for rep in range(2):
            n = len(slots)
            k = torch.from_numpy(rng.standard_normal((n, hkv, d)).astype(np.float32) * 3).to(cuda).to(tdt)
            v = torch.from_numpy(rng.standard_normal((n, hkv, d)).astype(np.float32) * 3).to(cuda).to(tdt)
            q = torch.from_numpy(rng.standard_normal((n, hq, d)).astype(np.float16)).to(cuda)
            meta = torch.tensor(list(slots) + list(range(n + 1)), dtype=torch.int32, device=cuda)
            mapping = torch.empty(n, dtype=torch.int32, device=cuda)
            pos = torch.empty(n, dtype=torch.int32, device=cuda)
            _native.check(lib.emx_cache_slots(meta[:n].data_ptr(), meta[n:].data_ptr(), n, n, bt.data_ptr(), S, mb,
                                              bs, a[4].data_ptr(), mapping.data_ptr(), pos.data_ptr(), st))
            qa = torch.empty_like(q)
            _native.check(lib.emx_fp8_cache_write_rope(
                k.data_ptr(), v.data_ptr(), code, mapping.data_ptr(), n, hkv, d, bs, nb,
                a[0].data_ptr(), a[1].data_ptr(), a[2].data_ptr(), a[3].data_ptr(), ws.data_ptr(), ws.numel(),
                pos.data_ptr(), inv.data_ptr(), rope.dims, int(trad), q.data_ptr(), qa.data_ptr(), hq, st))
            qb = torch.empty_like(q)
            _native.check(lib.emx_fp8_cache_append_rope(
                k.data_ptr(), v.data_ptr(), code, meta[:n].data_ptr(), n, bt.data_ptr(), S, mb,
                b[4].data_ptr(), counter.data_ptr(), hkv, d, bs, nb, b[0].data_ptr(), b[1].data_ptr(),
                b[2].data_ptr(), b[3].data_ptr(), inv.data_ptr(), rope.dims, int(trad), q.data_ptr(), qb.data_ptr(),
                hq, st))
            torch.cuda.synchronize()
            assert torch.equal(qa, qb), (slots, rep)
            for x, y in zip(a, b):
                assert torch.equal(x, y), (slots, rep)
            assert not counter.any()
