"""Fused RoPE on the GPU: the rotation kernel vs a float64 restatement (fp32 angles, as the reference's
mlx.core.fast.rope forms them), the fused quantize-on-write bit-identical to rotate-then-write, and
concatenate_to_cache with a RotaryEmbedding vs the same RoPE applied as a plain callable."""

import numpy as np
import pytest
import torch

from easymlx_amd import AffinePageCacheView, OperationRegistry, PageMetadata, RotaryEmbedding, build_query_start_loc
from easymlx_amd import _native
from easymlx_amd.caching.paged import affine_pool
from tests.helpers import assert_attention_close

pytestmark = pytest.mark.gpu


def _np_rope_f16(x16, pos, inv32, dims, traditional):
    """Angles as fp32 products (position * inv_freq), rotation in float64, rounded to fp16."""
    x = x16.astype(np.float64)
    th = (pos.astype(np.float32)[:, None] * inv32[None, :]).astype(np.float64)  # [rows, half]
    c, s = np.cos(th)[:, None, :], np.sin(th)[:, None, :]
    half = dims // 2
    out = x.copy()
    if traditional:
        x0, x1 = x[..., 0:dims:2], x[..., 1:dims:2]
        out[..., 0:dims:2], out[..., 1:dims:2] = x0 * c - x1 * s, x0 * s + x1 * c
    else:
        x0, x1 = x[..., :half], x[..., half:dims]
        out[..., :half], out[..., half:dims] = x0 * c - x1 * s, x0 * s + x1 * c
    return out.astype(np.float16)


def _rope_rows(x, pos, rope):
    lib = _native.load()
    _native.check(lib.emx_rope_rows(x.data_ptr(), int(x.shape[0]), int(x.shape[1]), int(x.shape[2]), pos.data_ptr(),
                                    rope.inv_freq(x.device).data_ptr(), rope.dims, int(rope.traditional),
                                    torch.cuda.current_stream(x.device).cuda_stream))


@pytest.mark.parametrize("traditional", [False, True])
@pytest.mark.parametrize("kind", ["default", "llama3", "half-dims"])
def test_rope_rows_vs_float64(cuda, traditional, kind):
    print(f"[rope rows {kind} traditional={traditional}]", flush=True)
    rng = np.random.default_rng(8)
    if kind == "llama3":
        rope = RotaryEmbedding.llama3(128, base=500000.0, traditional=traditional)
    else:
        rope = RotaryEmbedding(128 if kind == "default" else 64, base=10000.0, traditional=traditional)
    x = (rng.standard_normal((300, 8, 128)) * 3).astype(np.float16)
    pos = rng.integers(0, 40000, 300).astype(np.int32)
    xt = torch.from_numpy(x).to(cuda)
    _rope_rows(xt, torch.from_numpy(pos).to(cuda), rope)
    got = xt.cpu().numpy()
    exp = _np_rope_f16(x, pos, rope.inv_freq_cpu.numpy(), rope.dims, traditional)
    diff = np.abs(got.astype(np.float64) - exp.astype(np.float64))
    # one fp16 ulp at the larger magnitude of the two, plus the fp32 arithmetic of the rotation
    # (|x| * 2^-22 absolute: products and sin / cos rounded in fp32 -- it shows where x0*c - x1*s cancels)
    ulp = np.spacing(np.maximum(np.abs(got), np.abs(exp)).astype(np.float16)).astype(np.float64)
    arith = np.abs(x.astype(np.float64)).max(axis=-1, keepdims=True) * 2.0 ** -22
    assert np.all(diff <= ulp + arith), f"max {np.max(diff / (ulp + arith))} of the bound"
    assert np.mean(got == exp) > 0.99
    assert np.array_equal(got[..., rope.dims:], x[..., rope.dims:])


@pytest.mark.parametrize("bits,T,rot,trad", [(4, 300, 128, 0), (4, 32, 128, 0), (8, 77, 128, 0), (4, 32, 64, 0),
                                             (4, 300, 64, 0), (8, 32, 128, 0), (4, 32, 128, 1), (8, 40, 64, 1),
                                             (4, 7, 32, 0), (4, 24, 128, 0)])
def test_fused_write_equals_rotate_then_write(cuda, bits, T, rot, trad):
    """One launch (rotate K in LDS, quantize) == emx_rope_rows on K, then emx_affine_cache_write: every byte.
    The queries come out turned into a separate tensor (dims past rot copied), or turned in place."""
    print(f"[fused rope write bits={bits} T={T} rot={rot} traditional={trad}]", flush=True)
    rng = np.random.default_rng(9 + bits + T)
    hkv, d, bs, nb = 8, 128, 128, 16
    rope = RotaryEmbedding.llama3(rot, base=500000.0, traditional=bool(trad))
    k = torch.from_numpy((rng.standard_normal((T, hkv, d)) * 2).astype(np.float16)).to(cuda)
    v = torch.from_numpy((rng.standard_normal((T, hkv, d)) * 2).astype(np.float16)).to(cuda)
    slots = torch.from_numpy(rng.permutation(nb * bs)[:T].astype(np.int32)).to(cuda)
    if T == 24:  # consecutive slots: tokens of the call share value words
        slots = torch.arange(100, 100 + T, dtype=torch.int32, device=cuda)
    pos = torch.from_numpy(rng.integers(0, 30000, T).astype(np.int32)).to(cuda)
    tables = torch.zeros((1, 1), dtype=torch.int32, device=cuda)
    lens = torch.zeros(1, dtype=torch.int32, device=cuda)
    a = affine_pool(num_blocks=nb, num_kv_heads=hkv, head_dim=d, block_size=bs, bits=bits, group_size=64,
                    block_tables=tables, kv_lens=lens)
    b = affine_pool(num_blocks=nb, num_kv_heads=hkv, head_dim=d, block_size=bs, bits=bits, group_size=64,
                    block_tables=tables, kv_lens=lens)
    lib = _native.load()
    st = torch.cuda.current_stream(cuda).cuda_stream
    inv = rope.inv_freq(cuda)
    q = torch.from_numpy(rng.standard_normal((T, 32, d)).astype(np.float16)).to(cuda)
    q0 = q.clone()
    qo = torch.full_like(q, float("nan"))  # every element written by the launch
    qa = q.clone()  # turned in place

    def call(q_in, q_out):
        _native.check(lib.emx_affine_cache_write_rope(
            k.data_ptr(), v.data_ptr(), slots.data_ptr(), T, hkv, d, 64, bits, bs, nb, a.key_cache.data_ptr(),
            a.k_scales.data_ptr(), a.k_biases.data_ptr(), a.value_cache.data_ptr(), a.v_scales.data_ptr(),
            a.v_biases.data_ptr(), pos.data_ptr(), inv.data_ptr(), rope.dims, trad, q_in, q_out.data_ptr(), 32, st))

    call(q.data_ptr(), qo)
    call(None, qa)  # the same write again: the pages come out the same
    kr, qb = k.clone(), q.clone()
    _rope_rows(kr, pos, rope)
    _rope_rows(qb, pos, rope)
    b.write_slots(kr, v, slots)
    torch.cuda.synchronize()
    assert torch.equal(q, q0), "queries_in left as it was"
    assert torch.equal(qo, qb), "queries turned out of place"
    assert torch.equal(qa, qb), "queries turned in place"
    for name in ("key_cache", "k_scales", "k_biases", "value_cache", "v_scales", "v_biases"):
        assert torch.equal(getattr(a, name), getattr(b, name)), name


def test_concatenate_fused_vs_callable(cuda):
    """Prefill then decode steps: RotaryEmbedding (fused) vs the same RoPE as a plain callable (rotated in torch,
    then written): queries within 2 fp16 ulp, attention outputs within the attention tolerance."""
    print("[concatenate fused rope]", flush=True)
    rng = np.random.default_rng(10)
    S, hq, hkv, d = 3, 32, 8, 128
    rope = RotaryEmbedding.llama3(128, base=500000.0)
    plain = lambda x, offset=0: rope(x, offset=offset)  # noqa: E731 -- not a RotaryEmbedding: unfused path
    views = [AffinePageCacheView.init(num_seqs=S, max_seq_len=800, num_kv_heads=hkv, head_dim=d, block_size=128,
                                      bits=4, group_size=64, device=cuda) for _ in range(2)]
    op = OperationRegistry.create("unified_attention")
    for qlens in ([200, 37, 1], [1, 1, 1], [20, 1, 64]):
        T = sum(qlens)
        q = torch.from_numpy(rng.standard_normal((T, hq, d)).astype(np.float16)).to(cuda)
        k = torch.from_numpy((rng.standard_normal((T, hkv, d)) * 2).astype(np.float16)).to(cuda)
        v = torch.from_numpy((rng.standard_normal((T, hkv, d)) * 2).astype(np.float16)).to(cuda)
        outs = []
        for view, r in zip(views, (rope, plain)):
            md = PageMetadata(query_start_loc=build_query_start_loc(qlens, device=cuda), slot_ids=tuple(range(S)))
            qq, kc, vc, md = view.concatenate_to_cache(q, k, v, cache_metadata=md, rope=r)
            res = op(query=qq, key=kc, value=vc, cache_metadata=md, cache_view=view, scale=d ** -0.5)
            outs.append((qq.float().cpu().numpy(), res.attention_outputs.float().cpu().numpy()))
        torch.cuda.synchronize()
        (qa, oa), (qb, ob) = outs
        ulp = np.spacing(np.maximum(np.abs(qa), np.abs(qb)).astype(np.float16)).astype(np.float64)
        arith = np.abs(q.float().cpu().numpy()).max(axis=-1, keepdims=True) * 2.0 ** -21
        assert np.all(np.abs(qa - qb) <= 2 * ulp + arith), f"queries differ at step {qlens}"
        assert_attention_close(oa, ob.astype(np.float64), f"fused vs callable {qlens}")
        assert views[0].kv_lens.cpu().tolist() == views[1].kv_lens.cpu().tolist()


@pytest.mark.parametrize("traditional,T,hkv", [(False, 200, 8), (True, 200, 8), (False, 24, 8), (False, 300, 1),
                                                (True, 300, 1)])
def test_fp8_fused_write_equals_rotate_then_write(cuda, traditional, T, hkv):
    """FP8 cache: the call's scale and the codes over the turned keys, in the write kernels == emx_rope_rows on K,
    then the plain FP8 write: every byte of the pages and every page scale.  T = 24 (8 heads) and T = 300 (one
    head): the one-launch write, the latter with too many (token, pair) angles for its LDS table, so every
    value is turned with its own sincosf."""
    from easymlx_amd import Fp8PageCacheView

    print(f"[fp8 fused rope write traditional={traditional} T={T} hkv={hkv}]", flush=True)
    rng = np.random.default_rng(11 + traditional + T)
    d, bs, nb = 128, 32, 64  # T = 24: the one-launch write (queries turned by its extra workgroups)
    rope = RotaryEmbedding.llama3(128, base=500000.0, traditional=traditional)
    k = torch.from_numpy((rng.standard_normal((T, hkv, d)) * 2).astype(np.float16)).to(cuda)
    v = torch.from_numpy((rng.standard_normal((T, hkv, d)) * 2).astype(np.float16)).to(cuda)
    slots = torch.from_numpy(rng.permutation(nb * bs)[:T].astype(np.int32)).to(cuda)
    pos = torch.from_numpy(rng.integers(0, 30000, T).astype(np.int32)).to(cuda)

    def view():
        shape = (nb, bs, hkv, d)
        return Fp8PageCacheView(key_cache=torch.zeros(shape, dtype=torch.uint8, device=cuda),
                                value_cache=torch.zeros(shape, dtype=torch.uint8, device=cuda),
                                k_scales=torch.zeros(nb, device=cuda), v_scales=torch.zeros(nb, device=cuda),
                                block_tables=torch.zeros((1, 1), dtype=torch.int32, device=cuda),
                                kv_lens=torch.zeros(1, dtype=torch.int32, device=cuda), block_size=bs,
                                num_kv_heads=hkv, head_dim=d)

    a, b = view(), view()
    lib = _native.load()
    ws = torch.empty(int(lib.emx_fp8_write_workspace_bytes()), dtype=torch.uint8, device=cuda)
    q = torch.from_numpy(rng.standard_normal((T, 16, d)).astype(np.float16)).to(cuda)
    q0 = q.clone()
    qo = torch.full_like(q, float("nan"))  # every element written by the launch
    _native.check(lib.emx_fp8_cache_write_rope(
        k.data_ptr(), v.data_ptr(), _native.DTYPE_F16, slots.data_ptr(), T, hkv, d, bs, nb, a.key_cache.data_ptr(),
        a.value_cache.data_ptr(), a.k_scales.data_ptr(), a.v_scales.data_ptr(), ws.data_ptr(), ws.numel(),
        pos.data_ptr(), rope.inv_freq(cuda).data_ptr(), rope.dims, int(traditional), q.data_ptr(), qo.data_ptr(), 16,
        torch.cuda.current_stream(cuda).cuda_stream))
    kr, qb = k.clone(), q.clone()
    _rope_rows(kr, pos, rope)
    _rope_rows(qb, pos, rope)
    b.write_slots(kr, v, slots)
    torch.cuda.synchronize()
    assert torch.equal(q, q0), "queries_in left as it was"
    assert torch.equal(qo, qb), "queries"
    for name in ("key_cache", "value_cache", "k_scales", "v_scales"):
        assert torch.equal(getattr(a, name), getattr(b, name)), name


def test_fp8_concatenate_fused_vs_callable(cuda):
    """Fp8PageCacheView.concatenate_to_cache with a RotaryEmbedding vs the same RoPE as a plain callable."""
    from easymlx_amd import Fp8PageCacheView, paged_attention

    print("[fp8 concatenate fused rope]", flush=True)
    rng = np.random.default_rng(13)
    S, hq, hkv, d, bs, mb = 3, 32, 8, 128, 32, 16
    rope = RotaryEmbedding(128, base=10000.0)
    plain = lambda x, offset=0: rope(x, offset=offset)  # noqa: E731

    def view():
        nb = S * mb
        shape = (nb, bs, hkv, d)
        return Fp8PageCacheView(key_cache=torch.zeros(shape, dtype=torch.uint8, device=cuda),
                                value_cache=torch.zeros(shape, dtype=torch.uint8, device=cuda),
                                k_scales=torch.zeros(nb, device=cuda), v_scales=torch.zeros(nb, device=cuda),
                                block_tables=torch.arange(nb, dtype=torch.int32, device=cuda).reshape(S, mb),
                                kv_lens=torch.zeros(S, dtype=torch.int32, device=cuda), block_size=bs,
                                num_kv_heads=hkv, head_dim=d)

    views = [view(), view()]
    for qlens in ([150, 31, 1], [1, 1, 1]):
        T = sum(qlens)
        q = torch.from_numpy(rng.standard_normal((T, hq, d)).astype(np.float16)).to(cuda)
        k = torch.from_numpy((rng.standard_normal((T, hkv, d)) * 2).astype(np.float16)).to(cuda)
        v = torch.from_numpy((rng.standard_normal((T, hkv, d)) * 2).astype(np.float16)).to(cuda)
        outs = []
        for vw, r in zip(views, (rope, plain)):
            md = PageMetadata(query_start_loc=build_query_start_loc(qlens, device=cuda), slot_ids=tuple(range(S)))
            qq, kc, vc, md = vw.concatenate_to_cache(q, k, v, cache_metadata=md, rope=r)
            o = paged_attention(qq, kc, vc, md.block_tables, md.kv_lens, md.query_start_loc, k_scale=vw.k_scales,
                                v_scale=vw.v_scales)
            outs.append(o.float().cpu().numpy())
        torch.cuda.synchronize()
        assert_attention_close(outs[0], outs[1].astype(np.float64), f"fp8 fused vs callable {qlens}")
