"""emx_fp8_cache_write_noalloc (library-held scratch, no workspace) against emx_fp8_cache_write.

Both entry points are called through the C ABI on the same inputs, each into its
own zero-initialised cache; codes and per-page scales must be bit-identical.
Two calls in a row on the no-alloc entry point, the second smaller (both take
the two-launch path whose maxima live in the scratch), then a decode-size call
(one launch, no scratch).
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _caches(nb, bs, hkv, d, dev):
    shape = (nb, bs, hkv, d)
    return (torch.zeros(shape, dtype=torch.uint8, device=dev), torch.zeros(shape, dtype=torch.uint8, device=dev),
            torch.zeros(nb, device=dev), torch.zeros(nb, device=dev))


def test_fp8_noalloc_matches_workspace_entry_point(cuda):
    from easymlx_amd import _native

    lib = _native.load()
    rng = np.random.default_rng(31)
    nb, bs, hkv, d = 96, 128, 4, 128
    stream = torch.cuda.current_stream(cuda).cuda_stream
    ref = _caches(nb, bs, hkv, d, cuda)
    got = _caches(nb, bs, hkv, d, cuda)
    ws = torch.empty(lib.emx_fp8_write_workspace_bytes(), dtype=torch.uint8, device=cuda)
    for t in (4096, 1024, 24):  # 2M and 512K values per tensor: two launches; 12K: one launch
        print(f"[fp8 noalloc t={t}]", flush=True)
        k = torch.from_numpy((rng.standard_normal((t, hkv, d)) * rng.uniform(0.2, 6.0, (1, hkv, d)))
                             .astype(np.float16)).to(cuda)
        v = torch.from_numpy(rng.standard_normal((t, hkv, d)).astype(np.float16)).to(cuda)
        slot = rng.permutation(nb * bs)[:t].astype(np.int32)
        slot[rng.random(t) < 0.05] = -1
        s = torch.from_numpy(slot).to(cuda)
        common = (k.data_ptr(), v.data_ptr(), _native.DTYPE_F16, s.data_ptr(), t, hkv, d, bs, nb)
        _native.check(lib.emx_fp8_cache_write(*common, *(x.data_ptr() for x in ref), ws.data_ptr(), ws.numel(),
                                              stream))
        _native.check(lib.emx_fp8_cache_write_noalloc(*common, *(x.data_ptr() for x in got), stream))
        torch.cuda.synchronize()
        for a, b, name in zip(got, ref, ("key_cache", "value_cache", "k_scales", "v_scales")):
            assert torch.equal(a, b), f"{name} differs after the {t}-token write"


def test_fp8_noalloc_one_slot_per_stream(cuda):
    """Two streams writing at once each get a scratch slot of their own (bit-identical to the workspace entry
    point on both); a stream beyond the slots is refused with NotImplementedError, nothing written."""
    from easymlx_amd import _native

    lib = _native.load()
    rng = np.random.default_rng(77)
    nb, bs, hkv, d, t = 96, 128, 4, 128, 2048  # 1M values per tensor: the two-launch path (scratch)
    ws = torch.empty(lib.emx_fp8_write_workspace_bytes(), dtype=torch.uint8, device=cuda)
    streams = [torch.cuda.Stream(cuda) for _ in range(2)]
    jobs = []
    for i, s in enumerate(streams):
        k = torch.from_numpy((rng.standard_normal((t, hkv, d)) * (1 + 3 * i)).astype(np.float16)).to(cuda)
        v = torch.from_numpy(rng.standard_normal((t, hkv, d)).astype(np.float16)).to(cuda)
        slot = torch.from_numpy(rng.permutation(nb * bs)[:t].astype(np.int32)).to(cuda)
        jobs.append((k, v, slot, _caches(nb, bs, hkv, d, cuda), _caches(nb, bs, hkv, d, cuda)))
    torch.cuda.synchronize()
    for rep in range(3):  # both streams' launches interleave on the GPU
        for s, (k, v, slot, got, _) in zip(streams, jobs):
            common = (k.data_ptr(), v.data_ptr(), _native.DTYPE_F16, slot.data_ptr(), t, hkv, d, bs, nb)
            _native.check(lib.emx_fp8_cache_write_noalloc(*common, *(x.data_ptr() for x in got), s.cuda_stream))
    torch.cuda.synchronize()
    st = torch.cuda.current_stream(cuda).cuda_stream
    for k, v, slot, got, ref in jobs:
        common = (k.data_ptr(), v.data_ptr(), _native.DTYPE_F16, slot.data_ptr(), t, hkv, d, bs, nb)
        for rep in range(3):
            _native.check(lib.emx_fp8_cache_write(*common, *(x.data_ptr() for x in ref), ws.data_ptr(), ws.numel(),
                                                  st))
        torch.cuda.synchronize()
        for a, b, name in zip(got, ref, ("key_cache", "value_cache", "k_scales", "v_scales")):
            assert torch.equal(a, b), f"{name} differs (per-stream scratch)"
    # more streams than slots: the first stream past the slots is refused
    k, v, slot, got, _ = jobs[0]
    common = (k.data_ptr(), v.data_ptr(), _native.DTYPE_F16, slot.data_ptr(), t, hkv, d, bs, nb)
    extra = []
    refused = False
    for _ in range(9):
        s = torch.cuda.Stream(cuda)
        extra.append(s)
        rc = lib.emx_fp8_cache_write_noalloc(*common, *(x.data_ptr() for x in got), s.cuda_stream)
        if rc == _native.EMX_ERR_UNSUPPORTED:
            refused = True
            with pytest.raises(NotImplementedError, match="streams"):
                _native.check(rc)
            break
        _native.check(rc)
    torch.cuda.synchronize()
    assert refused, "a ninth stream was not refused"
