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
