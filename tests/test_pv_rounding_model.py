"""A float64 model of the decode kernels' PV arithmetic: P' = p * v_scale rounded once to fp16 and its rounding
error folded into the fp32 bias term at the centre code 2^(bits-1).

The short-context stress batches of ``test_gpu_decode.py::test_decode_bias_cancellation`` (large value biases,
outputs near zero where sum P' * code cancels against sum p * v_bias) are run through three versions of the
arithmetic against the exact attention (float64, fp32-dequantized values, as the oracle): a single uncentred fp16
P', the centred one the kernels use, and P' as fp16 hi + lo (two MFMA passes).  This pins the claim that the
centred form keeps those batches well inside the attention tolerance, for the 4x4x4 kernel's operand (elements 2,
3 of each quad enter / 16) and the 16x16 kernel's.
"""

import numpy as np
import pytest

from easymlx_amd.workloads import decode_workload
from oracle.affine import affine_quantize, unpack_codes

ATOL, RTOL = 2e-3, 1e-2


def _h16(x):
    return x.astype(np.float16).astype(np.float32)


def _worst(wl, div16):
    d, g, hkv, hq, bits = wl.head_dim, wl.group_size, wl.num_kv_heads, wl.num_q_heads, wl.bits
    G, HG, c0 = d // g, hq // hkv, 2 ** (bits - 1)
    kc, ks, kb = affine_quantize(wl.k, g, bits)
    vc, vs, vb = affine_quantize(wl.v, g, bits)
    kd = (unpack_codes(kc, bits).reshape(-1, hkv, G, g) * ks.astype(np.float64)[..., None]
          + kb.astype(np.float64)[..., None]).reshape(-1, hkv, d)
    vcod = unpack_codes(vc, bits).astype(np.float64).reshape(-1, hkv, G, g)
    vs32, vb64 = vs.astype(np.float32), vb.astype(np.float64)
    vd = (vcod * vs32.astype(np.float64)[..., None] + vb64[..., None]).reshape(-1, hkv, d)
    worst = {"single": 0.0, "centred": 0.0, "hi_lo": 0.0}
    off = 0
    for si, n in enumerate(wl.kv_lens):
        n = int(n)
        K, V = kd[off:off + n], vd[off:off + n]
        for h in range(hq):
            kh = h // HG
            s = (K[:, kh] @ wl.q[si, h].astype(np.float64)) / np.sqrt(d)
            e = np.exp(s - s.max())
            exact = (e[:, None] * V[:, kh]).sum(0) / e.sum()
            tol = ATOL + RTOL * np.abs(exact)
            p = np.exp(s - s.max()).astype(np.float32)
            lsum = p.sum(dtype=np.float64)
            for gi in range(G):
                x = (p * vs32[off:off + n, kh, gi]).astype(np.float32)
                if div16:  # elements 2, 3 of each token quad enter the 4x4x4 MFMA divided by 16
                    f = np.where(np.arange(n) % 4 >= 2, 1 / 16, 1.0).astype(np.float32)
                    hi = _h16(x * f) / f
                else:
                    hi = _h16(x)
                lo = x - hi
                C = vcod[off:off + n, kh, gi]
                pb = (p.astype(np.float64) * vb64[off:off + n, kh, gi]).sum()
                sl = slice(gi * g, (gi + 1) * g)
                for name, o in (("single", (hi[:, None] * C).sum(0) + pb),
                                ("centred", (hi[:, None] * C).sum(0) + pb + (lo * c0).sum()),
                                ("hi_lo", ((hi + lo)[:, None] * C).sum(0) + pb)):
                    worst[name] = max(worst[name], float((np.abs(o / lsum - exact[sl]) / tol[sl]).max()))
        off += n
    return worst


@pytest.mark.parametrize("seed,bits,hq,gs,div16", [(332, 4, 64, 64, False), (334, 4, 32, 64, True),
                                                  (331, 8, 32, 64, False)])
def test_centred_p_prime_within_tolerance(seed, bits, hq, gs, div16):
    wl = decode_workload(seed=seed, num_seqs=120, ctx_range=(1, 256), bits=bits, num_q_heads=hq, group_size=gs)
    w = _worst(wl, div16)
    assert w["hi_lo"] < 1e-2
    assert w["centred"] < 0.6, w
    assert w["centred"] < w["single"], w
