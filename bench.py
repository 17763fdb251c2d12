"""Benchmark: 4-bit-KV paged decode attention, batch 32, Llama-3-8B head shape, on one MI355X.

One step = one decode call of the hot path (paged attention over affine
4-bit pages: 32 sequences x 8 KV heads x contexts U[512, 4096], 32 query
heads, head_dim 128, page 128, group 64) with all inputs resident in HBM.
Steps rotate over >= 4 independent copies of the page pool (>= 1.5 GiB in
total) so the 256 MB Infinity Cache cannot serve the K/V reads.  The calls are
made through the C ABI with prepared argument lists (the Python wrapper's host
cost per call exceeds the kernel's), after checking that they reproduce the
public operator's result on every pool.

Prints one JSON line.  ``value`` = achieved HBM GB/s on algorithmic bytes
(K/V codes + scales + biases of every live token) over the timed steps.
Auxiliary fields (not the headline), each over its own rotated pools: the
ragged unified step (c3: four 512-token prefill chunks + 28 decode rows), the
long-context decode (c4: 8 x 32768 tokens, Hq 64) and the fused
quantize-on-write (one appended token per c2 sequence; four 512-token chunks).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=400)
    p.add_argument("--warmup", type=int, default=40)
    p.add_argument("--pool-gib", type=float, default=1.5, help="total size of the rotated page pools")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-aux", action="store_true", help="skip the c3 / c4 / quantize-on-write measurements")
    p.add_argument("--aux-only", choices=("c3", "c4", "write", "op", "fp8", "shapes"),
                   help="run one auxiliary measurement alone and print its JSON (for profiler runs)")
    p.add_argument("--layers", type=int, default=32,
                   help="decode calls per model step: kv_lens change at every step's first call (Llama-3-8B: 32)")
    p.add_argument("--cpu-seqs", type=int, default=0, help="sequences in the CPU baseline sample (0 = auto)")
    p.add_argument("--copy-probe-mib", type=int, default=0,
                   help="after the timed region, run 5 plain device copies of this size (counter calibration)")
    return p.parse_args()


def cpu_baseline(wl, n_seqs: int | None):
    """Time the C oracle (scalar restatement, OpenMP over (seq, kv_head)) on a bounded sample."""
    from oracle.affine import affine_quantize

    lib_path = os.path.join(ROOT, "oracle", "c", "liboracle.so")
    if not os.path.exists(lib_path):
        return None
    lib = ctypes.CDLL(lib_path)
    cores = min(len(os.sched_getaffinity(0)), 16)
    os.environ.setdefault("OMP_NUM_THREADS", str(cores))
    P = ctypes.c_void_p
    lib.oracle_decode_affine.argtypes = [P] * 9 + [ctypes.c_int] * 9 + [ctypes.c_float, P]
    n = n_seqs or wl.num_seqs
    bs, hkv, d, g, bits = wl.block_size, wl.num_kv_heads, wl.head_dim, wl.group_size, wl.bits
    lens = wl.kv_lens[:n]
    ntok = int(lens.sum())
    slot = wl.slot[:ntok]
    nb = wl.num_blocks
    res = {}
    for name, x in (("k", wl.k[:ntok]), ("v", wl.v[:ntok])):
        c, s, b = affine_quantize(x, g, bits)
        C = np.zeros((nb, bs, hkv, c.shape[-1]), np.uint32)
        S = np.zeros((nb, bs, hkv, s.shape[-1]), np.float16)
        B = np.zeros_like(S)
        C[slot // bs, slot % bs], S[slot // bs, slot % bs], B[slot // bs, slot % bs] = c, s, b
        res[name] = (C, S.view(np.uint16), B.view(np.uint16))
    q = np.ascontiguousarray(wl.q[:n]).view(np.uint16)
    tables = np.ascontiguousarray(wl.block_tables[:n])
    out = np.zeros((n, wl.num_q_heads, d), np.float32)
    ptr = lambda a: a.ctypes.data_as(P)  # noqa: E731
    reps, t_total = 0, 0.0
    while t_total < 12.0 and reps < 2000:
        t0 = time.perf_counter()
        lib.oracle_decode_affine(ptr(q), ptr(res["k"][0]), ptr(res["k"][1]), ptr(res["k"][2]), ptr(res["v"][0]),
                                 ptr(res["v"][1]), ptr(res["v"][2]), ptr(tables), ptr(np.ascontiguousarray(lens)), n,
                                 wl.num_q_heads, hkv, d, bs, nb, tables.shape[1], bits, g,
                                 ctypes.c_float(1.0 / math.sqrt(d)), ptr(out))
        t_total += time.perf_counter() - t0
        reps += 1
    per = t_total / reps
    per_tok_head = 2 * (d * bits // 8 + (d // g) * 4)
    nbytes = ntok * hkv * per_tok_head
    return {
        "value": round(nbytes / per / 1e9, 4),
        "unit": "GB/s",
        "cores": cores,
        "host_cores": {"affinity": len(os.sched_getaffinity(0)), "cpu_count": os.cpu_count()},
        "kind": "port",
        "sample": f"C oracle (oracle/c/oracle.c, OpenMP over (seq, kv_head), {cores} threads) on {n} of "
                  f"{wl.num_seqs} sequences of the same workload ({ntok} tokens), {reps} reps, {per * 1e3:.1f} ms "
                  f"each = {n / per:.1f} decode rows/s",
        "numpy_restatement": numpy_baseline(wl, res),
    }


def numpy_baseline(wl, pages, n_seqs=4, budget_s=8.0):
    """The NumPy restatement of the reference's CPU path (``_paged_attention_reference``,
    unified_attention.py:187-281, as ``oracle.paged_attention``) plus the affine dequantize, timed on a bounded
    sample of the c2 workload (its first ``n_seqs`` sequences)."""
    from oracle.affine import affine_dequantize
    from oracle.paged_attention import paged_attention as np_attention

    bs, g, bits = wl.block_size, wl.group_size, wl.bits
    lens = wl.kv_lens[:n_seqs]
    ntok = int(lens.sum())
    q = wl.q[:n_seqs]
    qsl = np.arange(n_seqs + 1, dtype=np.int32)
    # only the sample's pages (renumbered), so each call dequantizes what it reads
    used = [int(b) for s in range(n_seqs) for b in wl.block_tables[s, :-(-int(lens[s]) // bs)]]
    remap = {b: i for i, b in enumerate(used)}
    tables = np.array([[remap.get(int(b), -1) for b in row] for row in wl.block_tables[:n_seqs]], np.int32)
    sub = {n: tuple(a[used] for a in pages[n]) for n in ("k", "v")}
    reps, t_total = 0, 0.0
    while t_total < budget_s and reps < 50:
        t0 = time.perf_counter()
        kc = affine_dequantize(sub["k"][0], sub["k"][1].view(np.float16), sub["k"][2].view(np.float16), g, bits,
                               round_to_fp16=False)
        vc = affine_dequantize(sub["v"][0], sub["v"][1].view(np.float16), sub["v"][2].view(np.float16), g, bits,
                               round_to_fp16=False)
        np_attention(q, kc, vc, tables, lens, qsl, compute_dtype=np.float32)
        t_total += time.perf_counter() - t0
        reps += 1
    per = t_total / reps
    nbytes = ntok * wl.num_kv_heads * 2 * (wl.head_dim * bits // 8 + (wl.head_dim // g) * 4)
    blas = {k: os.environ.get(k) for k in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS")}
    return {"value": round(nbytes / per / 1e9, 4), "unit": "GB/s", "kind": "port",
            "sample": f"oracle.paged_attention (numpy, fp32) + oracle.affine.affine_dequantize of the sample's pages "
                      f"per call, first {n_seqs} sequences of c2 ({ntok} tokens), {reps} reps, {per * 1e3:.1f} ms each",
            "threads_env": blas}


def measured_traffic():
    """HBM bytes per decode call from the committed counter summary (two rocprofv3 --pmc passes)."""
    path = os.path.join(ROOT, "profiles", "decode_q4_c2_hbm_traffic.md")
    try:
        for line in open(path):
            if line.startswith("TRAFFIC_BYTES_PER_CALL:"):
                return int(line.split(":")[1]), os.path.relpath(path, ROOT)
    except OSError:
        pass
    return None, None


class Setup:
    """Rotated copies of one workload's page pool and prepared C-ABI attention calls over them.

    The calls go straight through the C ABI (the drop-in boundary) with argument
    lists prepared here: the Python wrapper's host cost per call (validation,
    conversions) exceeds one ~30 us decode call and would otherwise be what is
    timed.  Each prepared call is checked to reproduce the public operator's
    output bit for bit.
    """

    def __init__(self, wl, pool_gib, dev, min_pools=4):
        import torch

        from easymlx_amd import _native, paged_attention
        from easymlx_amd.caching import affine_pool

        self.wl = wl
        mk = dict(num_blocks=wl.num_blocks, num_kv_heads=wl.num_kv_heads, head_dim=wl.head_dim,
                  block_size=wl.block_size, bits=wl.bits, group_size=wl.group_size)
        base = affine_pool(**mk, block_tables=torch.from_numpy(wl.block_tables).to(dev),
                           kv_lens=torch.from_numpy(wl.kv_lens).to(dev))
        base.write_slots(torch.from_numpy(wl.k).to(dev), torch.from_numpy(wl.v).to(dev),
                         torch.from_numpy(wl.slot.astype(np.int32)).to(dev))
        names = ("k_codes", "v_codes", "k_scales", "k_biases", "v_scales", "v_biases")
        self.pool_bytes = sum(getattr(base, n).numel() * getattr(base, n).element_size() for n in names)
        self.n_pools = max(min_pools, math.ceil(pool_gib * 2**30 / self.pool_bytes))
        self.pools = [base]
        for _ in range(self.n_pools - 1):
            p = affine_pool(**mk, block_tables=base.block_tables, kv_lens=base.kv_lens)
            for n in names:
                getattr(p, n).copy_(getattr(base, n))
            self.pools.append(p)
        q = torch.from_numpy(wl.q).to(dev)
        qsl = torch.from_numpy(wl.query_start_loc).to(dev)
        self.out = out = torch.empty_like(q)
        self._keep = (q, qsl)
        paged_attention(q, base.k_codes, base.v_codes, base.block_tables, base.kv_lens, qsl,
                        k_scales=base.k_scales, k_biases=base.k_biases, v_scales=base.v_scales,
                        v_biases=base.v_biases, bits=wl.bits, group_size=wl.group_size,
                        single_token_decode=bool(wl.single_token_decode), out=out)
        torch.cuda.synchronize()
        assert torch.isfinite(out).all(), f"non-finite attention output ({wl.name})"
        eager = out.clone()

        lib = _native.load()
        self._fn = lib.emx_paged_attention_affine
        self._check = _native.check
        T, hq, d = (int(x) for x in q.shape)
        S = int(wl.block_tables.shape[0])
        nws = lib.emx_paged_workspace_bytes(S, hq, wl.num_kv_heads, d, wl.block_tables.shape[1], wl.block_size)
        if not wl.single_token_decode:  # the prefill key split's partial states
            nws += lib.emx_paged_prefill_workspace_bytes(T, S, hq, wl.num_kv_heads, d)
        self.ws = torch.zeros(nws, dtype=torch.uint8, device=dev)
        stream = torch.cuda.current_stream(dev).cuda_stream
        self.args = [
            (q.data_ptr(), T, hq, d, p.k_codes.data_ptr(), p.k_scales.data_ptr(), p.k_biases.data_ptr(),
             p.v_codes.data_ptr(), p.v_scales.data_ptr(), p.v_biases.data_ptr(), wl.num_blocks, wl.block_size,
             wl.num_kv_heads, wl.bits, wl.group_size, p.block_tables.data_ptr(), S, wl.block_tables.shape[1],
             p.kv_lens.data_ptr(), qsl.data_ptr(), 1.0 / math.sqrt(d), 0, int(wl.single_token_decode),
             self.ws.data_ptr(), self.ws.numel(), out.data_ptr(), stream)
            for p in self.pools
        ]
        for i in range(self.n_pools):  # same result as the public operator, on every pool
            out.zero_()
            self.call(i)
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"C-ABI call differs from paged_attention ({wl.name})"

        # The same batch one decode step earlier: every sequence one token shorter (its pages hold
        # the token too).  Alternating the two every `layers` calls gives each model step's first
        # layer new kv_lens, as in serving; the decode's plan is keyed by the per-sequence item
        # counts, which a one-token step changes only where a sequence crosses an item boundary.
        lens_b = wl.kv_lens.copy()
        if wl.single_token_decode:
            lens_b = np.maximum(lens_b - 1, np.minimum(lens_b, 1)).astype(lens_b.dtype)
        self.kv_lens_b = torch.from_numpy(lens_b).to(dev)
        self.bytes_b = int(wl.kv_bytes() * (int(lens_b.sum()) / max(1, int(wl.kv_lens.sum()))))
        ikl = 18  # position of kv_lens in the argument tuple
        self.args_b = [a[:ikl] + (self.kv_lens_b.data_ptr(),) + a[ikl + 1:] for a in self.args]
        out_b = torch.empty_like(out)
        paged_attention(q, base.k_codes, base.v_codes, base.block_tables, self.kv_lens_b, qsl,
                        k_scales=base.k_scales, k_biases=base.k_biases, v_scales=base.v_scales,
                        v_biases=base.v_biases, bits=wl.bits, group_size=wl.group_size,
                        single_token_decode=bool(wl.single_token_decode), out=out_b)
        torch.cuda.synchronize()
        eager_b = out_b.clone()
        out.zero_()
        self.call(0, alt=True)
        torch.cuda.synchronize()
        assert torch.equal(out, eager_b), f"C-ABI call differs from paged_attention ({wl.name}, kv_lens b)"

        # the page-read probe over the same pools: exactly the slices this call reads, loads only
        self._probe = lib.emx_probe_page_read
        self.sink = torch.zeros(2048, dtype=torch.int32, device=dev)
        self.probe_args = [
            (p.k_codes.data_ptr(), p.k_scales.data_ptr(), p.k_biases.data_ptr(), p.v_codes.data_ptr(),
             p.v_scales.data_ptr(), p.v_biases.data_ptr(), wl.num_blocks, wl.block_size, wl.num_kv_heads, d, wl.bits,
             wl.group_size, p.block_tables.data_ptr(), S, wl.block_tables.shape[1], p.kv_lens.data_ptr(),
             self.sink.data_ptr(), self.sink.numel(), stream)
            for p in self.pools
        ]
        lens = np.maximum(wl.kv_lens.astype(np.int64), 0)
        per_tok = 2 * wl.head_dim * wl.bits // 8 + 4 * (wl.head_dim // wl.group_size) * 2
        self.probe_bytes = int(((lens + 63) // 64).sum()) * 64 * wl.num_kv_heads * per_tok

    def call(self, i, alt=False):
        rc = self._fn(*(self.args_b if alt else self.args)[i % self.n_pools])
        if rc:
            self._check(rc)

    def step_call(self, i, layers):
        """Call i of a run of model decode steps of `layers` layer calls each: kv_lens change at
        every step's first layer (the two contents alternate), the other layers repeat them."""
        self.call(i, alt=(i // layers) % 2 == 1)

    def set_probe_grid(self, words):
        self.probe_args = [a[:17] + (int(words),) + a[18:] for a in self.probe_args]

    def probe(self, i):
        rc = self._probe(*self.probe_args[i % self.n_pools])
        if rc:
            self._check(rc)


def warm(fn, seconds):
    """Clocks ramp up under sustained load: keep calling for about `seconds` before timing."""
    import torch

    t_end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < t_end:
        for _ in range(32):
            fn(i)
            i += 1
        torch.cuda.synchronize()


def b2b_us(fn, n, reps=5):
    """Device time per call (us) of n calls issued back to back, HIP events on the launch stream around all
    n; the median over `reps` such runs (single runs of a long kernel varied by up to 15% on MI355X)."""
    import torch

    res = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        for i in range(n):
            fn(i)
        b.record()
        torch.cuda.synchronize()
        res.append(a.elapsed_time(b) * 1e3 / n)
    return float(np.median(res))


def event_us(fn, n):
    """Per-call times (us) from HIP events recorded on the launch stream around each call."""
    import torch

    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for i, (a, b) in enumerate(evs):
        a.record()
        fn(i)
        b.record()
    torch.cuda.synchronize()
    return np.array([a.elapsed_time(b) for a, b in evs]) * 1e3


def aux_c3(dev):
    """c3: ragged unified step, prefill rows on the MFMA prefill kernel and single-token rows on split-K."""
    from easymlx_amd.workloads import config

    wl = config("c3")
    st = Setup(wl, 1.0, dev)
    warm(st.call, 0.5)
    us = float(np.median(event_us(st.call, 100)))
    b2b = b2b_us(st.call, 100)
    qlens = np.diff(wl.query_start_loc)
    pre = qlens > 1
    visible = 0  # keys seen by the prefill rows (causal: row j of a chunk after p cached tokens sees p + j + 1)
    for p, n in zip(wl.kv_lens[pre] - qlens[pre], qlens[pre]):
        visible += int(n * p + n * (n + 1) // 2)
    flops = 4 * wl.head_dim * wl.num_q_heads * visible
    nbytes = wl.kv_bytes()
    return {
        "workload": "c3: 4 prefill chunks x 512 (prior U[0,2048]) + 28 decode rows (ctx U[256,4096]), 4-bit, "
                    "Hq 32 / Hkv 8, D 128, page 128, group 64 (seed 3)",
        "us_p50": round(us, 2),
        "us_back_to_back": round(b2b, 2),
        "prefill_gflop": round(flops / 1e9, 3),
        "kv_bytes": int(nbytes),
        "prefill_tflops": round(flops / (b2b * 1e-6) / 1e12, 1),
        "kv_GBs": round(nbytes / (b2b * 1e3), 1),
        "timing": "us_p50: events around each call (launch gap included); rates: back to back",
    }


def aux_c4(dev):
    """c4: long-context decode, 8 sequences x 32768 tokens, Hq 64 / Hkv 8 (KV bytes exceed the 256 MB cache)."""
    from easymlx_amd.workloads import config

    wl = config("c4")
    st = Setup(wl, 0.0, dev, min_pools=2)
    warm(st.call, 0.5)
    us = float(np.median(event_us(st.call, 100)))
    b2b = b2b_us(st.call, 100)
    nbytes = wl.kv_bytes()
    probe = {}
    for words in (256, 512, 1024):
        st.set_probe_grid(words)
        probe[words] = b2b_us(st.probe, 100)
    pus = min(probe.values())
    return {"workload": "c4: 8 seqs x 32768 tokens, 4-bit, Hq 64 / Hkv 8, D 128, page 128, group 64 (seed 4)",
            "measured_read_peak": {"us": round(pus, 2), "GBs": round(st.probe_bytes / (pus * 1e3), 1),
                                   "frac_of_it": round(pus / b2b, 4)},
            "us_p50": round(us, 2), "us_back_to_back": round(b2b, 2), "kv_bytes": int(nbytes),
            "kv_GBs": round(nbytes / (b2b * 1e3), 1), "frac": round(nbytes / (b2b * 1e3) / HBM_PEAK_GBS, 4),
            "timing": "us_p50: events around each call (launch gap included); kv_GBs and frac: back to back"}


def aux_shapes(dev):
    """The c2 batch (seed 2 lengths, 4-bit, group 64) at other page sizes and head sizes: page 16 (the
    reference's PageCacheConfig default), 32 and 64, and head_dim 64 and 256, each over its own rotated pools."""
    from easymlx_amd.workloads import decode_workload

    res = {}
    for name, kw in (("page16", dict(block_size=16)), ("page32", dict(block_size=32)),
                     ("page64", dict(block_size=64)), ("d64", dict(head_dim=64)), ("d256", dict(head_dim=256))):
        wl = decode_workload(name, seed=2, bits=4, **kw)
        st = Setup(wl, 1.0, dev)
        warm(st.call, 0.3)
        us = b2b_us(st.call, 100)
        nbytes = wl.kv_bytes()
        res[name] = {"block_size": wl.block_size, "head_dim": wl.head_dim, "us_back_to_back": round(us, 2),
                     "kv_bytes": int(nbytes), "kv_GBs": round(nbytes / (us * 1e3), 1),
                     "frac": round(nbytes / (us * 1e3) / HBM_PEAK_GBS, 4)}
        del st
        import torch

        torch.cuda.empty_cache()
    res["workload"] = "c2 batch (32 seqs, ctx U[512,4096], seed 2), 4-bit group 64, Hq 32 / Hkv 8; back to back"
    return res


def aux_fp8(dev):
    """FP8 (E4M3, per-page scale) cache: c2-shaped decode (batch 32, ctx U[512,4096]) and a 32-token write.

    The decode rotates over copies of the page pool (>= 1 GiB in all) so the 256 MB Infinity Cache cannot serve
    the pages; HIP events per call.
    """
    import torch

    from easymlx_amd import Fp8PageCacheView, _native, paged_attention
    from easymlx_amd.workloads import decode_workload

    wl = decode_workload(seed=2, bits=None)
    nb = wl.num_blocks
    shape = (nb, wl.block_size, wl.num_kv_heads, wl.head_dim)
    view = Fp8PageCacheView(key_cache=torch.zeros(shape, dtype=torch.uint8, device=dev),
                            value_cache=torch.zeros(shape, dtype=torch.uint8, device=dev),
                            k_scales=torch.zeros(nb, device=dev), v_scales=torch.zeros(nb, device=dev),
                            block_tables=torch.from_numpy(wl.block_tables).to(dev),
                            kv_lens=torch.from_numpy(wl.kv_lens).to(dev), block_size=wl.block_size,
                            num_kv_heads=wl.num_kv_heads, head_dim=wl.head_dim)
    view.write_slots(torch.from_numpy(wl.k).to(dev), torch.from_numpy(wl.v).to(dev),
                     torch.from_numpy(wl.slot.astype(np.int32)).to(dev))
    q = torch.from_numpy(wl.q).to(dev)
    qsl = torch.from_numpy(wl.query_start_loc).to(dev)
    out = torch.empty_like(q)
    pool_bytes = 2 * view.key_cache.numel()
    pools = [(view.key_cache, view.value_cache, view.k_scales, view.v_scales)]
    while len(pools) * pool_bytes < 2**30:
        pools.append(tuple(t.clone() for t in pools[0]))

    def call(i=0):
        kc, vc, ks, vs = pools[i % len(pools)]
        paged_attention(q, kc, vc, view.block_tables, view.kv_lens, qsl, k_scale=ks, v_scale=vs,
                        single_token_decode=True, out=out)

    warm(call, 0.3)
    us = float(np.median(event_us(call, 100)))
    b2b = b2b_us(call, 100)
    # measured read peak: the FP8 page-read probe over the same pools (the rows the decode reads, loads only)
    lib = _native.load()
    sink = torch.zeros(2048, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    mb = int(wl.block_tables.shape[1])

    def probe_call(i=0, words=1024):
        kc, vc, ks, vs = pools[i % len(pools)]
        _native.check(lib.emx_probe_page_read_fp8(
            kc.data_ptr(), vc.data_ptr(), ks.data_ptr(), vs.data_ptr(), nb, wl.block_size, wl.num_kv_heads,
            wl.head_dim, view.block_tables.data_ptr(), wl.num_seqs, mb, view.kv_lens.data_ptr(), sink.data_ptr(),
            words, stream))

    probe = {}
    for words in (256, 512, 1024, 2048):
        warm(lambda i=0: probe_call(i, words), 0.1)
        probe[words] = b2b_us(lambda i=0: probe_call(i, words), 100)
    pus = min(probe.values())
    lens = np.maximum(wl.kv_lens.astype(np.int64), 0)
    probe_bytes = int(((lens + 31) // 32).sum()) * wl.num_kv_heads * (2 * 32 * wl.head_dim + 8)
    n_fp8_pools = len(pools)
    del pools
    nbytes = int(wl.kv_lens.astype(np.int64).sum()) * wl.num_kv_heads * 2 * wl.head_dim
    kk = torch.randn(wl.num_seqs, wl.num_kv_heads, wl.head_dim, device=dev).half()
    slot = torch.from_numpy((wl.block_tables[:, 0] * wl.block_size).astype(np.int32)).to(dev)
    w = lambda i=0: view.write_slots(kk, kk, slot)  # noqa: E731
    warm(w, 0.2)
    wus = float(np.median(event_us(w, 100)))
    # the c3-shaped unified step (4 x 512 prefill rows + 28 decode rows) over an FP8 cache
    from easymlx_amd.workloads import unified_workload

    uw = unified_workload("c3", bits=None)
    ushape = (uw.num_blocks, uw.block_size, uw.num_kv_heads, uw.head_dim)
    uv = Fp8PageCacheView(key_cache=torch.zeros(ushape, dtype=torch.uint8, device=dev),
                          value_cache=torch.zeros(ushape, dtype=torch.uint8, device=dev),
                          k_scales=torch.zeros(uw.num_blocks, device=dev), v_scales=torch.zeros(uw.num_blocks, device=dev),
                          block_tables=torch.from_numpy(uw.block_tables).to(dev),
                          kv_lens=torch.from_numpy(uw.kv_lens).to(dev), block_size=uw.block_size,
                          num_kv_heads=uw.num_kv_heads, head_dim=uw.head_dim)
    uv.write_slots(torch.from_numpy(uw.k).to(dev), torch.from_numpy(uw.v).to(dev),
                   torch.from_numpy(uw.slot.astype(np.int32)).to(dev))
    uq = torch.from_numpy(uw.q).to(dev)
    uqsl = torch.from_numpy(uw.query_start_loc).to(dev)
    uout = torch.empty_like(uq)

    def ucall(i=0):
        paged_attention(uq, uv.key_cache, uv.value_cache, uv.block_tables, uv.kv_lens, uqsl, k_scale=uv.k_scales,
                        v_scale=uv.v_scales, out=uout)

    warm(ucall, 0.3)
    uus = float(np.median(event_us(ucall, 50)))
    return {"workload": "fp8 e4m3 cache, c2 shape: batch 32, Hq 32 / Hkv 8, D 128, page 128, ctx U[512,4096] (seed 2)",
            "rotated_pools": n_fp8_pools, "pool_bytes": int(pool_bytes),
            "unified_c3_shape_us_p50": round(uus, 2),
            "decode_us_p50": round(us, 2), "decode_us_back_to_back": round(b2b, 2), "kv_bytes": nbytes,
            "measured_read_peak": {"us": round(pus, 2), "GBs": round(probe_bytes / (pus * 1e3), 1),
                                   "frac_of_it": round(pus / b2b, 4)},
            "kv_GBs": round(nbytes / (b2b * 1e3), 1), "frac": round(nbytes / (b2b * 1e3) / HBM_PEAK_GBS, 4),
            "write_32_tokens_us_p50": round(wus, 2),
            "timing": "*_us_p50: events around each call (launch gap included); kv_GBs and frac: back to back"}


def aux_quantize_on_write(dev):
    """Fused quantize-on-write (4-bit, group 64): one appended token per c2 sequence; 4 x 512-token chunks."""
    import torch

    from easymlx_amd import _native
    from easymlx_amd.caching import affine_pool
    from easymlx_amd.workloads import config

    wl = config("c2")
    bs, hkv, d = wl.block_size, wl.num_kv_heads, wl.head_dim
    nb = wl.num_blocks + 16
    view = affine_pool(num_blocks=nb, num_kv_heads=hkv, head_dim=d, block_size=bs, bits=4, group_size=64,
                       block_tables=torch.from_numpy(wl.block_tables).to(dev),
                       kv_lens=torch.from_numpy(wl.kv_lens).to(dev))
    fn = _native.load().emx_affine_cache_write
    stream = torch.cuda.current_stream(dev).cuda_stream
    width = wl.block_tables.shape[1]
    appends = [int(wl.block_tables[s, min(int(wl.kv_lens[s]) // bs, width - 1)]) * bs + int(wl.kv_lens[s]) % bs
               for s in range(wl.num_seqs)]
    chunks = [(wl.num_blocks + 4 * c) * bs + i for c in range(4) for i in range(512)]
    res = {}
    for name, slots in (("append_1_token_x32_seqs", appends), ("prefill_4x512_tokens", chunks)):
        n = len(slots)
        k = torch.randn(n, hkv, d, device=dev).half()
        v = torch.randn(n, hkv, d, device=dev).half()
        s = torch.tensor(slots, dtype=torch.int32, device=dev)
        args = (k.data_ptr(), v.data_ptr(), s.data_ptr(), n, hkv, d, 64, 4, bs, nb, view.k_codes.data_ptr(),
                view.k_scales.data_ptr(), view.k_biases.data_ptr(), view.v_codes.data_ptr(),
                view.v_scales.data_ptr(), view.v_biases.data_ptr(), stream)

        def call(i, args=args):
            rc = fn(*args)
            if rc:
                _native.check(rc)

        warm(call, 0.3)
        us = float(np.median(event_us(call, 200)))
        moved = n * hkv * (2 * d * 2 + 2 * (d // 2 + 4 * (d // 64)))  # fp16 K,V in; codes + scale/bias out
        res[name] = {"tokens": n, "us_p50": round(us, 2), "GBs_in_plus_out": round(moved / (us * 1e3), 1)}
    # a decode step's append with Llama-3 RoPE fused in: K rotated inside the write, Q (32 heads) by the same launch
    from easymlx_amd import RotaryEmbedding

    lib = _native.load()
    rope = RotaryEmbedding.llama3(d, base=500000.0)
    inv = rope.inv_freq(dev)
    n = len(appends)
    k = torch.randn(n, hkv, d, device=dev).half()
    v = torch.randn(n, hkv, d, device=dev).half()
    q = torch.randn(n, 32, d, device=dev).half()
    q_out = torch.empty_like(q)  # the turned queries (the inputs stay as they are)
    s = torch.tensor(appends, dtype=torch.int32, device=dev)
    pos = torch.from_numpy(wl.kv_lens.astype(np.int32)).to(dev)

    def call_rope(i):
        rc = lib.emx_affine_cache_write_rope(
            k.data_ptr(), v.data_ptr(), s.data_ptr(), n, hkv, d, 64, 4, bs, nb, view.k_codes.data_ptr(),
            view.k_scales.data_ptr(), view.k_biases.data_ptr(), view.v_codes.data_ptr(), view.v_scales.data_ptr(),
            view.v_biases.data_ptr(), pos.data_ptr(), inv.data_ptr(), d, 0, q.data_ptr(), q_out.data_ptr(), 32, stream)
        if rc:
            _native.check(rc)

    warm(call_rope, 0.3)
    res["append_1_token_x32_seqs_rope_q_and_k"] = {"tokens": n,
                                                   "us_p50": round(float(np.median(event_us(call_rope, 200))), 2)}
    # the reference's logical layout at the op: the c2 decode given codes [nb, bs, Hkv, W] and scales
    # [nb, bs, Hkv, G] converts the whole pool to pages for the call
    from easymlx_amd import paged_attention
    from easymlx_amd.caching.paged import pages_from_logical

    view.write_slots(torch.from_numpy(wl.k).to(dev), torch.from_numpy(wl.v).to(dev),
                     torch.from_numpy(wl.slot.astype(np.int32)).to(dev))
    lg = view.to_logical()
    qd = torch.from_numpy(wl.q).to(dev)
    qsl = torch.from_numpy(wl.query_start_loc).to(dev)
    pages = pages_from_logical(lg["k_codes"], lg["k_scales"], lg["k_biases"], lg["v_codes"], lg["v_scales"],
                               lg["v_biases"], 4, 64)

    def convert(i):
        pages_from_logical(lg["k_codes"], lg["k_scales"], lg["k_biases"], lg["v_codes"], lg["v_scales"],
                           lg["v_biases"], 4, 64, out=pages)

    def decode_pages(i):
        paged_attention(qd, view.k_codes, view.v_codes, view.block_tables, view.kv_lens, qsl, k_scales=view.k_scales,
                        k_biases=view.k_biases, v_scales=view.v_scales, v_biases=view.v_biases, bits=4, group_size=64,
                        single_token_decode=True)

    def decode_logical(i):
        paged_attention(qd, lg["k_codes"], lg["v_codes"], view.block_tables, view.kv_lens, qsl,
                        k_scales=lg["k_scales"], k_biases=lg["k_biases"], v_scales=lg["v_scales"],
                        v_biases=lg["v_biases"], bits=4, group_size=64, single_token_decode=True)

    lay = {"pool_bytes": int(sum(t.numel() * t.element_size() for t in pages))}
    for name, fn_ in (("convert_pool", convert), ("decode_on_pages", decode_pages),
                      ("decode_from_logical_layout", decode_logical)):
        warm(fn_, 0.3)
        lay[name + "_us_p50"] = round(float(np.median(event_us(fn_, 50))), 2)
    lay["what"] = ("the c2 batch through paged_attention given the reference's logical affine layout: the op "
                   "converts the whole pool to pages for the call (a caller that keeps the cache converts it once, "
                   "AffinePageCacheView.from_logical); one pool, so the decode is partly served by the Infinity "
                   "Cache here")
    res["logical_layout_at_the_op"] = lay
    return res


def aux_op_layer_step(dev, steps=100, layers=32):
    """The public op as a runner calls it, per layer-step of c2: ``concatenate_to_cache`` (quantize-on-write of
    one token per sequence, Llama-3 RoPE fused) then ``UnifiedAttention.forward_native``, over ``layers``
    layers with a cache each (one decode step).  Wall clock per layer-step: eager Python calls, and the decode
    step captured once in a HIP graph through ``CompiledPagedCacheProxy`` (the counterpart of the reference's
    compiled decode, which compiles the whole model step) and replayed."""
    import torch

    from easymlx_amd import CompiledPagedCacheProxy, Fp8PageCacheView, PageMetadata, RotaryEmbedding, UnifiedAttention
    from easymlx_amd.caching import affine_pool
    from easymlx_amd.workloads import config

    wl = config("c2")
    S, hq, hkv, d, bs = wl.num_seqs, wl.num_q_heads, wl.num_kv_heads, wl.head_dim, wl.block_size
    extra = 2  # fresh pages per sequence for the appended tokens
    tables = np.full((S, wl.block_tables.shape[1] + extra), -1, np.int32)
    for s in range(S):
        used = -(-int(wl.kv_lens[s]) // bs)
        tables[s, :used] = wl.block_tables[s, :used]
        tables[s, used:used + extra] = wl.num_blocks + extra * s + np.arange(extra)
    rope = RotaryEmbedding.llama3(d, base=500000.0)
    op = UnifiedAttention()
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn((S, hq, d), device=dev, generator=g).half()
    k = torch.randn((S, hkv, d), device=dev, generator=g).half()
    v = torch.randn((S, hkv, d), device=dev, generator=g).half()
    res = {"layers_per_step": layers}
    for mode in ("eager", "graph", "fp8_eager", "fp8_graph"):
        nbp = wl.num_blocks + extra * S

        def make_view():
            if mode.startswith("fp8"):  # the reference's FP8 cache on the same pages
                shape = (nbp, bs, hkv, d)
                view = Fp8PageCacheView(key_cache=torch.zeros(shape, dtype=torch.uint8, device=dev),
                                        value_cache=torch.zeros(shape, dtype=torch.uint8, device=dev),
                                        k_scales=torch.zeros(nbp, device=dev), v_scales=torch.zeros(nbp, device=dev),
                                        block_tables=torch.from_numpy(tables).to(dev),
                                        kv_lens=torch.from_numpy(wl.kv_lens).to(dev), block_size=bs,
                                        num_kv_heads=hkv, head_dim=d)
            else:
                view = affine_pool(num_blocks=nbp, num_kv_heads=hkv, head_dim=d, block_size=bs, bits=4,
                                   group_size=64, block_tables=torch.from_numpy(tables).to(dev),
                                   kv_lens=torch.from_numpy(wl.kv_lens).to(dev))
            view.write_slots(torch.from_numpy(wl.k).to(dev), torch.from_numpy(wl.v).to(dev),
                             torch.from_numpy(wl.slot.astype(np.int32)).to(dev))
            return view

        views = [make_view() for _ in range(layers)]
        md0 = PageMetadata(query_start_loc=torch.arange(S + 1, dtype=torch.int32, device=dev),
                           slot_ids=tuple(range(S)))
        qlens = (1,) * S
        caches = [CompiledPagedCacheProxy(w) if mode.endswith("graph") else w for w in views]
        outs = []

        def step():
            x = q
            for cache, view in zip(caches, views):
                q2, kc, vc, md = cache.concatenate_to_cache(x, k, v, cache_metadata=md0, rope=rope, query_lens=qlens)
                x = op.forward_native(query=q2, key=kc, value=vc, cache_metadata=md, cache_view=view).attention_outputs
            outs[:] = [x]

        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            step()
            if mode.endswith("graph"):
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=side):
                    step()
                run = graph.replay
            else:
                run = step
            # warm up as long as the timed run: the first time the host runs far ahead of
            # the GPU (no synchronizing call in the step) costs ~40 ms once
            for _ in range(steps):
                run()
            side.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                run()
            side.synchronize()
            res[f"{mode}_us_per_layer_step"] = round((time.perf_counter() - t0) / (steps * layers) * 1e6, 2)
        del views, caches
    res["workload"] = (f"c2 decode step through the public op over {layers} layers (a cache each): per layer "
                       "concatenate_to_cache (1 token x 32 seqs, Llama-3 RoPE fused) + "
                       "UnifiedAttention.forward_native (its output is the next layer's query); wall clock per "
                       "layer-step; graph: the whole step in one HIP graph, replayed; fp8_*: the same over an "
                       "FP8 (E4M3, per-page scale) cache")
    return res

def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; multi-GPU runs are out of scope"}))
        sys.exit(2)

    import torch

    from easymlx_amd.workloads import config

    dev = torch.device("cuda", 0)
    if args.aux_only:
        fn = {"c3": aux_c3, "c4": aux_c4, "write": aux_quantize_on_write, "op": aux_op_layer_step,
              "fp8": aux_fp8, "shapes": aux_shapes}[args.aux_only]
        print(json.dumps({args.aux_only: fn(dev)}))
        return
    wl = config("c2")
    bytes_per_step = wl.kv_bytes()
    st = Setup(wl, args.pool_gib, dev)
    layers = max(1, args.layers)
    step_call = lambda i: st.step_call(i, layers)  # noqa: E731
    for i in range(args.warmup):
        step_call(i)
    warm(step_call, 1.0)

    # ---- timed region: exactly `steps` decode calls (layer calls of consecutive model steps: kv_lens
    # change at every step's first layer), bracketed by HIP events on the launch stream
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    for i in range(args.steps):
        step_call(i)
    ev1.record()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    n_alt = sum(1 for i in range(args.steps) if (i // layers) % 2 == 1)
    bytes_per_step = ((args.steps - n_alt) * wl.kv_bytes() + n_alt * st.bytes_b) / args.steps
    ms_per_step = elapsed / args.steps * 1e3
    call_us = ev0.elapsed_time(ev1) * 1e3 / args.steps  # device time per call, back to back
    achieved = bytes_per_step / (call_us * 1e-6) / 1e9
    # the two kinds of call apart: kv_lens as the previous call's (cached plan) / new every call
    us_cached = b2b_us(st.call, 200)
    us_new = b2b_us(lambda i: st.call(i, alt=i % 2 == 1), 200)

    # ---- per-call times with events around each call (includes each launch's dispatch gap)
    kt = event_us(step_call, min(args.steps, 200))
    k_avg_us = float(kt.mean())

    # ---- measured read-stream peak: the page-read probe over the same rotated pools (same page slices,
    # loads only), back to back
    warm(st.probe, 0.3)
    probe_grid = {}
    for words in (256, 512, 1024, 2048):  # workgroups; the best is the peak
        st.set_probe_grid(words)
        probe_grid[words] = round(b2b_us(st.probe, 200), 3)
    probe_wgs = min(probe_grid, key=probe_grid.get)
    probe_us = probe_grid[probe_wgs]
    probe_bytes = st.probe_bytes
    probe_gbs = probe_bytes / (probe_us * 1e-6) / 1e9

    if args.copy_probe_mib:
        n = args.copy_probe_mib << 20
        src = torch.ones(n // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    n_pools, pool_bytes = st.n_pools, st.pool_bytes
    del st
    aux = None
    if not args.no_aux:
        torch.cuda.empty_cache()
        aux = {"c3_unified": aux_c3(dev)}
        torch.cuda.empty_cache()
        aux["c4_long_context"] = aux_c4(dev)
        torch.cuda.empty_cache()
        aux["quantize_on_write"] = aux_quantize_on_write(dev)
        aux["op_layer_step"] = aux_op_layer_step(dev)
        aux["fp8_cache"] = aux_fp8(dev)
        torch.cuda.empty_cache()
        aux["other_shapes"] = aux_shapes(dev)

    value = bytes_per_step / (ms_per_step * 1e-3) / 1e9
    traffic, traffic_src = measured_traffic()
    cpu = None if args.no_cpu_baseline else cpu_baseline(wl, args.cpu_seqs or None)
    line = {
        "metric": "4-bit-KV paged decode: achieved HBM GB/s (% of peak) + tokens/s, batch 32",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 codes, fp16 scale/bias, fp32 accumulate",
        "data": "synthetic (seeded N(0,1) x per-channel gains U[0.5,4], quantized on the GPU)",
        "config": {
            "workload": "c2: 4-bit affine paged decode, batch 32, Hq 32 / Hkv 8, D 128, page 128, group 64, "
                        "ctx U[512,4096] (seed 2)",
            "global_batch": wl.num_seqs,
            "context_tokens": int(wl.kv_lens.sum()),
            "kv_bytes_per_step": int(bytes_per_step),
            "rotated_pools": n_pools,
            "pool_bytes": int(pool_bytes),
        },
        "tokens_per_s_per_layer": round(wl.num_seqs / (ms_per_step * 1e-3), 1),
        "tokens_per_s_attention_32_layers": round(wl.num_seqs / (ms_per_step * 1e-3 * 32), 1),
        "us_per_layer_step": round(ms_per_step * 1e3, 3),
        "call_us_back_to_back": round(call_us, 3),
        "plan_cache": {"layers_per_step": layers, "us_same_kv_lens": round(us_cached, 3),
                       "us_new_kv_lens_every_call": round(us_new, 3),
                       "what": "the decode keeps its work split in the workspace, keyed by the per-sequence "
                               "counts of 256-token items: the other layers of a step reuse it, and so does "
                               "the next step unless a sequence crosses an item boundary; the timed calls "
                               "alternate kv_lens one decode step apart (every sequence one token longer) every "
                               "`layers_per_step` calls, and every call for us_new_kv_lens_every_call"},
        "kernel_us": {"mean": round(k_avg_us, 3), "p10": round(float(np.percentile(kt, 10)), 3),
                      "p50": round(float(np.percentile(kt, 50)), 3), "p90": round(float(np.percentile(kt, 90)), 3)},
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "measured_read_peak": {"GBs": round(probe_gbs, 1), "us": round(probe_us, 3), "bytes": probe_bytes,
                                   "frac_of_it": round(achieved / probe_gbs, 4),
                                   "us_by_workgroups": probe_grid,
                                   "what": "emx_probe_page_read: loads of exactly the page slices the call reads "
                                           "(64-token slices with a live token), nothing else, back to back over "
                                           "the same rotated pools"},
            "kernel": "emx::decode_q4_d128<64,4> (one launch per decode call; split-K merge fused)",
        },
        "cpu_baseline": cpu,
        "aux": aux,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
