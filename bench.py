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


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=400)
    p.add_argument("--warmup", type=int, default=40)
    p.add_argument("--pool-gib", type=float, default=1.5, help="total size of the rotated page pools")
    p.add_argument("--no-cpu-baseline", action="store_true")
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
        "kind": "port",
        "sample": f"C oracle (oracle/c/oracle.c, OpenMP over (seq, kv_head)) on {n} of {wl.num_seqs} sequences of the "
                  f"same workload ({ntok} tokens), {reps} reps, {per * 1e3:.1f} ms each = {n / per:.1f} decode rows/s",
    }


def measured_traffic():
    """HBM bytes per decode call from the committed counter summary (two rocprofv3 --pmc passes)."""
    path = os.path.join(ROOT, "profiles", "decode_affine_c2_hbm_traffic.md")
    try:
        for line in open(path):
            if line.startswith("TRAFFIC_BYTES_PER_CALL:"):
                return int(line.split(":")[1]), os.path.relpath(path, ROOT)
    except OSError:
        pass
    return None, None


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; multi-GPU runs are out of scope"}))
        sys.exit(2)

    import torch

    from easymlx_amd import _native, paged_attention
    from easymlx_amd.caching import affine_pool
    from easymlx_amd.workloads import config

    dev = torch.device("cuda", 0)
    wl = config("c2")
    bytes_per_step = wl.kv_bytes()

    base = affine_pool(num_blocks=wl.num_blocks, num_kv_heads=wl.num_kv_heads, head_dim=wl.head_dim,
                       block_size=wl.block_size, bits=wl.bits, group_size=wl.group_size,
                       block_tables=torch.from_numpy(wl.block_tables).to(dev),
                       kv_lens=torch.from_numpy(wl.kv_lens).to(dev))
    base.write_slots(torch.from_numpy(wl.k).to(dev), torch.from_numpy(wl.v).to(dev),
                     torch.from_numpy(wl.slot.astype(np.int32)).to(dev))
    pool_bytes = sum(t.numel() * t.element_size() for t in
                     (base.k_codes, base.v_codes, base.k_scales, base.k_biases, base.v_scales, base.v_biases))
    n_pools = max(4, math.ceil(args.pool_gib * 2**30 / pool_bytes))
    pools = [base] + [
        affine_pool(num_blocks=wl.num_blocks, num_kv_heads=wl.num_kv_heads, head_dim=wl.head_dim,
                    block_size=wl.block_size, bits=wl.bits, group_size=wl.group_size,
                    block_tables=base.block_tables, kv_lens=base.kv_lens)
        for _ in range(n_pools - 1)
    ]
    for p in pools[1:]:
        for dst, src in ((p.k_codes, base.k_codes), (p.v_codes, base.v_codes), (p.k_scales, base.k_scales),
                         (p.k_biases, base.k_biases), (p.v_scales, base.v_scales), (p.v_biases, base.v_biases)):
            dst.copy_(src)
    q = torch.from_numpy(wl.q).to(dev)
    qsl = torch.from_numpy(wl.query_start_loc).to(dev)
    out = torch.empty_like(q)

    def step(i):
        p = pools[i % n_pools]
        paged_attention(q, p.k_codes, p.v_codes, p.block_tables, p.kv_lens, qsl, k_scales=p.k_scales,
                        k_biases=p.k_biases, v_scales=p.v_scales, v_biases=p.v_biases, bits=wl.bits,
                        group_size=wl.group_size, single_token_decode=True, out=out)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all(), "non-finite decode output"
    eager = out.clone()

    # Timed calls go straight through the C ABI (the drop-in boundary) with their argument
    # lists prepared here: the Python wrapper's host cost per call (validation, conversions)
    # exceeds one ~30 us call and would otherwise be what is timed.
    lib = _native.load()
    fn = lib.emx_paged_attention_affine
    S, hq, d = (int(x) for x in q.shape)
    ws = torch.zeros(lib.emx_paged_workspace_bytes(S, hq, wl.num_kv_heads, d, wl.block_tables.shape[1],
                                                   wl.block_size), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    call_args = [
        (q.data_ptr(), S, hq, d, p.k_codes.data_ptr(), p.k_scales.data_ptr(), p.k_biases.data_ptr(),
         p.v_codes.data_ptr(), p.v_scales.data_ptr(), p.v_biases.data_ptr(), wl.num_blocks, wl.block_size,
         wl.num_kv_heads, wl.bits, wl.group_size, p.block_tables.data_ptr(), S, wl.block_tables.shape[1],
         p.kv_lens.data_ptr(), qsl.data_ptr(), 1.0 / math.sqrt(d), 0, 1, ws.data_ptr(), ws.numel(), out.data_ptr(),
         stream)
        for p in pools
    ]

    def call(i):
        rc = fn(*call_args[i % n_pools])
        if rc:
            _native.check(rc)

    for i in range(n_pools):                                      # same result as the public op, every pool
        out.zero_()
        call(i)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), "C-ABI call differs from paged_attention"

    # clocks ramp up under sustained load: keep calling for ~1 s before timing
    t_end = time.perf_counter() + 1.0
    i = 0
    while time.perf_counter() < t_end:
        for _ in range(64):
            call(i)
            i += 1
        torch.cuda.synchronize()

    # ---- timed region: exactly `steps` decode calls
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        call(i)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed / args.steps * 1e3

    # ---- per-call time with HIP events on the launch stream
    n_ev = min(args.steps, 200)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n_ev)]
    for i, (a, b) in enumerate(evs):
        a.record()
        call(i)
        b.record()
    torch.cuda.synchronize()
    kt = np.array([a.elapsed_time(b) for a, b in evs]) * 1e3  # us
    k_avg_us = float(kt.mean())
    achieved = bytes_per_step / (k_avg_us * 1e-6) / 1e9

    if args.copy_probe_mib:
        n = args.copy_probe_mib << 20
        src = torch.ones(n // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

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
            "kernel": "emx::decode_affine_d128<4,64,4> + emx::decode_merge_d128<4> (one decode call)",
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
