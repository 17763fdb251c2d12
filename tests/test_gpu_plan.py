"""The 4-bit decode's plan cache in the workspace.

A pure decode call on the 4-bit kernel keeps its workgroup ranges and first
items in the workspace; the next call with the same kv_lens and shape reuses
them.  The cached path must give the bits the computing path gives: the ranges
are the same function of kv_lens, so the kernel does the same arithmetic in the
same order.  Cases: a repeat (the second call runs on the cached plan), changed
kv_lens, changed block tables under the same kv_lens (the cached first pages
are stale), and shapes interleaved on one workspace.
"""

import numpy as np
import pytest
import torch

from easymlx_amd import _native, paged_attention
from easymlx_amd.workloads import decode_workload
from tests.helpers import assert_attention_close, gpu_cache, oracle_expected

pytestmark = pytest.mark.gpu


def _workspace(wl, cuda):
    lib = _native.load()
    need = lib.emx_paged_workspace_bytes(wl.num_seqs, wl.num_q_heads, wl.num_kv_heads, wl.head_dim,
                                         wl.block_tables.shape[1], wl.block_size)
    assert need > 0
    return torch.zeros(need, dtype=torch.uint8, device=cuda)


def _call(wl, view, cuda, ws, kv_lens=None, block_tables=None, window=None):
    q = torch.from_numpy(wl.q).to(cuda)
    out = paged_attention(
        q, view.k_codes, view.v_codes, view.block_tables if block_tables is None else block_tables,
        view.kv_lens if kv_lens is None else kv_lens, torch.from_numpy(wl.query_start_loc).to(cuda),
        k_scales=view.k_scales, k_biases=view.k_biases, v_scales=view.v_scales, v_biases=view.v_biases,
        bits=wl.bits, group_size=wl.group_size, single_token_decode=True, sliding_window=window, workspace=ws)
    torch.cuda.synchronize()
    return out.clone()


def _wl(seed, seqs, hq=32, hkv=8, ctx=(512, 4096), gs=64):
    return decode_workload(seed=seed, num_seqs=seqs, num_q_heads=hq, num_kv_heads=hkv, ctx_range=ctx, bits=4,
                           group_size=gs)


def test_plan_repeat_bit_identical(cuda):
    print("[plan repeat]", flush=True)
    wl = _wl(31, 24)
    view = gpu_cache(wl, cuda)
    ws = _workspace(wl, cuda)
    first = _call(wl, view, cuda, ws)   # computes its ranges, commits a plan
    second = _call(wl, view, cuda, ws)  # runs on the committed plan
    third = _call(wl, view, cuda, ws)
    fresh = _call(wl, view, cuda, _workspace(wl, cuda))
    assert torch.equal(first, second) and torch.equal(second, third) and torch.equal(first, fresh)
    assert_attention_close(second.float().cpu().numpy(), oracle_expected(wl), "plan repeat")


def test_plan_kv_lens_change(cuda):
    print("[plan kv_lens change]", flush=True)
    wl = _wl(32, 20)
    view = gpu_cache(wl, cuda)
    ws = _workspace(wl, cuda)
    _call(wl, view, cuda, ws)
    _call(wl, view, cuda, ws)
    rng = np.random.default_rng(5)
    for trial in range(3):
        lens = np.maximum(wl.kv_lens - rng.integers(0, 700, wl.num_seqs), 1).astype(np.int32)
        if trial == 2:
            lens[3] = 0  # a sequence without tokens
        kl = torch.from_numpy(lens).to(cuda)
        got = _call(wl, view, cuda, ws, kv_lens=kl)
        again = _call(wl, view, cuda, ws, kv_lens=kl)
        fresh = _call(wl, view, cuda, _workspace(wl, cuda), kv_lens=kl)
        assert torch.equal(got, fresh) and torch.equal(again, fresh), f"trial {trial}"
        assert_attention_close(got.float().cpu().numpy(), oracle_expected(wl, kv_lens=lens), f"kv_lens {trial}")


def test_plan_block_tables_change(cuda):
    """Same kv_lens, pages moved: the cached first pages are stale and must be reloaded."""
    print("[plan block tables change]", flush=True)
    wl = _wl(33, 16)
    view = gpu_cache(wl, cuda)
    rng = np.random.default_rng(9)
    perm = rng.permutation(wl.num_blocks).astype(np.int32)
    moved = decode_workload(seed=33, num_seqs=16, num_q_heads=32, num_kv_heads=8, ctx_range=(512, 4096), bits=4,
                            group_size=64)
    tables = np.where(wl.block_tables >= 0, perm[np.maximum(wl.block_tables, 0)], -1).astype(np.int32)
    moved.block_tables = tables
    moved.slot = (perm[wl.slot // wl.block_size].astype(np.int64) * wl.block_size + wl.slot % wl.block_size)
    view2 = gpu_cache(moved, cuda)
    ws = _workspace(wl, cuda)
    a = _call(wl, view, cuda, ws)
    b = _call(wl, view, cuda, ws)
    c = _call(moved, view2, cuda, ws)  # cached ranges hold, cached pages do not
    d = _call(wl, view, cuda, ws)
    assert torch.equal(a, b) and torch.equal(a, c) and torch.equal(a, d)


def test_plan_shapes_interleaved(cuda):
    print("[plan shapes interleaved]", flush=True)
    cases = [_wl(34, 12), _wl(35, 5, hq=16, hkv=8, ctx=(1, 900)), _wl(36, 40, ctx=(64, 700)),
             _wl(37, 7, hq=64, hkv=4, gs=128, ctx=(100, 3000))]
    views = [gpu_cache(w, cuda) for w in cases]
    size = max(_workspace(w, cuda).numel() for w in cases)
    ws = torch.zeros(size, dtype=torch.uint8, device=cuda)
    fresh = [_call(w, v, cuda, torch.zeros(size, dtype=torch.uint8, device=cuda)) for w, v in zip(cases, views)]
    for rnd in range(3):
        for i, (w, v) in enumerate(zip(cases, views)):
            got = _call(w, v, cuda, ws)
            assert torch.equal(got, fresh[i]), f"round {rnd} case {i}"
            got = _call(w, v, cuda, ws)
            assert torch.equal(got, fresh[i]), f"round {rnd} case {i} repeat"
    # a sliding window changes the ranges: cached plans of the unwindowed call must not be used
    w, v = cases[0], views[0]
    win = _call(w, v, cuda, ws, window=300)
    win_fresh = _call(w, v, cuda, torch.zeros(size, dtype=torch.uint8, device=cuda), window=300)
    assert torch.equal(win, win_fresh)
    assert_attention_close(win.float().cpu().numpy(), oracle_expected(w, sliding_window=300), "window")


def test_plan_kept_across_token_growth(cuda):
    """kv_lens that grow by a token per call keep their item counts (the plan holds) until a
    sequence crosses an item boundary; the token masks and, under a sliding window, the first
    items follow this call's kv_lens, not the plan's."""
    print("[plan token growth]", flush=True)
    wl = _wl(38, 24, ctx=(1400, 3000))
    view = gpu_cache(wl, cuda)
    ws = _workspace(wl, cuda)
    base = (np.maximum(wl.kv_lens - 12, 1)).astype(np.int32)
    base[0] = 256 * 3 - 2  # crosses an item boundary within the calls below
    base[1] = 256 * 5
    for window in (None, 300, 512):
        for step in range(6):
            lens = (base + step).astype(np.int32)
            kl = torch.from_numpy(lens).to(cuda)
            got = _call(wl, view, cuda, ws, kv_lens=kl, window=window)
            fresh = _call(wl, view, cuda, _workspace(wl, cuda), kv_lens=kl, window=window)
            assert torch.equal(got, fresh), f"window {window} step {step}"
            if step in (0, 3, 5):
                assert_attention_close(got.float().cpu().numpy(), oracle_expected(wl, kv_lens=lens,
                                                                                   sliding_window=window or 0),
                                       f"window {window} step {step}")


def test_plan_one_sequence_changes(cuda):
    """A change of one sequence's item count, at any position of the batch, invalidates the plan
    (every lane of every wave votes on the mismatch)."""
    print("[plan one sequence]", flush=True)
    wl = _wl(39, 150, ctx=(300, 1500))
    view = gpu_cache(wl, cuda)
    ws = _workspace(wl, cuda)
    _call(wl, view, cuda, ws)
    for si in (1, 37, 63, 64, 100, 149):
        lens = wl.kv_lens.copy()
        lens[si] = max(1, int(lens[si]) - 256)  # one item fewer
        kl = torch.from_numpy(lens.astype(np.int32)).to(cuda)
        got = _call(wl, view, cuda, ws, kv_lens=kl)
        fresh = _call(wl, view, cuda, _workspace(wl, cuda), kv_lens=kl)
        assert torch.equal(got, fresh), f"sequence {si}"
        back = _call(wl, view, cuda, ws)
        assert torch.equal(back, _call(wl, view, cuda, _workspace(wl, cuda))), f"sequence {si} back"
