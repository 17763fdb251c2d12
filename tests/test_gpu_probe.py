"""Page-read probe (``emx_probe_page_read``, the bench's measured read-stream peak): it must read exactly the
bytes of every 64-token slice of a page-head holding a live token (K codes, V codes, four scale / bias runs) --
the XOR of all 32-bit words it read equals the same XOR taken on the host over those slices, with pages shared
between sequences, invalid page ids, partial last pages and empty sequences in the tables."""

import numpy as np
import pytest
import torch

from easymlx_amd import _native

pytestmark = pytest.mark.gpu


def _host_xor(kc, vc, par, tables, lens, bs, bits):
    nt = 64 if bits == 4 else 32
    nb, hkv = kc.shape[:2]
    x = np.uint32(0)
    for s in range(tables.shape[0]):
        for pg in range(tables.shape[1]):
            for h in range(bs // 64):
                t0 = 64 * h
                b = int(tables[s, pg])
                if pg * bs + t0 >= max(int(lens[s]), 0) or not 0 <= b < nb:
                    continue
                for kvh in range(hkv):
                    words = [kc[b, kvh, t0:t0 + 64].ravel(),
                             vc[b, kvh, t0 // nt:(t0 + 64) // nt].ravel()]
                    words += [p[b, kvh, :, t0:t0 + 64].copy().view(np.uint32).ravel() for p in par]
                    for w in words:
                        x ^= np.bitwise_xor.reduce(w)
    return x


@pytest.mark.parametrize("bits,bs,gs", [(4, 128, 64), (8, 128, 64), (4, 64, 32), (8, 64, 128)])
def test_probe_reads_exactly_the_live_slices(cuda, bits, bs, gs):
    print(f"[probe bits={bits} bs={bs} gs={gs}]", flush=True)
    rng = np.random.default_rng(bits * 7 + bs + gs)
    nb, hkv, d, S, mb = 40, 3, 128, 5, 6
    G, W, nt = d // gs, d * bits // 32, 64 if bits == 4 else 32
    kc = rng.integers(0, 2**32, (nb, hkv, bs, W), dtype=np.uint64).astype(np.uint32)
    vc = rng.integers(0, 2**32, (nb, hkv, bs // nt, d, 8), dtype=np.uint64).astype(np.uint32)
    par = [rng.integers(0, 2**16, (nb, hkv, G, bs), dtype=np.uint64).astype(np.uint16) for _ in range(4)]
    tables = rng.integers(0, nb, (S, mb)).astype(np.int32)
    tables[0, 1] = tables[1, 0]  # a page shared by two sequences
    tables[2, 2] = -1            # an invalid page id inside the live range
    tables[3, 0] = nb + 5
    lens = np.array([mb * bs, 3 * bs + 1, 5 * bs - 64, 0, 70], dtype=np.int32)
    dev = lambda a: torch.from_numpy(a.view(np.int32) if a.dtype == np.uint32 else a.view(np.float16)).to(cuda)  # noqa: E731
    tk, tv, tp = dev(kc), dev(vc), [dev(p) for p in par]
    tt, tl = dev(tables), dev(lens)
    sink = torch.zeros(1024, dtype=torch.int32, device=cuda)
    lib = _native.load()
    rc = lib.emx_probe_page_read(tk.data_ptr(), tp[0].data_ptr(), tp[1].data_ptr(), tv.data_ptr(), tp[2].data_ptr(),
                                 tp[3].data_ptr(), nb, bs, hkv, d, bits, gs, tt.data_ptr(), S, mb, tl.data_ptr(),
                                 sink.data_ptr(), sink.numel(), torch.cuda.current_stream(cuda).cuda_stream)
    _native.check(rc)
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    assert got == _host_xor(kc, vc, par, tables, lens, bs, bits)


def test_probe_rejects_unsupported_geometry(cuda):
    lib = _native.load()
    z = torch.zeros(64, dtype=torch.int32, device=cuda)
    p = z.data_ptr()
    rc = lib.emx_probe_page_read(p, p, p, p, p, p, 1, 32, 1, 128, 4, 64, p, 1, 1, p, p, 1, None)
    assert rc == _native.EMX_ERR_UNSUPPORTED and b"page_size" in lib.emx_last_error()


@pytest.mark.parametrize("bs", [128, 32])
def test_probe_fp8_reads_exactly_the_live_rows(cuda, bs):
    print(f"[probe fp8 bs={bs}]", flush=True)
    rng = np.random.default_rng(100 + bs)
    nb, hkv, d, S, mb = 30, 3, 128, 5, 6
    kc = rng.integers(0, 256, (nb, bs, hkv, d), dtype=np.uint8)
    vc = rng.integers(0, 256, (nb, bs, hkv, d), dtype=np.uint8)
    ks = rng.random(nb, dtype=np.float32) + 0.5
    vs = rng.random(nb, dtype=np.float32) + 0.5
    tables = rng.integers(0, nb, (S, mb)).astype(np.int32)
    tables[0, 1] = tables[1, 0]
    tables[2, 2] = -1
    lens = np.array([mb * bs, 3 * bs + 1, 5 * bs - 32, 0, 40], dtype=np.int32)
    x = np.uint32(0)
    for s in range(S):
        for pg in range(mb):
            for part in range(bs // 32):
                b = int(tables[s, pg])
                if pg * bs + 32 * part >= lens[s] or not 0 <= b < nb:
                    continue
                for kvh in range(hkv):
                    for c in (kc, vc):
                        x ^= np.bitwise_xor.reduce(c[b, 32 * part:32 * part + 32, kvh].copy().view(np.uint32).ravel())
                    x ^= ks[b:b + 1].view(np.uint32)[0] ^ vs[b:b + 1].view(np.uint32)[0]
    t = lambda a: torch.from_numpy(a).to(cuda)  # noqa: E731
    tk, tv, tks, tvs, tt, tl = t(kc), t(vc), t(ks), t(vs), t(tables), t(lens)
    sink = torch.zeros(1024, dtype=torch.int32, device=cuda)
    lib = _native.load()
    rc = lib.emx_probe_page_read_fp8(tk.data_ptr(), tv.data_ptr(), tks.data_ptr(), tvs.data_ptr(), nb, bs, hkv, d,
                                     tt.data_ptr(), S, mb, tl.data_ptr(), sink.data_ptr(), sink.numel(),
                                     torch.cuda.current_stream(cuda).cuda_stream)
    _native.check(rc)
    torch.cuda.synchronize()
    assert np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32)) == x


def test_stream_pointer_follows_the_current_stream(cuda):
    """The raw stream every entry point launches on is torch's current stream, inside a stream context too."""
    assert _native.stream_ptr(cuda) == torch.cuda.current_stream(cuda).cuda_stream
    side = torch.cuda.Stream(cuda)
    with torch.cuda.stream(side):
        assert _native.stream_ptr(cuda) == side.cuda_stream
    assert _native.stream_ptr(torch.device("cuda")) == torch.cuda.current_stream().cuda_stream
