"""ctypes binding of ``libemx_attn.so`` (the C ABI declared in ``include/emx_attn.h``).

The library is built in-tree by ``easymlx_amd._build.build_native()`` (also run
by ``__graft_entry__.build()``).  There is no fallback: if the library is
missing every entry point raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

_LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib")
LIB_PATH = os.path.join(_LIB_DIR, "libemx_attn.so")

EMX_OK = 0
EMX_ERR_INVALID = -1
EMX_ERR_UNSUPPORTED = -2
EMX_ERR_HIP = -3
APPEND_COUNTER_INTS = 4  # EMX_APPEND_COUNTER_INTS: the device ints a decode append counts on

DTYPE_F16 = 0
DTYPE_BF16 = 1
DTYPE_F32 = 2

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_long
_F = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); must match include/emx_attn.h exactly.
SIGNATURES: dict[str, tuple] = {
    "emx_version": (_I, []),
    "emx_last_error": (ctypes.c_char_p, []),
    "emx_affine_quantize": (_I, [_P, _L, _I, _I, _I, _P, _P, _P, _P]),
    "emx_affine_cache_write": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P]),
    "emx_affine_cache_write_rope": (_I, [_P, _P, _P] + [_I] * 7 + [_P] * 6 + [_P, _P, _I, _I, _P, _P, _I, _P]),
    "emx_fp8_cache_write_rope": (
        _I, [_P, _P, _I, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _SZ, _P, _P, _I, _I, _P, _P, _I, _P]),
    "emx_rope_rows": (_I, [_P, _I, _I, _I, _P, _P, _I, _I, _P]),
    "emx_affine_cache_append_rope": (_I, [_P, _P, _P, _I, _P, _I, _I, _P, _P] + [_I] * 6 + [_P] * 7 + [_I, _I, _P, _P,
                                                                                                    _I, _P]),
    "emx_fp8_cache_append_rope": (
        _I, [_P, _P, _I, _P, _I, _P, _I, _I, _P, _P] + [_I] * 4 + [_P] * 5 + [_I, _I, _P, _P, _I, _P]),
    "emx_cache_slots": (_I, [_P, _P, _I, _I, _P, _I, _I, _I, _P, _P, _P, _P]),
    "emx_dense_cache_write": (_I, [_P, _P, _I, _P, _I, _I, _I, _I, _I, _P, _P, _P]),
    "emx_copy_blocks": (_I, [_I, _P, _P, _I, _P, _I, _P, _SZ, _P]),
    "emx_copy_blocks_workspace_bytes": (_SZ, [_I, _P, _I]),
    "emx_gather_kv_affine": (_I, [_P] * 6 + [_I] * 6 + [_P, _I, _I, _P, _I, _I, _P, _P, _P]),
    "emx_affine_pages_from_logical": (_I, [_P] * 6 + [_I] * 6 + [_P] * 7),
    "emx_affine_logical_from_pages": (_I, [_P] * 6 + [_I] * 6 + [_P] * 7),
    "emx_probe_page_read": (_I, [_P] * 6 + [_I] * 6 + [_P, _I, _I, _P, _P, _I, _P]),
    "emx_probe_page_read_fp8": (_I, [_P] * 4 + [_I] * 4 + [_P, _I, _I, _P, _P, _I, _P]),
    "emx_gather_kv_fp8": (_I, [_P] * 4 + [_I] * 4 + [_P, _I, _I, _P, _I, _I, _P, _P, _P]),
    "emx_gather_kv_dense": (_I, [_P, _P] + [_I] * 5 + [_P, _I, _I, _P, _I, _I, _P, _P, _P]),
    "emx_zero_blocks": (_I, [_I, _P, _P, _I, _P, _I, _P]),
    "emx_paged_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I, _I]),
    "emx_paged_prefill_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I]),
    "emx_paged_attention_affine": (
        _I,
        [_P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _I, _I, _P, _P, _F, _I, _I, _P, _SZ, _P, _P],
    ),
    "emx_paged_attention_dense": (
        _I,
        [_P, _I, _I, _I, _I, _P, _P, _I, _I, _I, _P, _I, _I, _P, _P, _F, _I, _I, _P, _SZ, _P, _P],
    ),
    "emx_fp8_write_workspace_bytes": (_SZ, []),
    "emx_fp8_cache_write": (_I, [_P, _P, _I, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _SZ, _P]),
    "emx_fp8_cache_write_noalloc": (_I, [_P, _P, _I, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P]),
    "emx_paged_attention_fp8": (
        _I,
        [_P, _I, _I, _I, _I, _P, _P, _P, _P, _I, _I, _I, _P, _I, _I, _P, _P, _F, _I, _I, _P, _SZ, _P, _P],
    ),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class NativeLibraryMissing(RuntimeError):
    """Raised when ``libemx_attn.so`` has not been built."""


def stream_ptr(device) -> int:
    """The raw HIP stream torch currently launches on for ``device`` (what every entry point takes)."""
    global _raw_stream, _torch
    if _raw_stream is None:
        import torch

        _torch = torch
        # torch's own accessor of the current raw stream (no Stream object per call); the public route otherwise
        _raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None) or (
            lambda i: torch.cuda.current_stream(i).cuda_stream)
    idx = device.index
    return _raw_stream(idx if idx is not None else _torch.cuda.current_device())


_raw_stream = None
_torch = None


def load() -> ctypes.CDLL:
    """Load (once) and return the native library, with argtypes bound."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise NativeLibraryMissing(
                    f"{LIB_PATH} not found; build it with `python -c 'import __graft_entry__ as g; g.build()'`"
                )
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(rc: int) -> None:
    """Map a C status code to the reference's Python exception conventions."""
    if rc == EMX_OK:
        return
    msg = load().emx_last_error().decode("utf-8", "replace")
    if rc == EMX_ERR_INVALID:
        raise ValueError(msg)
    if rc == EMX_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)
