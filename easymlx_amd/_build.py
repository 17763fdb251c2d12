"""In-tree build of ``easymlx_amd/_lib/libemx_attn.so`` with hipcc for gfx950."""

from __future__ import annotations

import os
import shutil
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(_HERE, "csrc")
SOURCES = [os.path.join(CSRC, "emx_attn.hip")]
DEPENDS = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hpp", ".hip"))]
OUT = os.path.join(_HERE, "_lib", "libemx_attn.so")

HIPCC_FLAGS = [
    "-O3",
    "--offload-arch=gfx950",
    "-std=c++17",
    "-shared",
    "-fPIC",
    # no packed-fp32 VALU ops anywhere in device code
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # leading kernel arguments arrive in SGPRs with the wave (gfx950 kernel-argument preload)
    "-mllvm",
    "-amdgpu-kernarg-preload-count=16",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm required to build libemx_attn.so)")
    return path


def build_native(verbose: bool = False) -> str:
    """Compile the HIP library; always recompiles.  Returns the .so path."""
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    tmp = OUT + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, *SOURCES, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{res.stderr[-4000:]}")
    if verbose:
        print(" ".join(cmd))
    os.replace(tmp, OUT)
    return OUT
