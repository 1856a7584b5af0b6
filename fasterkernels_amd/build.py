"""Builds the gfx950 shared library ``libfsk_decode.so`` in-tree with hipcc.

Usage: ``python -m fasterkernels_amd.build`` (or ``__graft_entry__.build()``).
The library is a plain C-ABI ``.so`` (see include/fsk_decode.h); Python loads
it with ctypes, so no torch extension machinery is involved.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
SRC = os.path.join(PKG_DIR, "csrc", "fsk_decode.hip")
INCLUDE = os.path.join(REPO_DIR, "include")
LIB_NAME = "libfsk_decode.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
ARCH = "gfx950"


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; ROCm is required to build libfsk_decode.so")
    return path


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        # Packed-FP32 VALU ops are kept out of the generated code on purpose.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-fvisibility=hidden",
        f"-I{INCLUDE}",
    ]


def build(verbose: bool = False) -> str:
    """Compiles the library (always) and returns its path."""
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), *compile_flags(), SRC, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns about the device-only target feature; ignore it.
    noise = ("packed-fp32-ops", "hip-link", "not a recognized feature")
    msgs = [ln for ln in (res.stderr or "").splitlines() if not any(n in ln for n in noise)]
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs), file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
