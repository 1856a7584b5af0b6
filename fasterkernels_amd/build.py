"""Builds the gfx950 shared library ``libfsk_decode.so`` and its torch-tensor
binding ``_fsk_torch`` in-tree.

Usage: ``python -m fasterkernels_amd.build`` (or ``__graft_entry__.build()``).
The library is a plain C-ABI ``.so`` (see include/fsk_decode.h), built with
hipcc for gfx950.  The binding (csrc/fsk_torch.cpp) is host-only C++ against
torch's headers, linked to the library; the Python entry points call it (one
C++ call per decode), and native.py's ctypes binding covers the rest of the
C ABI (options, timing, debug entry points).
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
STAMPS_PATH = os.path.join(PKG_DIR, "libfsk_decode_stamps.so")  # -DFSK_WAVE_STAMPS (measurement build)
TORCH_SRC = os.path.join(PKG_DIR, "csrc", "fsk_torch.cpp")
TORCH_EXT = "_fsk_torch"


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
        # The leading scalar/pointer kernel arguments (the partial kernel's
        # lengths pointers and batch) arrive in SGPRs at dispatch.
        "-mllvm", "-amdgpu-kernarg-preload-count=3",
        "-fvisibility=hidden",
        f"-Wl,-soname,{LIB_NAME}",
        f"-I{INCLUDE}",
    ]


def torch_ext_path() -> str:
    import sysconfig
    return os.path.join(PKG_DIR, TORCH_EXT + sysconfig.get_config_var("EXT_SUFFIX"))


def torch_ext_command(out: str) -> list[str]:
    """g++ line of the binding: torch's headers and pybind11, the C ABI header,
    linked to libfsk_decode.so next to it (rpath $ORIGIN) and to torch."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension as ce
    cxx = shutil.which("g++") or shutil.which("c++")
    if not cxx:
        raise RuntimeError("a host C++ compiler (g++) is required to build the torch binding")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [cxx, "-O2", "-std=c++17", "-shared", "-fPIC", "-fvisibility=hidden",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", f"-DTORCH_EXTENSION_NAME={TORCH_EXT}",
           "-DTORCH_API_INCLUDE_EXTENSION_H", "-Wno-deprecated-declarations",
           f"-I{INCLUDE}", f"-I{sysconfig.get_paths()['include']}"]
    cmd += [f"-I{p}" for p in ce.include_paths()]
    cmd += [TORCH_SRC, "-o", out, f"-L{PKG_DIR}", "-l:" + LIB_NAME, "-Wl,-rpath,$ORIGIN"]
    for lib_dir in ce.library_paths():
        cmd += [f"-L{lib_dir}", f"-Wl,-rpath,{lib_dir}"]
    cmd += ["-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python"]
    return cmd


def build_torch_ext(verbose: bool = False) -> str:
    """Compiles the torch binding (always; needs libfsk_decode.so built first)."""
    out = torch_ext_path()
    tmp = out + ".tmp"
    cmd = torch_ext_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("building the torch binding failed:\n" + (res.stderr or "")[-4000:])
    os.replace(tmp, out)
    return out


def build_library(out: str, extra: list[str], verbose: bool) -> str:
    tmp = out + ".tmp"
    cmd = [hipcc(), *compile_flags(), *extra, SRC, "-o", tmp]
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
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> str:
    """Compiles the library, its wave-stamp twin and the torch binding
    (always) and returns the library's path."""
    build_library(LIB_PATH, [], verbose)
    build_library(STAMPS_PATH, ["-DFSK_WAVE_STAMPS=1"], verbose)
    build_torch_ext(verbose)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
