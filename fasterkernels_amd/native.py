"""ctypes binding of libfsk_decode.so (the C ABI in include/fsk_decode.h).

The library is built in-tree by ``python -m fasterkernels_amd.build``.  Nothing
here falls back to another implementation: if the library is missing, every
decode entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libfsk_decode.so")

# Status codes and enums (mirrors include/fsk_decode.h).
FSK_OK = 0
FSK_ERR_INVALID = -1
FSK_ERR_UNSUPPORTED = -2
FSK_ERR_WORKSPACE = -3
FSK_ERR_HIP = -4

FSK_F16, FSK_BF16, FSK_F32, FSK_E4M3 = 0, 1, 2, 3
FSK_SINK_EXP, FSK_SINK_LINEAR = 0, 1
FSK_LAYOUT_VARLEN, FSK_LAYOUT_PAGED, FSK_LAYOUT_DENSE = 0, 1, 2

DTYPE_CODES = {
    torch.float16: FSK_F16,
    torch.bfloat16: FSK_BF16,
    torch.float32: FSK_F32,
    torch.float8_e4m3fn: FSK_E4M3,
}
SINK_MODES = {"exp": FSK_SINK_EXP, "linear": FSK_SINK_LINEAR}

# Every exported symbol of the C ABI, with its ctypes signature.
_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float
SIGNATURES = {
    "fsk_last_error": (ctypes.c_char_p, []),
    "fsk_version": (_I, []),
    "fsk_set_option": (_I, [ctypes.c_char_p, _L]),
    "fsk_workspace_bytes": (_L, [_I, _I, _I, _I, _I, _L, _I, _I]),
    "fsk_decode_varlen": (_I, [_P, _L, _L, _P, _L, _L, _P, _L, _L, _P, _L, _P, _I, _P, _P,
                               _P, _L, _L, _I, _I, _I, _I, _I, _I, _I, _F, _P, _L, _I, _P]),
    "fsk_decode_paged": (_I, [_P, _L, _L, _P, _L, _L, _L, _P, _L, _L, _L, _P, _L, _I, _P, _I, _I,
                              _P, _I, _P, _P, _P, _L, _L, _I, _I, _I, _I, _I, _I, _I, _F, _P, _L,
                              _I, _P]),
    "fsk_decode_varlen_host": (_I, [_P, _L, _L, _P, _L, _L, _P, _L, _L, _P, _L, _P, _I, _P, _P,
                                    _P, _L, _L, _I, _I, _I, _I, _I, _I, _I, _F, _P, _L, _I, _P]),
    "fsk_decode_paged_host": (_I, [_P, _L, _L, _P, _L, _L, _L, _P, _L, _L, _L, _P, _L, _I, _P, _I, _I,
                                   _P, _I, _P, _P, _P, _L, _L, _I, _I, _I, _I, _I, _I, _I, _F, _P, _L,
                                   _I, _P]),
    "fsk_decode_paged_noalloc": (_I, [_P, _L, _L, _P, _L, _L, _L, _P, _L, _L, _L, _P, _L, _I, _P, _I, _I,
                                      _P, _I, _P, _P, _P, _L, _L, _I, _I, _I, _I, _I, _I, _I, _F, _I, _P]),
    "fsk_decode_dense": (_I, [_P, _L, _L, _P, _L, _L, _L, _P, _L, _L, _L, _L, _P, _P, _P, _I, _P,
                              _P, _P, _P, _L, _L, _I, _I, _I, _I, _I, _I, _I, _F, _P, _L, _I, _P]),
    "fsk_score_workspace_bytes": (_L, [_I, _I, _I]),
    "fsk_decode_varlen_scores": (_I, [_P, _L, _L, _P, _L, _L, _P, _L, _L, _P, _L, _P, _I, _P, _P,
                                      _P, _L, _L, _I, _I, _I, _I, _I, _I, _I, _F, _P, _L, _I, _P, _I, _P]),
    "fsk_decode_paged_scores": (_I, [_P, _L, _L, _P, _L, _L, _L, _P, _L, _L, _L, _P, _L, _I, _P, _I, _I,
                                     _P, _I, _P, _P, _P, _L, _L, _I, _I, _I, _I, _I, _I, _I, _F, _P, _L,
                                     _I, _P, _I, _P]),
    "fsk_paged_gather": (_I, [_P, _L, _L, _L, _P, _L, _I, _P, _I, _I, _I, _I, _I, _I, _P, _P]),
    "fsk_paged_write": (_I, [_P, _L, _L, _P, _L, _L, _P, _L, _P, _L, _L, _L, _P, _L, _L, _L, _I, _I,
                             _I, _I, _I, _I, _P, _P, _P, _L, _P, _L, _P]),
    "fsk_fp8_decode_table": (_I, [_P, _P]),
    "fsk_debug_split": (_I, [_L, _I, _I, _I, _I, _L, _I, _I, _I, _I, _P, _P, _P, _P, _P]),
    "fsk_enable_kernel_timing": (_I, [_I]),
    "fsk_kernel_timing": (_I, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                               ctypes.POINTER(ctypes.c_int64)]),
}

# The two debug entry points of the wave-stamp build (libfsk_decode_stamps.so).
STAMP_SIGNATURES = {
    "fsk_debug_wave_stamps": (_I, [_P, _I]),
    "fsk_debug_clear_wave_stamps": (_I, []),
}

_lock = threading.Lock()
_lib = None


class FskError(RuntimeError):
    """A HIP-side failure reported by libfsk_decode."""


def load() -> ctypes.CDLL:
    """Loads the library once and declares every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run `python -m fasterkernels_amd.build` "
                    "(the HIP library is required, there is no fallback)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def use_stamped_library() -> ctypes.CDLL:
    """Loads the wave-stamp build instead of the normal library (before any
    other use of this module in the process): the partial kernel then records
    each wave's timeline (fsk_debug_wave_stamps).  Its soname is the normal
    library's, so the torch binding imported afterwards binds to it."""
    global LIB_PATH
    if _lib is not None:
        raise RuntimeError("the library is already loaded in this process")
    from .build import STAMPS_PATH
    LIB_PATH = STAMPS_PATH
    lib = load()
    for name, (res, args) in STAMP_SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def check(status: int) -> None:
    """Maps a library status to the Python exception the reference would raise."""
    if status == FSK_OK:
        return
    msg = load().fsk_last_error().decode(errors="replace")
    if status == FSK_ERR_INVALID:
        raise ValueError(msg)
    if status == FSK_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    if status == FSK_ERR_WORKSPACE:
        raise RuntimeError(msg)
    raise FskError(f"libfsk_decode status {status}: {msg}")


def set_option(name: str, value: int) -> None:
    check(load().fsk_set_option(name.encode(), int(value)))
    _WS_CACHE.clear()  # workspace sizes follow the split options


# (device, layout, batch, hq, hkv, d, kv_extent, page_size, chunk_tokens) -> bytes
_WS_CACHE: dict = {}
_WS_CACHE_MAX = 4096


def workspace_bytes(layout: int, batch: int, hq: int, hkv: int, d: int, kv_extent: int,
                    page_size: int = 16, chunk_tokens: int = 0, device_index: int | None = None) -> int:
    """fsk_workspace_bytes for the current device, or for ``device_index``
    (then cached: the size depends only on the arguments, the device's CU
    count and the library options)."""
    key = (device_index, layout, batch, hq, hkv, d, kv_extent, page_size, chunk_tokens)
    if device_index is not None:
        n = _WS_CACHE.get(key)
        if n is not None:
            return n
        n = launch(device_index, load().fsk_workspace_bytes, layout, batch, hq, hkv, d, kv_extent, page_size,
                   chunk_tokens)
    else:
        n = load().fsk_workspace_bytes(layout, batch, hq, hkv, d, kv_extent, page_size, chunk_tokens)
    if n < 0:
        check(int(n))
    if device_index is not None:
        if len(_WS_CACHE) >= _WS_CACHE_MAX:
            _WS_CACHE.clear()  # (a varlen serving loop has a new total length every step)
        _WS_CACHE[key] = int(n)
    return int(n)


def score_workspace_bytes(batch: int, hq: int, score_blocks: int) -> int:
    n = load().fsk_score_workspace_bytes(batch, hq, score_blocks)
    if n < 0:
        check(int(n))
    return int(n)


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def raw_stream(index: int) -> int:
    """Handle of torch's current stream on device ``index``."""
    if _raw_stream is not None:
        return _raw_stream(index)
    return torch.cuda.current_stream(index).cuda_stream


_ext = None


def ext():
    """The torch binding (fasterkernels_amd._fsk_torch, built next to the
    library by ``python -m fasterkernels_amd.build``): one C++ call per decode
    or KV write.  Raises if it is not built; there is no other path."""
    global _ext
    if _ext is None:
        load()  # the C library first: the binding links this same file
        try:
            from . import _fsk_torch
        except ImportError as e:
            raise RuntimeError("the torch binding of libfsk_decode.so is not built; run "
                               f"`python -m fasterkernels_amd.build` ({e})") from None
        _ext = _fsk_torch
    return _ext


def stream_handle(device: torch.device | int) -> int:
    """Handle of torch's current stream on ``device``."""
    index = device if isinstance(device, int) else device.index
    if _raw_stream is not None and index is not None:
        return _raw_stream(index)
    return torch.cuda.current_stream(device).cuda_stream


def launch(device_index: int, fn, *args):
    """fn(*args) with ``device_index`` as the current HIP device (switched only
    when it is not already current)."""
    if torch._C._cuda_getDevice() == device_index:
        return fn(*args)
    with torch.cuda.device(device_index):
        return fn(*args)


def enable_kernel_timing(every_n: int = 1) -> None:
    """Record HIP events around every n-th decode call (0 disables)."""
    check(load().fsk_enable_kernel_timing(int(every_n)))


def kernel_timing():
    """(partial_ms, partial_plus_reduce_ms, calls) summed since the last read."""
    a, b, n = ctypes.c_double(), ctypes.c_double(), ctypes.c_int64()
    check(load().fsk_kernel_timing(ctypes.byref(a), ctypes.byref(b), ctypes.byref(n)))
    return a.value, b.value, n.value
