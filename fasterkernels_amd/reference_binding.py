"""ctypes-only binding of the varlen decode, as a reference maintainer would add it.

This is the whole of what the reference's ``fskernels/cuda/cuda_fd_gqa.py``
(:5-15, a JIT pybind build of ``flash_decode_api.cpp``) becomes when it binds
``libfsk_decode.so`` instead: no compiled Python-side binding, one ctypes call
per decode.  It imports nothing from this package, so it can be copied into
the reference tree unchanged; ``FSK_LIBRARY`` (or the ``path`` argument of
``load``) names the library, default: the in-tree build next to this file.

``flash_decode_gqa_varlen(q, k, v, cu_seqlens_k, sink=None)`` keeps the CUDA
module's positional signature and its numbers: the sink is folded linearly
into the softmax denominator (FSK_SINK_LINEAR), as
``fskernels/cuda/flash_decode_cuda.cu:151-153`` does.  Unlike the CUDA
extension it also takes bf16 (q, k and v of one dtype), never reads
``cu_seqlens_k`` back to the host, and raises instead of returning
uninitialised memory for an unsupported shape.
"""
from __future__ import annotations

import ctypes
import math
import os

import torch

_P, _I, _L, _F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float

# fsk_decode_varlen's parameters, in include/fsk_decode.h's order.
VARLEN_ARGTYPES = [
    _P, _L, _L,        # q, q_stride_b, q_stride_h
    _P, _L, _L,        # k, k_stride_t, k_stride_h
    _P, _L, _L,        # v, v_stride_t, v_stride_h
    _P, _L,            # cu_seqlens, total_tokens
    _P, _I,            # s_aux, sink_mode
    _P, _P,            # k_scale, v_scale
    _P, _L, _L,        # out, o_stride_b, o_stride_h
    _I, _I, _I, _I,    # batch, num_q_heads, num_kv_heads, head_dim
    _I, _I, _I, _F,    # q_dtype, kv_dtype, out_dtype, sm_scale
    _P, _L, _I,        # workspace, workspace_bytes, chunk_tokens
    _P,                # stream
]
WORKSPACE_ARGTYPES = [_I, _I, _I, _I, _I, _L, _I, _I]

FSK_LAYOUT_VARLEN = 0
FSK_SINK_LINEAR = 1
_DTYPES = {torch.float16: 0, torch.bfloat16: 1}

_lib = None


def load(path: str | None = None) -> ctypes.CDLL:
    """Opens the library once and declares the three entry points used here."""
    global _lib
    if _lib is None:
        path = path or os.environ.get("FSK_LIBRARY") or os.path.join(
            os.path.dirname(os.path.abspath(__file__)), "libfsk_decode.so")
        lib = ctypes.CDLL(path)
        lib.fsk_decode_varlen.restype = _I
        lib.fsk_decode_varlen.argtypes = VARLEN_ARGTYPES
        lib.fsk_workspace_bytes.restype = _L
        lib.fsk_workspace_bytes.argtypes = WORKSPACE_ARGTYPES
        lib.fsk_last_error.restype = ctypes.c_char_p
        lib.fsk_last_error.argtypes = []
        _lib = lib
    return _lib


def flash_decode_gqa_varlen(q, k, v, cu_seqlens_k, sink=None):
    """q [B, Hq, D], k/v [T, Hkv, D] (fp16 or bf16, head_dim contiguous,
    16-byte aligned rows), cu_seqlens_k [B+1] (int32 on the device, or
    converted), sink fp32 [Hq] or None -> new [B, Hq, D] in q's dtype."""
    lib = load()
    for name, t in (("q", q), ("k", k), ("v", v), ("cu_seqlens_k", cu_seqlens_k)):
        if not t.is_cuda:
            raise RuntimeError(f"{name} must be a CUDA (HIP) tensor")
    if q.dtype not in _DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"q, k and v must share one of float16 / bfloat16, got {q.dtype}, {k.dtype}, {v.dtype}")
    # The library reads these tensors through the sizes given here, so their
    # extents are checked first (a short tensor would be read past its end).
    if q.dim() != 3 or k.dim() != 3 or v.shape != k.shape or k.shape[2] != q.shape[2]:
        raise ValueError(f"q must be [B, Hq, D] and k, v [T, Hkv, D], got {tuple(q.shape)}, {tuple(k.shape)}, "
                         f"{tuple(v.shape)}")
    B, Hq, D = q.shape
    T, Hkv, _ = k.shape
    if cu_seqlens_k.numel() != B + 1:
        raise ValueError(f"cu_seqlens_k must have B + 1 = {B + 1} entries, got {cu_seqlens_k.numel()}")
    cu = cu_seqlens_k if (cu_seqlens_k.dtype == torch.int32 and cu_seqlens_k.is_contiguous()) \
        else cu_seqlens_k.to(torch.int32).contiguous()
    if sink is not None:
        if sink.numel() != Hq:
            raise ValueError(f"sink must have one entry per query head ({Hq}), got {sink.numel()}")
        sink = sink.to(device=q.device, dtype=torch.float32).reshape(Hq).contiguous()
    out = torch.empty_like(q)
    code = _DTYPES[q.dtype]
    with torch.cuda.device(q.device):  # the size follows the current device's CU count
        n = lib.fsk_workspace_bytes(FSK_LAYOUT_VARLEN, B, Hq, Hkv, D, T, 16, 0)
        if n < 0:
            _raise(lib, n)
        ws = torch.empty(n, dtype=torch.uint8, device=q.device)
        st = lib.fsk_decode_varlen(
            q.data_ptr(), q.stride(0), q.stride(1),
            k.data_ptr(), k.stride(0), k.stride(1),
            v.data_ptr(), v.stride(0), v.stride(1),
            cu.data_ptr(), T, None if sink is None else sink.data_ptr(), FSK_SINK_LINEAR,
            None, None, out.data_ptr(), out.stride(0), out.stride(1),
            B, Hq, Hkv, D, code, code, code, 1.0 / math.sqrt(D),
            ws.data_ptr(), n, 0, torch.cuda.current_stream(q.device).cuda_stream)
    if st != 0:
        _raise(lib, st)
    return out


def _raise(lib, status):
    """The library's status as an exception: bad argument -> ValueError,
    unsupported case -> NotImplementedError, anything else -> RuntimeError."""
    msg = lib.fsk_last_error().decode(errors="replace")
    raise (ValueError if status == -1 else NotImplementedError if status == -2 else RuntimeError)(msg)
