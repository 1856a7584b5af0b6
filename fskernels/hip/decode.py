"""GQA flash-decode entry points backed by the gfx950 HIP library.

Each function keeps the name, positional signature, tensor layouts and return
value of the reference entry point it replaces; new behaviour is only added
through keyword-only arguments.  Every call goes to the torch binding
(fasterkernels_amd/csrc/fsk_torch.cpp) in one C++ call, which validates the
tensors, allocates the output and a split-KV workspace through torch's
caching allocator and launches the HIP kernels on torch's current stream (no
host synchronisation, so the calls can be captured in a HIP graph).
"""
from __future__ import annotations

import math

import torch

from fasterkernels_amd import native as nat

FP8_DTYPE = torch.float8_e4m3fn
FP8_MAX = 448.0

# Split counts fixed before graph capture, as in the reference modules
# (fskernels/triton/triton_gqa_decode_hf.py:8-14, triton_gqa_decode_hf_fp8.py:156-161).
_DECODE_NUM_SPLITS: int = 1
_DECODE_NUM_SPLITS_FP8: int = 1


def set_num_splits(n: int) -> None:
    """Split-count hint for flash_decode_gqa_hf_dense_optimized.

    The HIP kernels always split the KV sequence across the GPU with a device
    work list; a value n above 1 makes every full-length sequence split into
    at least n parts (chunks of at most ceil(S_max / n) tokens, rounded up to
    32), finer where the GPU needs more work items; 1 leaves the split to the
    library.  Mirrors fskernels/triton/triton_gqa_decode_hf.py:12-14.
    """
    global _DECODE_NUM_SPLITS
    _DECODE_NUM_SPLITS = int(n)


def set_num_splits_fp8(n: int) -> None:
    """Split-count hint for flash_decode_gqa_hf_fp8 (see set_num_splits).

    Mirrors fskernels/triton/triton_gqa_decode_hf_fp8.py:159-161.
    """
    global _DECODE_NUM_SPLITS_FP8
    _DECODE_NUM_SPLITS_FP8 = int(n)


def quantize_to_fp8(x: torch.Tensor):
    """Per-tensor e4m3 quantisation: scale = max|x| / 448 (floored at 1e-12/448).

    Same formula and return value as
    fskernels/triton/triton_gqa_decode_hf_fp8.py:13-16: returns (x_fp8, scale)
    with scale a 0-dim fp32 tensor on x's device.
    """
    scale = x.abs().max().clamp(min=1e-12) / FP8_MAX
    x_fp8 = (x / scale).clamp(-FP8_MAX, FP8_MAX).to(FP8_DTYPE)
    return x_fp8, scale


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------
def _on_gpu(t: torch.Tensor, name: str, device: torch.device | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be on a GPU (HIP) device")
    if device is not None and t.get_device() != device.index:
        raise RuntimeError(f"{name} is on {t.device}, expected {device}")


def _inner_contig(t: torch.Tensor) -> torch.Tensor:
    """Innermost dim contiguous with 16-byte aligned rows, else a packed copy."""
    es = t.element_size()
    ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all((s * es) % 16 == 0 for s in t.stride()[:-1])
    return t if ok else t.contiguous()


def _int32(t: torch.Tensor, name: str, device: torch.device) -> torch.Tensor:
    _on_gpu(t, name, device)
    if t.dtype is torch.int32 and t.is_contiguous():
        return t
    return t.to(torch.int32).contiguous()


def _dtype_code(dt: torch.dtype, name: str) -> int:
    try:
        return nat.DTYPE_CODES[dt]
    except KeyError:
        raise NotImplementedError(f"{name}: unsupported dtype {dt}") from None


def _out_code(dt) -> int:
    """Output dtype code for the binding (-1: the query's dtype)."""
    return -1 if dt is None else _dtype_code(dt, "out_dtype")


def _sink_mode(mode: str) -> int:
    try:
        return nat.SINK_MODES[mode]
    except KeyError:
        raise ValueError(f"sink_mode must be 'exp' or 'linear', got {mode!r}") from None


_raw_stream = nat.raw_stream


def _stream(q) -> int:
    """torch's current HIP stream on q's device (0 for a host tensor, which
    the binding then rejects)."""
    if not isinstance(q, torch.Tensor):
        raise TypeError("q must be a torch.Tensor")
    index = q.get_device()
    return _raw_stream(index) if index >= 0 else 0


def _scale_tensor(s, like):
    """Scales are device fp32 scalars; a Python number becomes one on like's device."""
    if s is None or isinstance(s, torch.Tensor):
        return s
    return torch.tensor(float(s), dtype=torch.float32, device=like.device)


def _scores_out(wanted, score_blocks, extent_tokens, q, odt):
    """Block-score output [B, Hq, n] (n = score_blocks or ceil(extent / 128)), or None."""
    if not wanted:
        return None
    _on_gpu(q, "q")
    if q.dim() != 3:
        raise ValueError(f"q must be [batch, num_q_heads, head_dim], got {tuple(q.shape)}")
    n = int(score_blocks) if score_blocks is not None else max(1, -(-int(extent_tokens) // 128))
    if n <= 0:
        raise ValueError("score_blocks must be positive")
    return torch.empty((q.shape[0], q.shape[1], n), dtype=odt or q.dtype, device=q.device)


def _sm(sm_scale):
    return None if sm_scale is None else float(sm_scale)


# ---------------------------------------------------------------------------
# varlen
# ---------------------------------------------------------------------------
def flash_decode_gqa_varlen(q, k_varlen, v_varlen, cu_seqlens_k, s_aux=None, *,
                            sink_mode: str = "linear", k_scale=None, v_scale=None,
                            out_dtype: torch.dtype | None = None, sm_scale: float | None = None,
                            chunk_tokens: int = 0, return_block_scores: bool = False,
                            score_blocks: int | None = None):
    """Varlen GQA flash decode: out[b, h] = softmax(q[b,h] . K_b^T * sm_scale) V_b.

    Reference: fskernels/triton/triton_gqa_decode.py:126-155 (and the positional
    CUDA/TileLang variants fskernels/cuda/cuda_fd_gqa.py:14-15,
    fskernels/tilelang/tilelang_gqa_decode.py:135-172).  q [B, Hq, D];
    k_varlen / v_varlen [T, Hkv, D] packed by cu_seqlens_k int32 [B+1];
    cu_seqlens_k may be a host (CPU) tensor: the work plan is then built on
    the host from it (no device read of the lengths at the start of every
    workgroup; bit-identical results), for up to 64 sequences without block
    scores, and copied to the device otherwise.
    s_aux fp32 [Hq] sinks folded per ``sink_mode``: "linear" (default) adds
    the sink to the softmax denominator relative to the running maximum, as
    all three replaced kernels do (triton_gqa_decode.py:112-115,
    flash_decode_cuda.cu:151-153, tilelang_gqa_decode.py:117-120); "exp"
    treats it as one more logit with a zero value row (the reference tests'
    oracle, tests/test_triton_fd_gqa.py:27-33, and the sink-logit form of
    models with attention sinks).  Returns a new [B, Hq, D] tensor of q's dtype
    (``out_dtype`` overrides it).  fp8 K/V need k_scale / v_scale.

    ``return_block_scores=True`` returns ``(out, S)`` with S [B, Hq, n] the
    largest attention probability of each 128-token block of each sequence
    (0 past its end), the S output of the TileLang kernel
    (fskernels/tilelang/tilelang_gqa_decode.py:123-130); n = ``score_blocks``
    or enough blocks for total_tokens.
    """
    scores = None
    if return_block_scores:
        _on_gpu(k_varlen, "k_varlen")
        scores = _scores_out(True, score_blocks, k_varlen.shape[0], q, out_dtype)
    out = nat.ext().varlen(q, k_varlen, v_varlen, cu_seqlens_k, s_aux, _scale_tensor(k_scale, q),
                           _scale_tensor(v_scale, q), _out_code(out_dtype), _sink_mode(sink_mode), _sm(sm_scale),
                           int(chunk_tokens), scores, _stream(q))
    return out if scores is None else (out, scores)


# ---------------------------------------------------------------------------
# dense (HF static cache)
# ---------------------------------------------------------------------------
def _dense(q, k_cache, v_cache, cache_lens, start_k_offsets, num_splits, *, q_scale=None,
           k_scale=None, v_scale=None, out_dtype=None, s_aux=None, sink_mode="linear",
           sm_scale=None, chunk_tokens=0):
    if not chunk_tokens and num_splits and num_splits > 1:
        _on_gpu(k_cache, "k_cache")
        if k_cache.dim() != 4:
            raise ValueError("k_cache must be [batch, num_kv_heads, max_seqlen, head_dim]")
        S = k_cache.shape[2]
        # at least num_splits parts per sequence: chunks of at most this size
        chunk_tokens = -max(32, -(-math.ceil(S / num_splits) // 32) * 32)
    return nat.ext().dense(q, k_cache, v_cache, cache_lens, start_k_offsets, s_aux, _scale_tensor(q_scale, q),
                           _scale_tensor(k_scale, q), _scale_tensor(v_scale, q), _out_code(out_dtype),
                           _sink_mode(sink_mode), _sm(sm_scale), int(chunk_tokens), _stream(q))


def flash_decode_gqa_hf_dense_optimized(q, k_cache, v_cache, cache_lens, start_k_offsets=None,
                                        num_splits=None, *, s_aux=None, sink_mode: str = "linear",
                                        sm_scale: float | None = None):
    """Dense-cache split-KV decode over tokens [start_k_offsets[b], cache_lens[b]).

    Reference: fskernels/triton/triton_gqa_decode_hf.py:146-211.  q [B, Hq, D];
    k_cache / v_cache [B, Hkv, S_max, D] (HF static cache layout); cache_lens
    int32 [B]; start_k_offsets int32 [B] (None: zeros).  ``num_splits``
    (default: the set_num_splits value) is a split-count hint.
    """
    n = _DECODE_NUM_SPLITS if num_splits is None else num_splits
    return _dense(q, k_cache, v_cache, cache_lens, start_k_offsets, n, s_aux=s_aux,
                  sink_mode=sink_mode, sm_scale=sm_scale)


def flash_decode_gqa_hf_fp8(q_fp8, k_cache_fp8, v_cache_fp8, cache_lens, scale_q, scale_k,
                            scale_v, out_dtype, *, start_k_offsets=None, sm_scale: float | None = None):
    """FP8 e4m3 dense decode with per-tensor scales.

    Reference: fskernels/triton/triton_gqa_decode_hf_fp8.py:164-227.  q_fp8
    [B, Hq, D] and the caches [B, Hkv, S_max, D] are float8_e4m3fn; scale_* are
    0-dim fp32 device tensors (dequantised value = code * scale).  Q is
    dequantised to fp16 as the reference does (:47-50); K/V are dequantised
    exactly in registers and their scales applied in fp32.  Returns
    [B, Hq, D] in ``out_dtype``.  Keyword-only additions: ``start_k_offsets``
    (attend [start, cache_len) as the fp16/bf16 dense entry does) and
    ``sm_scale`` (default 1/sqrt(D)).
    """
    return _dense(q_fp8, k_cache_fp8, v_cache_fp8, cache_lens, start_k_offsets, _DECODE_NUM_SPLITS_FP8,
                  q_scale=scale_q, k_scale=scale_k, v_scale=scale_v, out_dtype=out_dtype,
                  sm_scale=sm_scale)


# ---------------------------------------------------------------------------
# paged
# ---------------------------------------------------------------------------
def paged_flash_decode(q, k_pool, v_pool, block_table, seq_lens, page_size, *, s_aux=None,
                       k_scale=None, v_scale=None, out_dtype: torch.dtype | None = None,
                       sink_mode: str = "linear", sm_scale: float | None = None,
                       chunk_tokens: int = 0, return_block_scores: bool = False,
                       score_blocks: int | None = None):
    """Paged GQA decode through a block table.

    Reference: fskernels/paged_attn/triton_paged_attn.py:96-125.  q [B, Hq, D];
    k_pool / v_pool [P, Hkv, page_size, D] (e.g. PagedKVCache.k_pool[layer]);
    block_table int32 [B, max_blocks] (logical page -> physical page, entries
    past a sequence's last page are never read); seq_lens int32 [B], on the
    GPU or in host memory (``PagedKVCache.get_seq_lens_tensor(ids,
    device="cpu")``): host lengths let the work plan be built on the host (no
    device read of the lengths at the start of every workgroup;
    bit-identical results), for up to 64 sequences without block scores, and
    are copied to the device otherwise.  The keyword-only arguments add sinks and fp8 (e4m3) pools with per-tensor
    scales, which the reference kernel does not have, and the block scores of
    flash_decode_gqa_varlen (default width: the block table's token capacity).
    """
    scores = None
    if return_block_scores:
        _on_gpu(block_table, "block_table")
        if block_table.dim() != 2:
            raise ValueError("block_table must be [batch, max_blocks]")
        scores = _scores_out(True, score_blocks, block_table.shape[1] * int(page_size), q, out_dtype)
    out = nat.ext().paged(q, k_pool, v_pool, block_table, seq_lens, int(page_size), s_aux,
                          _scale_tensor(k_scale, q), _scale_tensor(v_scale, q), _out_code(out_dtype),
                          _sink_mode(sink_mode), _sm(sm_scale), int(chunk_tokens), scores, _stream(q))
    return out if scores is None else (out, scores)


# ---------------------------------------------------------------------------
# debug exports
# ---------------------------------------------------------------------------
def paged_gather(pool, block_table, seq_lens):
    """Dense [B, Hkv, max_blocks*page_size, D] copy of a paged pool, read through
    the decode kernels' page-addressing routine (rows past seq_lens are zero)."""
    _on_gpu(pool, "pool")
    dev = pool.device
    pool = _inner_contig(pool)
    P, Hkv, PS, D = pool.shape
    bt = _int32(block_table, "block_table", dev)
    lens = _int32(seq_lens, "seq_lens", dev)
    if bt.dim() != 2:
        raise ValueError(f"block_table must be [batch, max_blocks], got {tuple(bt.shape)}")
    B, MB = bt.shape
    if lens.numel() < B:
        raise ValueError(f"seq_lens has {lens.numel()} entries for a batch of {B}")
    out = torch.empty((B, Hkv, MB * PS, D), dtype=pool.dtype, device=dev)
    lib = nat.load()
    st = nat.launch(dev.index, lib.fsk_paged_gather, pool.data_ptr(), pool.stride(0), pool.stride(1),
                    pool.stride(2), bt.data_ptr(), bt.stride(0), MB, lens.data_ptr(), P, PS, B, Hkv, D,
                    _dtype_code(pool.dtype, "pool"), out.data_ptr(), nat.stream_handle(dev))
    nat.check(st)
    return out


def fp8_decode_table(device="cuda"):
    """[2, 256] fp32: every e4m3 code through the kernels' f16 and bf16 routes
    (the kernel returns the 16-bit patterns; they are widened here)."""
    dev = torch.device(device)
    out = torch.empty(512, dtype=torch.int16, device=dev)
    lib = nat.load()
    st = nat.launch(dev.index, lib.fsk_fp8_decode_table, out.data_ptr(), nat.stream_handle(dev))
    nat.check(st)
    bits = out.cpu()
    return torch.stack([bits[:256].view(torch.float16).to(torch.float32),
                        bits[256:].view(torch.bfloat16).to(torch.float32)])
