"""HF transformers attention functions that run decode steps on the HIP kernels.

Reference: fskernels/triton/triton_gqa_decode_hf.py:218-258
(custom_hf_decode_attention_forward) and
fskernels/triton/triton_gqa_decode_hf_fp8.py:230-283
(custom_hf_decode_attention_forward_fp8).  They have the signature of
transformers' ``eager_attention_forward`` and are installed the way the
reference's scripts install theirs (benchmarks/run_hf_model_triton.py:9)::

    import transformers.models.qwen3.modeling_qwen3 as qwen3_mod
    qwen3_mod.eager_attention_forward = custom_hf_decode_attention_forward

or with ``patch_hf_attention()`` / ``patched_hf_attention()``.

A decode step (one query position) attends over the cache the model hands
in: key/value states [B, Hkv, S, D] from a dynamic cache (S = the sequence so
far) or a static cache (S = its capacity).  The attended range of each
sequence is computed on the device (see _decode_bounds), so the step needs no
host synchronisation and can be captured in a HIP graph.  Other calls
(prefill) go to transformers' own eager attention, as in the reference.

Differences from the reference, all deliberate:

* Decode is recognised by ``q_len == 1``.  The reference also requires
  ``past_key_values`` and ``cache_position`` in the keyword arguments; the
  installed transformers (5.x) passes neither on to the attention function,
  so that patch never takes its decode path there.  Without
  ``cache_position`` the range comes from the attention mask.
* A sliding window attends the last ``sliding_window`` positions
  ``[len - window, len)``.  The reference passes the clamped length as the end
  of the range (:244-250), which attends the wrong tokens once
  ``len > window``.
* ``scaling`` is the softmax scale the kernels use (the reference kernels use
  1/sqrt(D), the value Qwen3 passes).
* The fp8 path honours a sliding window too.
* With ``cache_position`` the mask is not read, as in the reference; without
  it, the mask's attended positions must form one contiguous range per
  sequence (true of causal, padding, static-cache and sliding-window masks).
"""
from __future__ import annotations

import contextlib
from typing import Optional, Tuple

import torch

from .decode import (_on_gpu, flash_decode_gqa_hf_dense_optimized, flash_decode_gqa_hf_fp8,
                     quantize_to_fp8)

try:  # captured before anything is patched, as the reference module does (:3)
    from transformers.models.qwen3.modeling_qwen3 import eager_attention_forward as _native_eager
except ImportError:  # pragma: no cover - transformers missing
    _native_eager = None

if getattr(_native_eager, "_fsk_patch", False):  # imported after a patch was installed by hand
    raise ImportError("fskernels.hip.hf must be imported before eager_attention_forward is patched")


def native_eager_attention_forward(*args, **kwargs):
    if _native_eager is None:
        raise RuntimeError("transformers is not installed")
    return _native_eager(*args, **kwargs)


def _decode_bounds(query_states: torch.Tensor, key_states: torch.Tensor, attention_mask,
                   kwargs) -> Optional[Tuple[torch.Tensor, Optional[torch.Tensor]]]:
    """(cache_lens, start_offsets) of a decode step, or None for other calls.

    All values are computed on the device:
    * with ``cache_position`` (transformers versions that pass it, and the
      reference's contract): length cache_position[-1] + 1 and, for a sliding
      window, start max(0, length - window);
    * otherwise from the attention mask's row for the query, [B, 1, 1, S]
      (0 or True = attended): the first and one past the last attended
      position, which covers left padding, a static cache's unused tail and
      sliding windows (the attended positions must be contiguous);
    * without a mask: all S positions, and the sliding window if one is given.
    """
    bsz, _, q_len, _ = query_states.shape
    if q_len != 1:
        return None
    _on_gpu(query_states, "query_states")
    S = key_states.shape[2]
    dev = query_states.device
    window = kwargs.get("sliding_window")
    cache_position = kwargs.get("cache_position")
    if cache_position is not None:
        lens = (cache_position[-1:] + 1).to(torch.int32).expand(bsz).contiguous()
    elif attention_mask is not None:
        row = attention_mask[:, 0, -1, :S]
        valid = row if row.dtype == torch.bool else row == 0
        valid = valid.expand(bsz, S)
        idx = torch.arange(S, device=dev, dtype=torch.int32)
        ends = torch.where(valid, idx + 1, 0).amax(-1)
        starts = torch.minimum(torch.where(valid, idx, S).amin(-1), ends)
        return ends.to(torch.int32).contiguous(), starts.to(torch.int32).contiguous()
    else:
        lens = torch.full((bsz,), S, dtype=torch.int32, device=dev)
    starts = None
    if window is not None:
        starts = torch.clamp(lens - int(window), min=0)
    return lens, starts


def custom_hf_decode_attention_forward(module: torch.nn.Module, query_states: torch.Tensor,
                                       key_states: torch.Tensor, value_states: torch.Tensor,
                                       attention_mask, scaling: float, dropout: float = 0.0, **kwargs):
    """eager_attention_forward replacement: decode steps on the split-KV HIP
    kernels over the dense cache, everything else on transformers' eager path.
    Returns (attn_output [B, Hq, D], None) on decode steps (reshaped by the
    caller exactly as eager's [B, 1, Hq, D])."""
    bounds = _decode_bounds(query_states, key_states, attention_mask, kwargs)
    if bounds is None:
        return native_eager_attention_forward(module, query_states, key_states, value_states,
                                              attention_mask, scaling, dropout, **kwargs)
    lens, starts = bounds
    out = flash_decode_gqa_hf_dense_optimized(query_states.squeeze(2), key_states, value_states, lens, starts,
                                              sm_scale=scaling)
    return out, None


def custom_hf_decode_attention_forward_fp8(module: torch.nn.Module, query_states: torch.Tensor,
                                           key_states: torch.Tensor, value_states: torch.Tensor,
                                           attention_mask, scaling: float, dropout: float = 0.0, **kwargs):
    """FP8 variant: Q, K and V are quantised per call with per-tensor scales
    (quantize_to_fp8, as triton_gqa_decode_hf_fp8.py:268-273 does) and decoded
    by the e4m3 kernels; the output keeps the query dtype."""
    bounds = _decode_bounds(query_states, key_states, attention_mask, kwargs)
    if bounds is None:
        return native_eager_attention_forward(module, query_states, key_states, value_states,
                                              attention_mask, scaling, dropout, **kwargs)
    lens, starts = bounds
    q8, sq = quantize_to_fp8(query_states.squeeze(2).float())
    k8, sk = quantize_to_fp8(key_states.float())
    v8, sv = quantize_to_fp8(value_states.float())
    out = flash_decode_gqa_hf_fp8(q8, k8, v8, lens, sq, sk, sv, query_states.dtype, start_k_offsets=starts,
                                  sm_scale=scaling)
    return out, None


custom_hf_decode_attention_forward._fsk_patch = True
custom_hf_decode_attention_forward_fp8._fsk_patch = True


def patch_hf_attention(fp8: bool = False, modeling_module=None):
    """Installs the decode attention as ``modeling_module.eager_attention_forward``
    (default: transformers' Qwen3 module) and returns the function it replaced."""
    if modeling_module is None:
        import transformers.models.qwen3.modeling_qwen3 as modeling_module
    prev = modeling_module.eager_attention_forward
    modeling_module.eager_attention_forward = (custom_hf_decode_attention_forward_fp8 if fp8
                                               else custom_hf_decode_attention_forward)
    return prev


@contextlib.contextmanager
def patched_hf_attention(fp8: bool = False, modeling_module=None):
    """Context manager form of patch_hf_attention; restores the previous function."""
    if modeling_module is None:
        import transformers.models.qwen3.modeling_qwen3 as modeling_module
    prev = patch_hf_attention(fp8, modeling_module)
    try:
        yield
    finally:
        modeling_module.eager_attention_forward = prev
