"""MI355X-native GQA flash decoding: the fskernels decode hot path on gfx950.

Entry points keep the reference's names and signatures:

* ``flash_decode_gqa_varlen`` -- varlen KV + sinks (fskernels/triton/triton_gqa_decode.py:126)
* ``paged_flash_decode`` / ``PagedKVCache`` / ``PAGE_SIZE`` -- paged KV (fskernels/paged_attn)
* ``flash_decode_gqa_hf_dense_optimized`` -- dense HF cache (fskernels/triton/triton_gqa_decode_hf.py:146)
* ``flash_decode_gqa_hf_fp8`` / ``quantize_to_fp8`` -- fp8 e4m3 KV (fskernels/triton/triton_gqa_decode_hf_fp8.py)
* ``paged_kv_write`` -- the KV write path behind ``PagedKVCache.append_kv``
  (fskernels/paged_attn/paged_kv_cache.py:109-132), batched, with e4m3 quantisation
"""
from .hip import (FP8_DTYPE, FP8_MAX, flash_decode_gqa_hf_dense_optimized, flash_decode_gqa_hf_fp8,
                  flash_decode_gqa_varlen, paged_flash_decode, paged_kv_write, quantize_to_fp8,
                  set_num_splits, set_num_splits_fp8)
from .paged_attn import PAGE_SIZE, PagedKVCache

__version__ = "0.1.0"

__all__ = [
    "FP8_DTYPE", "FP8_MAX", "PAGE_SIZE", "PagedKVCache", "flash_decode_gqa_varlen",
    "flash_decode_gqa_hf_dense_optimized", "flash_decode_gqa_hf_fp8", "paged_flash_decode", "paged_kv_write",
    "quantize_to_fp8", "set_num_splits", "set_num_splits_fp8",
]
