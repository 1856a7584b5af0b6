"""The single HIP backend of the decode hot path (gfx950): it replaces the
reference's fskernels.triton, fskernels.cuda and fskernels.tilelang decode
modules.  The HF attention patches are in fskernels.hip.hf."""
from .decode import (FP8_DTYPE, FP8_MAX, flash_decode_gqa_hf_dense_optimized,
                     flash_decode_gqa_hf_fp8, flash_decode_gqa_varlen, fp8_decode_table,
                     paged_flash_decode, paged_gather, quantize_to_fp8, set_num_splits,
                     set_num_splits_fp8)
from .kv_write import paged_kv_write

__all__ = [
    "FP8_DTYPE", "FP8_MAX", "flash_decode_gqa_varlen", "flash_decode_gqa_hf_dense_optimized",
    "flash_decode_gqa_hf_fp8", "paged_flash_decode", "quantize_to_fp8", "set_num_splits",
    "set_num_splits_fp8", "paged_gather", "fp8_decode_table", "paged_kv_write",
]
