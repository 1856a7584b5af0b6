"""fskernels: the GQA flash-decode hot path of coder0143/fasterkernels on MI355X.

The reference's module paths, with one HIP backend (gfx950) behind them:

* ``fskernels.hip`` -- the decode entry points that replace the Triton, CUDA
  and TileLang decode modules (``flash_decode_gqa_varlen``,
  ``flash_decode_gqa_hf_dense_optimized``, ``flash_decode_gqa_hf_fp8``,
  ``quantize_to_fp8``, ``set_num_splits[_fp8]``, ``paged_kv_write``) and the
  HF attention patches (``fskernels.hip.hf``);
* ``fskernels.paged_attn`` -- ``PagedKVCache``, ``PAGE_SIZE`` and
  ``paged_flash_decode`` (fskernels/paged_attn/__init__.py:1-4 of the reference);
* ``fskernels.engine`` -- HIP-graph decode steps and the whole-model graph
  runner (the reference's fskernels/engine/cuda_graph_runner.py).

The kernels are hand-written HIP in the native library ``libfsk_decode.so``
(package ``fasterkernels_amd``: sources, C ABI, build); nothing here falls
back to another implementation.
"""

__version__ = "0.2.0"
