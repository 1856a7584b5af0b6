"""The reference's import paths and positional signatures resolve to this
build (CPU: imports and signatures only, no kernel calls).

A reference caller switches ``fskernels.triton`` / ``fskernels.cuda`` /
``fskernels.tilelang`` decode imports to ``fskernels.hip`` (the one backend)
and keeps ``fskernels.paged_attn`` as it is.
"""
import inspect

import pytest


def positional(fn):
    """Names of the parameters a positional call can fill."""
    return [p.name for p in inspect.signature(fn).parameters.values()
            if p.kind in (p.POSITIONAL_ONLY, p.POSITIONAL_OR_KEYWORD)]


def test_paged_attn_exports():
    # fskernels/paged_attn/__init__.py:1-4
    from fskernels.paged_attn import PAGE_SIZE, PagedKVCache, paged_flash_decode
    from fskernels.paged_attn.paged_kv_cache import PAGE_SIZE as PS, PagedKVCache as PKC
    assert PAGE_SIZE == PS == 16 and PagedKVCache is PKC
    # triton_paged_attn.py:96-103
    assert positional(paged_flash_decode) == ["q", "k_pool", "v_pool", "block_table", "seq_lens", "page_size"]
    # paged_kv_cache.py:9-28 (dataclass fields), :65-154 (methods)
    fields = list(inspect.signature(PagedKVCache).parameters)[:8]
    assert fields == ["num_layers", "num_pages", "max_seqs", "max_blocks_per_seq", "num_kv_heads", "head_dim",
                      "dtype", "device"]
    for name in ("from_config", "allocate_sequence", "free_sequence", "append_kv", "get_block_table_tensor",
                 "get_seq_lens_tensor"):
        assert callable(getattr(PagedKVCache, name)), name
    assert positional(PagedKVCache.append_kv) == ["self", "seq_id", "layer_idx", "k", "v"]
    assert isinstance(PagedKVCache.pages_used, property) and isinstance(PagedKVCache.pages_free, property)


def test_hip_backend_exports():
    from fskernels import hip
    # triton_gqa_decode.py:126, tilelang_gqa_decode.py:135-141 (s_aux), cuda_fd_gqa.py:14 (5th positional)
    assert positional(hip.flash_decode_gqa_varlen) == ["q", "k_varlen", "v_varlen", "cu_seqlens_k", "s_aux"]
    # triton_gqa_decode_hf.py:146, :12
    assert positional(hip.flash_decode_gqa_hf_dense_optimized) == [
        "q", "k_cache", "v_cache", "cache_lens", "start_k_offsets", "num_splits"]
    assert positional(hip.set_num_splits) == ["n"]
    # triton_gqa_decode_hf_fp8.py:164, :159, :13, :9-10
    assert positional(hip.flash_decode_gqa_hf_fp8) == [
        "q_fp8", "k_cache_fp8", "v_cache_fp8", "cache_lens", "scale_q", "scale_k", "scale_v", "out_dtype"]
    assert positional(hip.set_num_splits_fp8) == ["n"]
    assert positional(hip.quantize_to_fp8) == ["x"]
    import torch
    assert hip.FP8_DTYPE is torch.float8_e4m3fn and hip.FP8_MAX == 448.0
    # the paged decode is the same function from both packages
    from fskernels.paged_attn import paged_flash_decode
    assert hip.paged_flash_decode is paged_flash_decode


def test_hf_patch_exports():
    pytest.importorskip("transformers")
    from fskernels.hip.hf import custom_hf_decode_attention_forward, custom_hf_decode_attention_forward_fp8
    # triton_gqa_decode_hf.py:218-227, triton_gqa_decode_hf_fp8.py:230-239
    want = ["module", "query_states", "key_states", "value_states", "attention_mask", "scaling", "dropout"]
    assert positional(custom_hf_decode_attention_forward) == want
    assert positional(custom_hf_decode_attention_forward_fp8) == want


def test_engine_exports():
    from fskernels.engine import HIPGraphCache, HIPGraphRunner
    # cuda_graph_runner.py:113-120 (constructor), :141, :172, :226 (life cycle), :44-45, :57-58, :84
    assert positional(HIPGraphRunner)[:5] == ["model", "batch_size", "max_seq_len", "device", "num_splits"]
    assert positional(HIPGraphRunner.prefill) == ["self", "input_ids"]
    assert positional(HIPGraphRunner.build) == ["self", "warmup_steps"]
    assert positional(HIPGraphRunner.step) == ["self", "next_token"]
    assert positional(HIPGraphCache) == ["config", "max_batch_size", "max_cache_len", "device", "dtype"]
    assert positional(HIPGraphCache.update)[:4] == ["self", "key_states", "value_states", "layer_idx"]
    assert positional(HIPGraphCache.get_seq_length) == ["self", "layer_idx"]


def test_no_other_backend_is_shipped():
    """One HIP backend: no Triton, TileLang or CUDA decode modules."""
    import importlib.util
    for name in ("fskernels.triton", "fskernels.cuda", "fskernels.tilelang"):
        assert importlib.util.find_spec(name) is None, name
