"""Whole-model decode step in a HIP graph.

Reference: fskernels/engine/cuda_graph_runner.py (CUDAGraphCache :30-94,
CUDAGraphRunner :97-237).  Same API and life cycle: ``prefill`` runs the
prompt through the model with a dynamic cache and moves it into a static
cache; ``build`` warms up and captures one single-token forward; ``step``
writes the next token and the position into static device buffers and
replays.  The attention of the captured forward is the HIP decode patch
(fasterkernels_amd.hip.hf), installed for the capture; it reads the sequence
length from the ``cache_position`` device tensor the runner passes.

The static cache stores each step's new K/V rows with the HIP write kernel:
a dense [B, Hkv, S, D] cache is a paged pool of B pages of S rows, so the
rows of sequence b at position p go to slot b * S + p, one launch for K and V
per layer (the reference issues two index_copy_ per layer, :76-80).
"""
from __future__ import annotations

from typing import Optional

import torch

from ..hip.kv_write import paged_kv_write


def get_kv_from_hf_cache(cache, layer_idx: int):
    """(keys, values) of one layer from an HF cache object
    (cuda_graph_runner.py:5-27): ``cache.layers[i].keys/.values``,
    ``cache.key_cache[i]/.value_cache[i]`` or ``cache[i]``."""
    if hasattr(cache, "layers") and layer_idx < len(cache.layers):
        layer = cache.layers[layer_idx]
        if hasattr(layer, "keys") and hasattr(layer, "values"):
            return layer.keys, layer.values
    if hasattr(cache, "key_cache") and hasattr(cache, "value_cache"):
        return cache.key_cache[layer_idx], cache.value_cache[layer_idx]
    try:
        kv = cache[layer_idx]
        return kv[0], kv[1]
    except Exception:
        pass
    raise AttributeError(f"Could not extract K/V states from cache object of type {type(cache)}")


class HIPGraphCache:
    """Static KV cache [num_layers, B, Hkv, max_len, D] whose write position is
    a device tensor (``_pos``), so a captured forward stores each replay's
    token at the current position (cuda_graph_runner.py:30-94)."""

    def __init__(self, config, max_batch_size: int, max_cache_len: int, device, dtype: torch.dtype):
        nl, hkv, d = config.num_hidden_layers, config.num_key_value_heads, config.head_dim
        self.key_cache = torch.zeros(nl, max_batch_size, hkv, max_cache_len, d, dtype=dtype, device=device)
        self.value_cache = torch.zeros_like(self.key_cache)
        self._pos = torch.zeros(1, dtype=torch.long, device=device)
        self._num_layers = nl
        self._row0 = torch.arange(max_batch_size, dtype=torch.long, device=device) * max_cache_len

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int, cache_kwargs=None):
        """Stores key/value states [B, Hkv, L, D] at positions
        cache_position (from ``cache_kwargs``) or ``_pos + arange(L)``, and
        returns the layer's whole static K/V."""
        B, hkv, L, d = key_states.shape
        S = self.key_cache.shape[3]
        cache_position = None
        if isinstance(cache_kwargs, dict):
            cache_position = cache_kwargs.get("cache_position")
        elif cache_kwargs is not None:
            cache_position = getattr(cache_kwargs, "cache_position", None)
        if cache_position is None:
            cache_position = self._pos + torch.arange(L, device=key_states.device)
        slots = (self._row0[:B, None] + cache_position.view(1, L)).reshape(-1)
        k = key_states.transpose(1, 2).reshape(B * L, hkv, d)
        v = value_states.transpose(1, 2).reshape(B * L, hkv, d)
        kc, vc = self.key_cache[layer_idx], self.value_cache[layer_idx]
        # [B, Hkv, S, D] seen as a pool of B pages of S rows
        paged_kv_write(k, v, kc, vc, slots)
        return kc, vc

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return int(self._pos.item())

    def load_from_cache(self, cache, seq_len: int):
        """Copies a prefill's K/V (any HF cache type) into the static buffers."""
        for li in range(self._num_layers):
            k, v = get_kv_from_hf_cache(cache, li)
            self.key_cache[li, :, :, :seq_len, :] = k
            self.value_cache[li, :, :, :seq_len, :] = v


class HIPGraphRunner:
    """Captures the single-token decode forward of an HF causal LM as a HIP
    graph (cuda_graph_runner.py:97-237)::

        runner = HIPGraphRunner(model, batch_size=1, max_seq_len=2048)
        logits = runner.prefill(input_ids)     # dynamic cache, any length
        runner.build()                         # warm-up + capture
        for _ in range(n):
            logits = runner.step(next_token)   # graph replay

    The model must use eager attention (``attn_implementation="eager"``);
    ``build`` installs the HIP decode attention for the capture.  Sequences of
    a batch share one position, as in the reference.
    """

    def __init__(self, model, batch_size: int, max_seq_len: int, device="cuda", num_splits: int = 8,
                 fp8: bool = False):
        self.model = model
        self.batch_size = batch_size
        self.max_seq_len = max_seq_len
        self.device = device
        self.num_splits = num_splits
        self.fp8 = fp8
        self.kv_cache: Optional[HIPGraphCache] = None
        self._graph: Optional[torch.cuda.CUDAGraph] = None
        self._static_input_ids = self._static_cache_pos = self._static_pos_ids = None
        self._static_logits = None
        self._position = 0
        self._attn_mask_dict = {"full_attention": None}

    def prefill(self, input_ids: torch.Tensor) -> torch.Tensor:
        """Prompt pass with a dynamic cache, moved into the static cache;
        returns the last position's logits [B, vocab] (:141-167)."""
        bsz, seq_len = input_ids.shape
        if seq_len >= self.max_seq_len:
            raise ValueError(f"prompt of {seq_len} tokens does not fit max_seq_len={self.max_seq_len}")
        with torch.no_grad():
            out = self.model(input_ids=input_ids, past_key_values=None, use_cache=True, logits_to_keep=1)
        self.kv_cache = HIPGraphCache(self.model.config, bsz, self.max_seq_len, self.device, self.model.dtype)
        self.kv_cache.load_from_cache(out.past_key_values, seq_len)
        self._position = seq_len
        if getattr(self.model.model, "has_sliding_layers", False):
            self._attn_mask_dict["sliding_attention"] = None
        return out.logits[:, -1, :]

    def _forward(self):
        return self.model(input_ids=self._static_input_ids, position_ids=self._static_pos_ids,
                          cache_position=self._static_cache_pos, past_key_values=self.kv_cache,
                          attention_mask=self._attn_mask_dict, use_cache=True, logits_to_keep=1)

    def build(self, warmup_steps: int = 5):
        """Warm-up steps, then capture one step at the next position (:172-221)."""
        from ..hip.decode import set_num_splits
        from ..hip.hf import patched_hf_attention
        if self.kv_cache is None:
            raise RuntimeError("Call prefill() first")
        set_num_splits(self.num_splits)
        bsz, pos0 = self.batch_size, self._position
        if pos0 + warmup_steps + 1 > self.max_seq_len:
            raise ValueError("max_seq_len leaves no room for the warm-up and capture steps")
        self._static_input_ids = torch.zeros(bsz, 1, dtype=torch.long, device=self.device)
        self._static_cache_pos = torch.tensor([pos0], dtype=torch.long, device=self.device)
        self._static_pos_ids = torch.full((bsz, 1), pos0, dtype=torch.long, device=self.device)
        with patched_hf_attention(fp8=self.fp8), torch.no_grad():
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for i in range(warmup_steps):
                    self._sync_position(pos0 + i)
                    self._forward()
            torch.cuda.current_stream().wait_stream(side)
            self._sync_position(pos0 + warmup_steps)
            self._graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self._graph):
                out = self._forward()
        self._static_logits = out.logits
        torch.cuda.synchronize()
        self._position = pos0

    def step(self, next_token: torch.Tensor) -> torch.Tensor:
        """Writes the token and position, replays; returns logits [B, vocab] (:226-232)."""
        if self._graph is None:
            raise RuntimeError("Call build() before step()")
        if self._position >= self.max_seq_len:
            raise RuntimeError("the static cache is full")
        self._static_input_ids.copy_(next_token.view(self.batch_size, 1))
        self._sync_position(self._position)
        self._graph.replay()
        self._position += 1
        return self._static_logits[:, -1, :]

    def _sync_position(self, pos: int):
        self._static_cache_pos.fill_(pos)
        self._static_pos_ids.fill_(pos)
        self.kv_cache._pos.fill_(pos)
