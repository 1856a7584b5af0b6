"""Whole-model decode of an HF causal LM, one HIP-graph replay per token.

API of the reference's fskernels/engine/cuda_graph_runner.py (prefill /
build / step of CUDAGraphRunner, :97-237, and a static cache class), built
here from this package's own pieces:

* ``HIPGraphCache`` -- the static KV cache ``[layers, B, Hkv, S, D]``.  Its
  write position is one device int64 scalar, ``position``, the position of
  the token being decoded.  ``update`` stores the new K/V rows of a layer with
  the HIP write kernel, seeing the dense cache as a pool of B pages of S rows
  (row p of sequence b is slot ``b * S + p``), and hands the layer's whole
  cache to the attention.
* The decode step is a ``DecodeGraph``: the model's forward of a static
  token buffer at ``position`` (position ids and cache position are views of
  that scalar, so the forward reads it on the device), followed by
  ``position += 1`` inside the graph.  Consecutive replays therefore walk the
  cache with no host write of the position; the host keeps only a counter
  for the bounds check.  The captured attention is the HIP decode patch of
  ``fskernels.hip.hf``, which takes the sequence length from the cache
  position tensor.
* ``prefill`` runs the prompt with HF's own dynamic cache and stores its K/V
  rows into the static cache with one write-kernel launch per layer and
  sequence, reading the rows in place (no dense copies).

Sequences of a batch share one position (one query token each).
"""
from __future__ import annotations

from typing import Optional

import torch

from ..hip.kv_write import paged_kv_write
from .hip_graph import DecodeGraph


class HIPGraphCache:
    """Static KV cache whose write position lives on the device.

    ``key_cache`` / ``value_cache``: ``[num_layers, B, Hkv, max_cache_len, D]``.
    ``position``: int64 device scalar (shape ``[1]``), the position the next
    ``update`` without an explicit ``cache_position`` writes at.
    ``seq_length``: host count of the positions filled so far (kept by the
    caller; reading it never synchronises).
    """

    def __init__(self, config, max_batch_size: int, max_cache_len: int, device, dtype: torch.dtype):
        self.num_layers = int(config.num_hidden_layers)
        hkv, d = int(config.num_key_value_heads), int(config.head_dim)
        shape = (self.num_layers, max_batch_size, hkv, max_cache_len, d)
        self.key_cache = torch.zeros(shape, dtype=dtype, device=device)
        self.value_cache = torch.zeros_like(self.key_cache)
        self.position = torch.zeros(1, dtype=torch.long, device=device)
        self.seq_length = 0
        # slot of row 0 of each sequence: the cache row b of a layer is page b
        self._first_slot = torch.arange(max_batch_size, dtype=torch.long, device=device) * max_cache_len

    def _store(self, layer_idx: int, k_rows, v_rows, slots) -> None:
        """Rows ``[n, Hkv, D]`` (any token/head strides) to slots of the layer."""
        paged_kv_write(k_rows, v_rows, self.key_cache[layer_idx], self.value_cache[layer_idx], slots)

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int, cache_kwargs=None):
        """HF cache hook: stores ``[B, Hkv, L, D]`` states at ``cache_position``
        (from ``cache_kwargs``, else ``position + arange(L)``) and returns the
        layer's whole static K/V ``[B, Hkv, S, D]``."""
        B, hkv, L, d = key_states.shape
        pos = None
        if isinstance(cache_kwargs, dict):
            pos = cache_kwargs.get("cache_position")
        elif cache_kwargs is not None:
            pos = getattr(cache_kwargs, "cache_position", None)
        if pos is None:
            pos = self.position + torch.arange(L, device=key_states.device)
        slots = (self._first_slot[:B, None] + pos.view(1, L)).reshape(B * L)
        # [B, Hkv, L, D] -> [B*L, Hkv, D]: a view when L == 1 (the decode step)
        k = key_states.transpose(1, 2).reshape(B * L, hkv, d)
        v = value_states.transpose(1, 2).reshape(B * L, hkv, d)
        self._store(layer_idx, k, v, slots)
        return self.key_cache[layer_idx], self.value_cache[layer_idx]

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.seq_length

    def store_prompt(self, hf_cache, length: int) -> None:
        """Stores rows [0, length) of every layer of a filled HF cache (the
        ``layers[i].keys`` / ``.values`` of transformers' Cache, each
        ``[B, Hkv, >= length, D]``) and sets the position to ``length``."""
        layers = getattr(hf_cache, "layers", None)
        if layers is None or len(layers) < self.num_layers:
            raise TypeError(f"expected a transformers Cache with {self.num_layers} filled layers, "
                            f"got {type(hf_cache).__name__}")
        dev = self.key_cache.device
        rows = torch.arange(length, dtype=torch.long, device=dev)
        for i in range(self.num_layers):
            k, v = layers[i].keys, layers[i].values
            for b in range(k.shape[0]):
                # sequence b's rows as [L, Hkv, D]: token stride D, head stride L_cache * D
                self._store(i, k[b, :, :length].transpose(0, 1), v[b, :, :length].transpose(0, 1),
                            self._first_slot[b] + rows)
        self.position.fill_(length)
        self.seq_length = length


class HIPGraphRunner:
    """Greedy-decoding driver of an HF causal LM with one graph replay per token::

        runner = HIPGraphRunner(model, batch_size=1, max_seq_len=2048)
        logits = runner.prefill(input_ids)      # [B, vocab] of the last prompt token
        runner.build()                          # warm-up + capture of the decode step
        for _ in range(n):
            logits = runner.step(next_token)    # [B, vocab]

    The model must use eager attention (``attn_implementation="eager"``);
    ``build`` installs the HIP decode attention for the warm-up and capture
    and removes it afterwards (the graph keeps the captured kernels).
    ``num_splits`` is the split-count hint of the dense decode entry point.
    """

    def __init__(self, model, batch_size: int, max_seq_len: int, device="cuda", num_splits: int = 8,
                 fp8: bool = False):
        self.model = model
        self.batch_size = int(batch_size)
        self.max_seq_len = int(max_seq_len)
        self.device = torch.device(device)
        self.num_splits = int(num_splits)
        self.fp8 = bool(fp8)
        self.kv_cache: Optional[HIPGraphCache] = None
        self._graph: Optional[DecodeGraph] = None
        self._tokens: Optional[torch.Tensor] = None
        # every attention layer type of the model maps to "no mask": the
        # patched decode attention bounds each sequence by the cache position
        types = getattr(model.config, "layer_types", None) or ["full_attention"]
        self._no_masks = {t: None for t in set(types)}

    def prefill(self, input_ids: torch.Tensor) -> torch.Tensor:
        """Runs the prompt ``[B, L]``, stores its K/V in a fresh static cache
        and returns the last position's logits ``[B, vocab]``."""
        B, L = input_ids.shape
        if B != self.batch_size:
            raise ValueError(f"batch of {B} prompts, runner built for {self.batch_size}")
        if L >= self.max_seq_len:
            raise ValueError(f"prompt of {L} tokens leaves no room in max_seq_len={self.max_seq_len}")
        with torch.no_grad():
            out = self.model(input_ids=input_ids, use_cache=True, logits_to_keep=1)
        cache = HIPGraphCache(self.model.config, B, self.max_seq_len, self.device, self.model.dtype)
        cache.store_prompt(out.past_key_values, L)
        self.kv_cache = cache
        self._graph = None
        return out.logits[:, -1, :]

    def _decode_step(self):
        """Forward of ``_tokens`` at the device position, then position + 1."""
        pos = self.kv_cache.position
        out = self.model(input_ids=self._tokens, position_ids=pos.view(1, 1).expand(self.batch_size, 1),
                         cache_position=pos, past_key_values=self.kv_cache, attention_mask=self._no_masks,
                         use_cache=True, logits_to_keep=1)
        pos.add_(1)
        return out.logits

    def build(self, warmup_steps: int = 5):
        """Captures the decode step after ``warmup_steps`` eager ones.  The
        warm-up steps write rows past the prompt; the position is then set
        back, so the first ``step`` overwrites them before anything reads
        them (a step attends to positions up to its own)."""
        from ..hip.decode import set_num_splits
        from ..hip.hf import patched_hf_attention

        if self.kv_cache is None:
            raise RuntimeError("Call prefill() first")
        start = self.kv_cache.seq_length
        if start + max(warmup_steps, 1) + 1 > self.max_seq_len:
            raise ValueError("max_seq_len leaves no room for the warm-up steps")
        set_num_splits(self.num_splits)
        self._tokens = torch.zeros(self.batch_size, 1, dtype=torch.long, device=self.device)
        self.kv_cache.position.fill_(start)
        with patched_hf_attention(fp8=self.fp8), torch.no_grad():
            self._graph = DecodeGraph(self._decode_step, warmup=max(warmup_steps, 1))
        self.kv_cache.position.fill_(start)
        torch.cuda.synchronize()

    def step(self, next_token: torch.Tensor) -> torch.Tensor:
        """Decodes ``next_token`` ``[B]`` (or ``[B, 1]``) at the next position;
        returns its logits ``[B, vocab]``."""
        if self._graph is None:
            raise RuntimeError("Call build() before step()")
        if self.kv_cache.seq_length >= self.max_seq_len:
            raise RuntimeError("the static cache is full")
        self._tokens.copy_(next_token.view(self.batch_size, 1))
        logits = self._graph.replay()
        self.kv_cache.seq_length += 1
        return logits[:, -1, :]
