"""HIP-graph capture of decode steps.

A decode step at serving batch sizes is a few microseconds of GPU work behind
tens of microseconds of host work (argument checks, ctypes, two or three
launches).  Capturing the step once and replaying it leaves one graph launch
per step.  The reference does this for a whole HF model
(fskernels/engine/cuda_graph_runner.py:97-237, see
fskernels.engine.HIPGraphRunner); this module does it for the decode
hot path itself:

* ``DecodeGraph`` captures any call of the decode / KV-write entry points.
  Inputs are read from the captured tensors at their fixed addresses, so the
  caller changes their contents in place between replays (query, lengths,
  block-table rows, new K/V rows, slots) and keeps shapes and dtypes fixed.
* ``PagedDecodeStep`` is the serving step for a fixed set of PagedKVCache
  sequences on one layer: store each sequence's new K/V row, then attend over
  the pages, in one graph, with the block table and lengths resident on the
  device.  Per step the host does the page bookkeeping and two small
  host-to-device copies.

Nothing here allocates during replay; workspaces and outputs come from the
graph's memory pool at capture time.
"""
from __future__ import annotations

from typing import Callable, List, Optional, Sequence

import torch

from ..hip.decode import paged_flash_decode
from ..hip.kv_write import paged_kv_write
from ..paged_attn.paged_kv_cache import PAGE_SIZE, PagedKVCache


class DecodeGraph:
    """Captures ``fn(*args, **kwargs)`` (after ``warmup`` eager calls on a side
    stream, as torch requires) and replays it.  ``output`` is the captured
    call's return value, rewritten by every replay."""

    def __init__(self, fn: Callable, *args, warmup: int = 1, **kwargs):
        self._call = lambda: fn(*args, **kwargs)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self._call()
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.output = self._call()

    def replay(self):
        self.graph.replay()
        return self.output


class PagedDecodeStep:
    """One captured decode step of a fixed batch of PagedKVCache sequences.

    Each ``step`` appends one token to every sequence (the same page
    bookkeeping as ``cache.append_kv`` per sequence, done on the host), then
    replays a graph that (1) stores the new K/V rows of layer ``layer_idx``
    and the new block-table entries with the write kernel and (2) runs the
    paged decode over the updated pages.  Write the step's inputs into
    ``q`` [B, Hq, D], ``k_new`` / ``v_new`` [B, Hkv, D] (or pass them to
    ``step``); the result is ``out`` [B, Hq, D].

    The block table is read from the cache's own device table (rows gathered
    for the batch inside the graph); slots and block-table stores (int64) and
    lengths (int32) reach the device in two small host-to-device copies per
    step.
    """

    def __init__(self, cache: PagedKVCache, layer_idx: int, seq_ids: Sequence[int], num_q_heads: int, *,
                 q_dtype: Optional[torch.dtype] = None, src_dtype: Optional[torch.dtype] = None,
                 out_dtype: Optional[torch.dtype] = None, s_aux: Optional[torch.Tensor] = None,
                 sink_mode: str = "linear"):
        cache._require_gpu()
        self.cache = cache
        self.layer = int(layer_idx)
        self.seq_ids: List[int] = list(seq_ids)
        B = len(self.seq_ids)
        if B == 0 or len(set(self.seq_ids)) != B:
            raise ValueError("seq_ids must be a non-empty list of distinct sequence slots")
        dev = cache.k_pool.device
        pool_dt = cache.dtype
        fp8 = pool_dt == torch.float8_e4m3fn
        qdt = q_dtype or (torch.bfloat16 if fp8 else pool_dt)
        sdt = src_dtype or qdt
        Hkv, D = cache.num_kv_heads, cache.head_dim
        self.q = torch.zeros(B, num_q_heads, D, dtype=qdt, device=dev)
        self.k_new = torch.zeros(B, Hkv, D, dtype=sdt, device=dev)
        self.v_new = torch.zeros_like(self.k_new)
        # device meta: slots [B] | block-table stores [B, 2] (int64), lengths [B] (int32)
        self._meta = torch.full((3 * B,), -1, dtype=torch.int64, device=dev)
        self._lens = torch.zeros(B, dtype=torch.int32, device=dev)
        self._rows = torch.tensor(self.seq_ids, dtype=torch.long, device=dev)
        slots = self._meta[:B]
        upd = self._meta[B:].view(B, 2)
        bt = cache.block_table
        kp, vp = cache.k_pool[self.layer], cache.v_pool[self.layer]
        ks, vs = cache.k_scale, cache.v_scale

        def step_fn():
            paged_kv_write(self.k_new, self.v_new, kp, vp, slots, k_scale=ks, v_scale=vs,
                           block_table=bt, bt_updates=upd)
            return paged_flash_decode(self.q, kp, vp, bt.index_select(0, self._rows), self._lens, PAGE_SIZE,
                                      s_aux=s_aux, k_scale=ks, v_scale=vs, out_dtype=out_dtype,
                                      sink_mode=sink_mode)

        # capture with every token skipped and no table stores: nothing changes
        self._graph = DecodeGraph(step_fn, warmup=1)
        self.out = self._graph.output

    def step(self, q: Optional[torch.Tensor] = None, k_new: Optional[torch.Tensor] = None,
             v_new: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Appends one token to every sequence and attends; returns ``out``."""
        if q is not None:
            self.q.copy_(q)
        if k_new is not None:
            self.k_new.copy_(k_new.reshape(self.k_new.shape))
        if v_new is not None:
            self.v_new.copy_(v_new.reshape(self.v_new.shape))
        B = len(self.seq_ids)
        slots, updates = self.cache._plan(self.seq_ids, 1)
        meta = slots + [-1] * (2 * B)
        for j, (flat, page) in enumerate(updates):
            meta[B + 2 * j] = flat
            meta[B + 2 * j + 1] = page
        lens = [self.cache._seq_lens[s] for s in self.seq_ids]
        # fresh pinned staging: torch's host allocator keeps it alive until the copy ran
        self._meta.copy_(torch.tensor(meta, dtype=torch.int64, pin_memory=True), non_blocking=True)
        self._lens.copy_(torch.tensor(lens, dtype=torch.int32, pin_memory=True), non_blocking=True)
        self._graph.replay()
        return self.out
