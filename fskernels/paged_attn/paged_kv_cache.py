"""Page-pool KV cache with the reference's API and memory layout.

Reference: fskernels/paged_attn/paged_kv_cache.py:6-154.  The layout is the
decode kernels' contract:

    k_pool / v_pool : [num_layers, num_pages, num_kv_heads, PAGE_SIZE, head_dim]
    block_table     : int32 [max_seqs, max_blocks_per_seq], -1 = unallocated

A sequence's token ``pos`` lives in page ``block_table[seq, pos // PAGE_SIZE]``
at row ``pos % PAGE_SIZE``; a page is taken from a LIFO free list when a
sequence reaches a page boundary.

Page bookkeeping stays on the host, as in the reference, with a host mirror of
every sequence's page list, so no call reads the device block table back (the
reference does, with ``.item()``, at :96 and :126).  On a GPU the rows are
stored by the gfx950 write kernel: one launch per call stores every token of a
batch and the new block-table entries together.  Like the reference's, the
cache can also be built in host memory (``device="cpu"``, e.g. for a cache
kept off the GPU); its rows are then stored with the reference's indexed
assignment (:128-130) on the host.  That is where the pools live, chosen at
construction, not a substitute for the kernel: GPU pools are only ever
written by the kernel, and the decode entry points reject host pools.  e4m3
pools (``dtype=torch.float8_e4m3fn``) can carry per-tensor
``k_scale``/``v_scale``; rows are then quantised on the way in
(``e4m3(clamp(x / scale, -448, 448))``, the same codes on both devices).
"""
from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import torch

from ..hip.kv_write import paged_kv_write

PAGE_SIZE = 16  # tokens per physical page


@dataclass
class PagedKVCache:
    """Pool of physical KV pages shared by all concurrent sequences.

    Usage::

        cache = PagedKVCache(num_layers, num_pages, max_seqs, max_blocks_per_seq,
                             num_kv_heads, head_dim, torch.float16, "cuda")
        sid = cache.allocate_sequence()
        cache.append_kv(sid, layer, k, v)          # k, v: [1, Hkv, 1, D]
        out = paged_flash_decode(q, cache.k_pool[layer], cache.v_pool[layer],
                                 cache.get_block_table_tensor([sid]),
                                 cache.get_seq_lens_tensor([sid]), PAGE_SIZE)
        cache.free_sequence(sid)

    Batched forms (no reference counterpart): ``append_kv_batch`` stores one
    token for each of several sequences in one launch; ``reserve_slots`` +
    ``write_kv`` take the slots of a step once and store every layer's rows
    with one launch each.
    """

    num_layers: int
    num_pages: int
    max_seqs: int
    max_blocks_per_seq: int
    num_kv_heads: int
    head_dim: int
    dtype: torch.dtype
    device: str
    k_scale: Optional[object] = None  # e4m3 pools: per-tensor scale (float or fp32 tensor)
    v_scale: Optional[object] = None

    def __post_init__(self):
        # One pool per layer for K and for V (paged_kv_cache.py:46-50).
        self.k_pool = torch.zeros(self.num_layers, self.num_pages, self.num_kv_heads, PAGE_SIZE,
                                  self.head_dim, dtype=self.dtype, device=self.device)
        self.v_pool = torch.zeros_like(self.k_pool)
        # Logical -> physical page map, -1 = unallocated (:53-56).
        self.block_table = torch.full((self.max_seqs, self.max_blocks_per_seq), -1,
                                      dtype=torch.int32, device=self.device)
        # Host-side metadata (:59-61) plus the host mirror of block_table rows.
        self._seq_lens: List[int] = [0] * self.max_seqs
        self._active: List[bool] = [False] * self.max_seqs
        self._free_pages: List[int] = list(range(self.num_pages))
        self._pages: List[List[int]] = [[] for _ in range(self.max_seqs)]
        self._journal = None  # (pages popped, {seq: (old length, old page count)}) of the call in progress
        if (self.k_scale is None) != (self.v_scale is None):
            raise ValueError("give both k_scale and v_scale or neither")
        if self.k_scale is not None:
            if self.dtype != torch.float8_e4m3fn:
                raise ValueError("k_scale/v_scale apply to float8_e4m3fn pools only")
            self.k_scale = torch.as_tensor(self.k_scale, dtype=torch.float32).reshape(()).to(self.k_pool.device)
            self.v_scale = torch.as_tensor(self.v_scale, dtype=torch.float32).reshape(()).to(self.k_pool.device)

    @classmethod
    def from_config(cls, config, num_pages: int = 4096, max_seqs: int = 16,
                    max_blocks_per_seq: int = 512, device: str = "cuda") -> "PagedKVCache":
        """Sized from an HF config; bf16 pools as in paged_kv_cache.py:64-82."""
        return cls(num_layers=config.num_hidden_layers, num_pages=num_pages, max_seqs=max_seqs,
                   max_blocks_per_seq=max_blocks_per_seq,
                   num_kv_heads=config.num_key_value_heads, head_dim=config.head_dim,
                   dtype=torch.bfloat16, device=device)

    # ------------------------------------------------------------------
    def allocate_sequence(self) -> int:
        """Lowest free slot id; RuntimeError when all are active (:85-91)."""
        for sid in range(self.max_seqs):
            if not self._active[sid]:
                self._active[sid] = True
                self._seq_lens[sid] = 0
                self._pages[sid] = []
                return sid
        raise RuntimeError("All sequence slots are occupied")

    def free_sequence(self, seq_id: int):
        """Returns the sequence's pages to the free list in logical order (:93-101)."""
        pages = self._pages[seq_id]
        n_pages = (self._seq_lens[seq_id] + PAGE_SIZE - 1) // PAGE_SIZE
        for lp in range(n_pages):
            pp = pages[lp] if lp < len(pages) else -1
            if pp >= 0:
                self._free_pages.append(pp)
        if n_pages:
            self.block_table[seq_id, :n_pages] = -1
        self._pages[seq_id] = []
        self._active[seq_id] = False
        self._seq_lens[seq_id] = 0

    def _alloc_page(self) -> int:
        if not self._free_pages:
            raise RuntimeError("Out of KV pages")
        pp = self._free_pages.pop()
        if self._journal is not None:
            self._journal[0].append(pp)
        return pp

    # ------------------------------------------------------------------
    def _plan(self, seq_ids: Sequence[int], num_tokens: int = 1) -> Tuple[List[int], List[Tuple[int, int]]]:
        """Host bookkeeping of appending ``num_tokens`` tokens to each listed
        sequence, in list order (a repeated id appends again, as repeated
        append_kv calls would).  Returns the slots (page * PAGE_SIZE + row,
        sequence-major) and the block-table stores (flat index, page).  All or
        nothing: a call that would run out of pages or past a block-table row
        raises before any state changes."""
        lens = {}
        need = 0
        for sid in seq_ids:
            pos = lens.get(sid, self._seq_lens[sid])
            end = pos + num_tokens
            if -(-end // PAGE_SIZE) > self.max_blocks_per_seq:
                raise IndexError(f"sequence {sid} would need more than max_blocks_per_seq="
                                 f"{self.max_blocks_per_seq} pages")
            need += -(-end // PAGE_SIZE) - -(-pos // PAGE_SIZE)
            lens[sid] = end
        if need > len(self._free_pages):
            raise RuntimeError("Out of KV pages")
        row_stride = self.block_table.stride(0)
        slots: List[int] = []
        updates: List[Tuple[int, int]] = []
        touched = self._journal[1] if self._journal is not None else None
        for sid in seq_ids:
            pages = self._pages[sid]
            pos = self._seq_lens[sid]
            if touched is not None and sid not in touched:
                touched[sid] = (pos, len(pages))
            for _ in range(num_tokens):
                lp, off = divmod(pos, PAGE_SIZE)
                if off == 0:
                    pp = self._alloc_page()
                    pages.append(pp)
                    updates.append((sid * row_stride + lp, pp))
                else:
                    pp = pages[lp]
                slots.append(pp * PAGE_SIZE + off)
                pos += 1
            self._seq_lens[sid] = pos
        return slots, updates

    def _require_gpu(self):
        if not self.k_pool.is_cuda:
            raise RuntimeError("this needs the cache's pools on a GPU (HIP) device; "
                               f"they are on {self.k_pool.device}, not a GPU")

    def _new_rows(self, t, name: str, n: int) -> torch.Tensor:
        """New K or V rows for ``n`` tokens, checked before any bookkeeping
        changes, on the pools' device: rows on another device (the CPU
        included) are copied there, as the reference's indexed store copies
        them (paged_kv_cache.py:128-130)."""
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if t.dim() == 4 and t.shape[2] == 1:
            rows = t.shape[0], t.shape[1], t.shape[3]
        elif t.dim() == 3:
            rows = tuple(t.shape)
        else:
            raise ValueError(f"{name} must be [n, Hkv, 1, D] or [n, Hkv, D], got {tuple(t.shape)}")
        if rows != (n, self.num_kv_heads, self.head_dim):
            raise ValueError(f"{name} holds {tuple(t.shape)} for {n} tokens of "
                             f"{self.num_kv_heads} heads x {self.head_dim}")
        if t.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise NotImplementedError(f"{name}: dtype {t.dtype} (f16, bf16 or f32 expected)")
        if t.device != self.k_pool.device:
            t = t.to(self.k_pool.device)
        return t

    @contextmanager
    def _all_or_nothing(self):
        """Restores the host bookkeeping (lengths, page lists, free list) if
        the body raises: planning, staging and the launch succeed together or
        leave no trace.  (The block-table stores ride the write launch, so a
        call that fails before or at the launch has stored none.)  _plan
        journals what it changes (the pages it pops, in order, and each
        touched sequence's old length and page count), so the cost is that of
        the call's own tokens, not of the pool or the batch."""
        journal = ([], {})
        self._journal = journal
        try:
            yield
        except BaseException:
            popped, touched = journal
            for sid, (length, n_pages) in touched.items():
                self._seq_lens[sid] = length
                del self._pages[sid][n_pages:]
            self._free_pages.extend(reversed(popped))
            raise
        finally:
            self._journal = None

    def _stage(self, slots, updates):
        """The slots and block-table stores as one int64 tensor on the pools'
        device (one host->device copy for GPU pools)."""
        vals = list(slots)
        for flat, page in updates:
            vals += (flat, page)
        if self.k_pool.is_cuda:
            host = torch.tensor(vals, dtype=torch.int64, pin_memory=True)
            dev = host.to(self.k_pool.device, non_blocking=True)
        else:
            dev = torch.tensor(vals, dtype=torch.int64)
        n = len(slots)
        return dev[:n], dev[n:].view(-1, 2)

    def _write(self, layer_idx, k, v, slot_dev, upd_dev):
        if self.k_pool.is_cuda:
            paged_kv_write(k, v, self.k_pool[layer_idx], self.v_pool[layer_idx], slot_dev,
                           k_scale=self.k_scale, v_scale=self.v_scale,
                           block_table=self.block_table, bt_updates=upd_dev)
        else:
            self._write_host(layer_idx, k, v, slot_dev, upd_dev)

    def _write_host(self, layer_idx, k, v, slots, upd=None):
        """Host-memory pools: the reference's block-table store and indexed
        row stores (paged_kv_cache.py:122-130) for every token at once, with
        the write kernel's rules (slots outside the pool are skipped; e4m3
        pools with scales store e4m3(clamp(x / scale, -448, 448)))."""
        if upd is not None and upd.numel():
            self.block_table.view(-1)[upd[:, 0]] = upd[:, 1].to(torch.int32)
        n = slots.numel()
        if n == 0:
            return
        slots = slots.reshape(n).to(torch.int64)
        ok = (slots >= 0) & (slots < self.num_pages * PAGE_SIZE)
        pages, rows = slots[ok] // PAGE_SIZE, slots[ok] % PAGE_SIZE
        for pool, x, scale in ((self.k_pool[layer_idx], k, self.k_scale), (self.v_pool[layer_idx], v, self.v_scale)):
            x = x.reshape(n, self.num_kv_heads, self.head_dim)[ok]
            if scale is not None:
                x = (x.to(torch.float32) / scale).clamp(-448.0, 448.0)
            pool[pages, :, rows, :] = x.to(pool.dtype)

    # ------------------------------------------------------------------
    def append_kv(self, seq_id: int, layer_idx: int, k: torch.Tensor, v: torch.Tensor):
        """Appends one token's K/V ([1, Hkv, 1, D]) to a sequence (:109-132).

        A new page is taken at every page boundary.  As in the reference, the
        sequence length advances on every call, so callers append each layer
        of a token through the same page bookkeeping.
        """
        self.append_kv_batch([seq_id], layer_idx, k, v)

    def append_kv_batch(self, seq_ids: Sequence[int], layer_idx: int, k: torch.Tensor, v: torch.Tensor):
        """append_kv for several tokens in one launch: token j of k/v
        ([n, Hkv, 1, D] or [n, Hkv, D]) goes to sequence seq_ids[j]; the
        bookkeeping is that of n append_kv calls in order."""
        n = len(seq_ids)
        k = self._new_rows(k, "k", n)
        v = self._new_rows(v, "v", n)
        if v.dtype != k.dtype:
            raise ValueError(f"k and v dtypes differ: {k.dtype} / {v.dtype}")
        with self._all_or_nothing():
            slots, updates = self._plan(list(seq_ids), 1)
            slot_dev, upd_dev = self._stage(slots, updates)
            self._write(layer_idx, k, v, slot_dev, upd_dev)

    def reserve_slots(self, seq_ids: Sequence[int], num_tokens: int = 1) -> torch.Tensor:
        """Takes ``num_tokens`` new positions in each listed sequence (pages as
        needed, block table stored on the device) and returns their slots, an
        int64 device tensor [len(seq_ids) * num_tokens], sequence-major, for
        ``write_kv`` of every layer (a host tensor for host pools)."""
        with self._all_or_nothing():
            slots, updates = self._plan(list(seq_ids), int(num_tokens))
            slot_dev, upd_dev = self._stage(slots, updates)
            if updates:
                empty = self.k_pool.new_empty((0, self.num_kv_heads, self.head_dim), dtype=torch.float32)
                self._write(0, empty, empty, slot_dev[:0], upd_dev)
        return slot_dev

    def write_kv(self, layer_idx: int, k: torch.Tensor, v: torch.Tensor, slot_mapping: torch.Tensor):
        """Stores rows k/v ([n, Hkv, D], any strides with a contiguous head_dim,
        or [n, Hkv, 1, D]) of one layer at slots from ``reserve_slots``."""
        if self.k_pool.is_cuda:
            paged_kv_write(k, v, self.k_pool[layer_idx], self.v_pool[layer_idx], slot_mapping,
                           k_scale=self.k_scale, v_scale=self.v_scale)
        else:
            n = slot_mapping.numel()
            k = self._new_rows(k, "k", n)
            v = self._new_rows(v, "v", n)
            self._write_host(layer_idx, k, v, slot_mapping.to(self.k_pool.device))

    # ------------------------------------------------------------------
    def get_block_table_tensor(self, active_seq_ids: List[int]) -> torch.Tensor:
        """Rows of the block table for the given sequences, [n, max_blocks] (:135-137)."""
        idx = torch.tensor(active_seq_ids, dtype=torch.long, device=self.device)
        return self.block_table[idx]

    def get_seq_lens_tensor(self, active_seq_ids: List[int], *, device=None) -> torch.Tensor:
        """int32 [n] lengths on the cache's device (:139-141), or on ``device``
        (keyword-only addition): ``device="cpu"`` gives host lengths, which
        ``paged_flash_decode`` takes as they are and builds its work plan
        from on the host, with no copy to the GPU."""
        lens = [self._seq_lens[sid] for sid in active_seq_ids]
        return torch.tensor(lens, dtype=torch.int32, device=self.device if device is None else device)

    # ------------------------------------------------------------------
    @property
    def pages_used(self) -> int:
        return self.num_pages - len(self._free_pages)

    @property
    def pages_free(self) -> int:
        return len(self._free_pages)

    def __repr__(self) -> str:
        return (f"PagedKVCache(pages={self.num_pages}, used={self.pages_used}, "
                f"seqs={sum(self._active)}/{self.max_seqs})")
