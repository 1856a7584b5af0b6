"""Page-pool KV cache with the reference's API and memory layout.

Reference: fskernels/paged_attn/paged_kv_cache.py:6-154.  The layout is the
decode kernels' contract:

    k_pool / v_pool : [num_layers, num_pages, num_kv_heads, PAGE_SIZE, head_dim]
    block_table     : int32 [max_seqs, max_blocks_per_seq], -1 = unallocated

A sequence's token ``pos`` lives in page ``block_table[seq, pos // PAGE_SIZE]``
at row ``pos % PAGE_SIZE``; a page is taken from a LIFO free list when a
sequence reaches a page boundary.  The host keeps a mirror of every
sequence's page list, so no call reads the device block table back (the
reference does, with ``.item()``, at :96 and :126); the resulting state is
identical.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List

import torch

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
    """

    num_layers: int
    num_pages: int
    max_seqs: int
    max_blocks_per_seq: int
    num_kv_heads: int
    head_dim: int
    dtype: torch.dtype
    device: str

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
        return self._free_pages.pop()

    # ------------------------------------------------------------------
    def append_kv(self, seq_id: int, layer_idx: int, k: torch.Tensor, v: torch.Tensor):
        """Appends one token's K/V ([1, Hkv, 1, D]) to a sequence (:109-132).

        A new page is taken at every page boundary.  As in the reference, the
        sequence length advances on every call, so callers append each layer
        of a token through the same page bookkeeping.
        """
        pos = self._seq_lens[seq_id]
        page_idx = pos // PAGE_SIZE
        page_offset = pos % PAGE_SIZE
        if page_offset == 0:
            pp = self._alloc_page()
            self.block_table[seq_id, page_idx] = pp
            self._pages[seq_id].append(pp)
        else:
            pp = self._pages[seq_id][page_idx]
        self.k_pool[layer_idx, pp, :, page_offset, :] = k[0, :, 0, :]
        self.v_pool[layer_idx, pp, :, page_offset, :] = v[0, :, 0, :]
        self._seq_lens[seq_id] = pos + 1

    # ------------------------------------------------------------------
    def get_block_table_tensor(self, active_seq_ids: List[int]) -> torch.Tensor:
        """Rows of the block table for the given sequences, [n, max_blocks] (:135-137)."""
        idx = torch.tensor(active_seq_ids, dtype=torch.long, device=self.device)
        return self.block_table[idx]

    def get_seq_lens_tensor(self, active_seq_ids: List[int]) -> torch.Tensor:
        """int32 [n] lengths on the cache's device (:139-141)."""
        lens = [self._seq_lens[sid] for sid in active_seq_ids]
        return torch.tensor(lens, dtype=torch.int32, device=self.device)

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
