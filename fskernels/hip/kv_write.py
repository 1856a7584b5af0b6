"""KV write path: store new tokens' K/V rows into paged pools on the GPU.

One launch of the gfx950 write kernel stores a batch of tokens (every KV head
of each) at precomputed slots, casting or quantising to the pool's element
type, and can apply block-table updates in the same launch.  It replaces the
per-token indexed copies of fskernels/paged_attn/paged_kv_cache.py:117-130.
The checks and the launch are one call of the torch binding
(fasterkernels_amd/csrc/fsk_torch.cpp).
"""
from __future__ import annotations

import torch

from fasterkernels_amd import native as nat


def paged_kv_write(k: torch.Tensor, v: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                   slot_mapping: torch.Tensor, *, k_scale: torch.Tensor | None = None,
                   v_scale: torch.Tensor | None = None, block_table: torch.Tensor | None = None,
                   bt_updates: torch.Tensor | None = None) -> None:
    """Writes token i of ``k``/``v`` ([n, Hkv, D] or [n, Hkv, 1, D]) into page
    ``slot_mapping[i] // page_size``, row ``slot_mapping[i] % page_size`` of
    ``k_pool``/``v_pool`` ([P, Hkv, page_size, D]).

    ``slot_mapping`` is an int64 device tensor; negative slots skip a token.
    f16/bf16 pools take a copy (round-to-nearest-even cast across types).
    e4m3 pools with ``k_scale``/``v_scale`` (one-element fp32 device tensors)
    store e4m3(clamp(x / scale, +-448)); without scales a plain e4m3 cast.
    ``bt_updates`` (int64 [m, 2] of (flat index, page)) are stored into the
    int32 ``block_table`` in the same launch.  Enqueued on the current stream.
    """
    if not isinstance(k_pool, torch.Tensor):
        raise TypeError("k_pool must be a torch.Tensor")
    index = k_pool.get_device()
    nat.ext().kv_write(k, v, k_pool, v_pool, slot_mapping, k_scale, v_scale, block_table, bt_updates,
                       nat.raw_stream(index) if index >= 0 else 0)
