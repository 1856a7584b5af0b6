"""KV write path: store new tokens' K/V rows into paged pools on the GPU.

One launch of the gfx950 write kernel stores a batch of tokens (every KV head
of each) at precomputed slots, casting or quantising to the pool's element
type, and can apply block-table updates in the same launch.  It replaces the
per-token indexed copies of fskernels/paged_attn/paged_kv_cache.py:117-130.
"""
from __future__ import annotations

import torch

from fasterkernels_amd import native as nat
from .decode import _on_gpu

_SRC_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
_POOL_DTYPES = (torch.float16, torch.bfloat16, torch.float8_e4m3fn)


def _rows(t: torch.Tensor, name: str) -> torch.Tensor:
    """[n, Hkv, D] view of new K/V given as [n, Hkv, D] or [n, Hkv, 1, D]."""
    if t.dim() == 4:
        if t.shape[2] != 1:
            raise ValueError(f"{name} as [n, Hkv, 1, D] must have a single position, got {tuple(t.shape)}")
        t = t[:, :, 0, :]
    if t.dim() != 3:
        raise ValueError(f"{name} must be [n, Hkv, D] or [n, Hkv, 1, D], got {tuple(t.shape)}")
    if t.dtype not in _SRC_DTYPES:
        raise NotImplementedError(f"{name}: dtype {t.dtype} (f16, bf16 or f32 expected)")
    es = t.element_size()
    if t.stride(-1) != 1 or t.data_ptr() % 16 or any((s * es) % 16 for s in t.stride()[:-1]):
        t = t.contiguous()
    return t


def _scale(s, name: str, device: torch.device):
    if s is None:
        return None
    if not isinstance(s, torch.Tensor) or s.dtype != torch.float32 or s.numel() != 1:
        raise ValueError(f"{name} must be a one-element fp32 device tensor")
    _on_gpu(s, name, device)
    return s


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
    for t, name in ((k_pool, "k_pool"), (v_pool, "v_pool")):
        _on_gpu(t, name)
        if t.dim() != 4:
            raise ValueError(f"{name} must be [P, Hkv, page_size, D], got {tuple(t.shape)}")
        if t.dtype not in _POOL_DTYPES:
            raise NotImplementedError(f"{name}: dtype {t.dtype} (f16, bf16 or e4m3 expected)")
        if t.stride(-1) != 1:
            raise ValueError(f"{name} must have a contiguous head_dim")
    dev = k_pool.device
    if v_pool.get_device() != dev.index or v_pool.shape != k_pool.shape or v_pool.dtype != k_pool.dtype:
        raise ValueError("k_pool and v_pool must match in shape, dtype and device")
    P, Hkv, ps, D = k_pool.shape
    k = _rows(k, "k")
    v = _rows(v, "v")
    _on_gpu(k, "k", dev)
    _on_gpu(v, "v", dev)
    n = k.shape[0]
    if tuple(k.shape) != (n, Hkv, D) or tuple(v.shape) != (n, Hkv, D) or v.dtype != k.dtype:
        raise ValueError(f"k/v must be [{n}, {Hkv}, {D}] of one dtype, got {tuple(k.shape)} / {tuple(v.shape)}")
    _on_gpu(slot_mapping, "slot_mapping", dev)
    if slot_mapping.dtype != torch.int64 or slot_mapping.numel() != n:
        raise ValueError(f"slot_mapping must be int64 with {n} entries")
    if slot_mapping.dim() != 1 or not slot_mapping.is_contiguous():
        slot_mapping = slot_mapping.reshape(n).contiguous()
    ks = _scale(k_scale, "k_scale", dev)
    vs = _scale(v_scale, "v_scale", dev)
    bt_ptr, bt_numel, upd_ptr, n_upd = None, 0, None, 0
    if bt_updates is not None and bt_updates.numel():
        if block_table is None:
            raise ValueError("bt_updates need block_table")
        _on_gpu(block_table, "block_table", dev)
        _on_gpu(bt_updates, "bt_updates", dev)
        if block_table.dtype != torch.int32 or not block_table.is_contiguous():
            raise ValueError("block_table must be a contiguous int32 tensor")
        if bt_updates.dtype != torch.int64 or bt_updates.dim() != 2 or bt_updates.shape[1] != 2:
            raise ValueError("bt_updates must be int64 [m, 2]")
        bt_updates = bt_updates.contiguous()
        bt_ptr, bt_numel = block_table.data_ptr(), block_table.numel()
        upd_ptr, n_upd = bt_updates.data_ptr(), bt_updates.shape[0]
    lib = nat.load()
    ks_, vs_, kps, vps = k.stride(), v.stride(), k_pool.stride(), v_pool.stride()  # (one call each)
    st = nat.launch(
        dev.index, lib.fsk_paged_write,
        k.data_ptr(), ks_[0], ks_[1], v.data_ptr(), vs_[0], vs_[1],
        slot_mapping.data_ptr(), n,
        k_pool.data_ptr(), kps[0], kps[1], kps[2],
        v_pool.data_ptr(), vps[0], vps[1], vps[2],
        P, ps, Hkv, D, nat.DTYPE_CODES[k.dtype], nat.DTYPE_CODES[k_pool.dtype],
        nat.ptr(ks), nat.ptr(vs), bt_ptr, bt_numel, upd_ptr, n_upd, nat.stream_handle(dev))
    nat.check(st)
