"""PagedKVCache host logic on CPU tensors (same API and state transitions as
fskernels/paged_attn/paged_kv_cache.py:6-154)."""
import types

import numpy as np
import pytest
import torch

from fasterkernels_amd.paged_attn import PAGE_SIZE, PagedKVCache
from oracle import decode_oracle as O


def make(num_pages=8, max_seqs=3, max_blocks=4, layers=2, hkv=2, d=8):
    return PagedKVCache(layers, num_pages, max_seqs, max_blocks, hkv, d, torch.float32, "cpu")


def kv(hkv=2, d=8, val=0.0):
    return torch.full((1, hkv, 1, d), val), torch.full((1, hkv, 1, d), -val)


def test_layout_and_init():
    c = make()
    assert PAGE_SIZE == 16
    assert c.k_pool.shape == (2, 8, 2, 16, 8) and c.v_pool.shape == c.k_pool.shape
    assert c.block_table.dtype == torch.int32 and (c.block_table == -1).all()
    assert c.pages_free == 8 and c.pages_used == 0
    assert repr(c) == "PagedKVCache(pages=8, used=0, seqs=0/3)"


def test_slots_lowest_first_and_exhaustion():
    c = make()
    assert [c.allocate_sequence() for _ in range(3)] == [0, 1, 2]
    with pytest.raises(RuntimeError, match="All sequence slots are occupied"):
        c.allocate_sequence()
    c.free_sequence(1)
    assert c.allocate_sequence() == 1


def test_append_allocates_pages_lifo_at_boundaries():
    c = make()
    s = c.allocate_sequence()
    for pos in range(33):
        k, v = kv(val=float(pos + 1))
        c.append_kv(s, 0, k, v)
    # pages come off the end of the free list: 7, 6, 5
    assert c.block_table[s, :4].tolist() == [7, 6, 5, -1]
    assert c.pages_used == 3
    assert c.get_seq_lens_tensor([s]).tolist() == [33]
    # token 17 lives in page block_table[s, 1] at row 1
    assert torch.equal(c.k_pool[0, 6, :, 1, :], torch.full((2, 8), 18.0))
    assert torch.equal(c.v_pool[0, 5, :, 0, :], torch.full((2, 8), -33.0))


def test_free_returns_pages_in_logical_order():
    c = make()
    s = c.allocate_sequence()
    for pos in range(20):
        c.append_kv(s, 0, *kv())
    c.free_sequence(s)
    assert (c.block_table[s] == -1).all()
    assert c.pages_free == 8
    # freed pages 7, 6 appended in logical order -> next allocation pops 6
    s2 = c.allocate_sequence()
    c.append_kv(s2, 0, *kv())
    assert c.block_table[s2, 0].item() == 6


def test_out_of_pages():
    c = make(num_pages=2)
    s = c.allocate_sequence()
    for pos in range(32):
        c.append_kv(s, 0, *kv())
    with pytest.raises(RuntimeError, match="Out of KV pages"):
        c.append_kv(s, 0, *kv())


def test_block_table_rows_and_lengths():
    c = make()
    a, b = c.allocate_sequence(), c.allocate_sequence()
    for _ in range(3):
        c.append_kv(a, 0, *kv())
    for _ in range(17):
        c.append_kv(b, 0, *kv())
    bt = c.get_block_table_tensor([b, a])
    assert bt.shape == (2, 4) and bt.dtype == torch.int32
    assert bt[0, :2].tolist() == c.block_table[b, :2].tolist()
    assert c.get_seq_lens_tensor([b, a]).tolist() == [17, 3]


def test_from_config_uses_bf16():
    cfg = types.SimpleNamespace(num_hidden_layers=3, num_key_value_heads=4, head_dim=64)
    c = PagedKVCache.from_config(cfg, num_pages=5, max_seqs=2, max_blocks_per_seq=3, device="cpu")
    assert c.k_pool.dtype == torch.bfloat16 and c.k_pool.shape == (3, 5, 4, 16, 64)


def test_cache_layout_decodes_like_dense_attention():
    """Tokens appended through the cache, read back with the oracle's paged
    addressing, give the same attention as the dense sequences."""
    g = torch.Generator().manual_seed(0)
    hkv, d, hq = 2, 16, 8
    c = make(num_pages=12, max_seqs=3, max_blocks=4, layers=1, hkv=hkv, d=d)
    lens = [5, 40, 17]
    dense_k, dense_v = [], []
    sids = [c.allocate_sequence() for _ in lens]
    for s, L in zip(sids, lens):
        ks = torch.randn(L, hkv, d, generator=g)
        vs = torch.randn(L, hkv, d, generator=g)
        for t in range(L):
            c.append_kv(s, 0, ks[t][None, :, None, :], vs[t][None, :, None, :])
        dense_k.append(ks.numpy())
        dense_v.append(vs.numpy())
    q = torch.randn(3, hq, d, generator=g).numpy()
    bt = c.get_block_table_tensor(sids).numpy()
    got = O.decode_paged(q, c.k_pool[0].numpy(), c.v_pool[0].numpy(), bt, lens)
    want = np.stack([O.attend(q[i], dense_k[i], dense_v[i]) for i in range(3)])
    assert np.allclose(got, want, atol=1e-12)
