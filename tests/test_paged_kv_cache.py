"""PagedKVCache host logic on the CPU: page bookkeeping, block-table stores and
slots, against the oracle's restatement of fskernels/paged_attn/paged_kv_cache.py
(RefPagedKVCache), and caches built in host memory, whose rows are stored on
the host (GPU pools are written by the HIP write kernel: the GPU tests)."""
import random
import types

import numpy as np
import pytest
import torch

from fskernels.paged_attn import PAGE_SIZE, PagedKVCache
from oracle import decode_oracle as O


def make(num_pages=8, max_seqs=3, max_blocks=4, layers=2, hkv=2, d=8, dtype=torch.float16):
    return PagedKVCache(layers, num_pages, max_seqs, max_blocks, hkv, d, dtype, "cpu")


def bt_after(cache, updates):
    """The block table the device would hold after the planned stores."""
    bt = cache.block_table.clone().view(-1)
    for flat, page in updates:
        bt[flat] = page
    cache.block_table.copy_(bt.view_as(cache.block_table))
    return cache.block_table


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


def test_plan_matches_reference_bookkeeping():
    """One token at a time: the same pages, block table and lengths as the
    reference's append_kv, and slots that address the reference's rows."""
    c = make()
    ref = O.RefPagedKVCache(1, 8, 3, 4, 2, 8, "f16")
    s = c.allocate_sequence()
    assert ref.allocate_sequence() == s
    for pos in range(33):
        slots, upd = c._plan([s])
        ref.append_kv(s, 0, np.zeros((2, 8), np.float32), np.zeros((2, 8), np.float32))
        bt_after(c, upd)
        page = ref.block_table[s, pos // 16]
        assert slots == [page * 16 + pos % 16]
    assert c.block_table[s].tolist() == ref.block_table[s].tolist() == [7, 6, 5, -1]
    assert c.get_seq_lens_tensor([s]).tolist() == [33]
    host = c.get_seq_lens_tensor([s], device="cpu")
    assert host.device.type == "cpu" and host.dtype == torch.int32 and host.tolist() == [33]
    assert c.pages_used == 3


def test_free_returns_pages_in_logical_order():
    c = make()
    s = c.allocate_sequence()
    bt_after(c, c._plan([s], 20)[1])
    c.free_sequence(s)
    assert (c.block_table[s] == -1).all()
    assert c.pages_free == 8
    s2 = c.allocate_sequence()
    slots, upd = c._plan([s2])
    assert upd == [(s2 * 4 + 0, 6)] and slots == [6 * 16]   # freed 7, 6 in logical order -> pops 6


def test_out_of_pages_is_all_or_nothing():
    c = make(num_pages=2)
    s = c.allocate_sequence()
    c._plan([s], 32)
    with pytest.raises(RuntimeError, match="Out of KV pages"):
        c._plan([s])
    assert c._seq_lens[s] == 32 and c.pages_free == 0
    # a batch that needs more pages than are free changes nothing
    c2 = make(num_pages=3)
    a, b = c2.allocate_sequence(), c2.allocate_sequence()
    with pytest.raises(RuntimeError, match="Out of KV pages"):
        c2._plan([a, b], 17)          # 2 + 2 pages
    assert c2.pages_free == 3 and c2._seq_lens[a] == c2._seq_lens[b] == 0


def test_block_table_width_is_checked_before_any_change():
    c = make(num_pages=16, max_blocks=2)
    s = c.allocate_sequence()
    with pytest.raises(IndexError):
        c._plan([s], 33)
    assert c.pages_free == 16 and c._seq_lens[s] == 0


def test_random_batches_match_per_token_reference():
    """Batched plans (repeated ids, multi-token reservations, frees) give the
    state a sequence of reference append_kv calls gives."""
    rnd = random.Random(7)
    for trial in range(20):
        P, S, MB = 40, 5, 6
        c = make(num_pages=P, max_seqs=S, max_blocks=MB, layers=1)
        ref = O.RefPagedKVCache(1, P, S, MB, 2, 8, "f16")
        live = []
        for step in range(30):
            op = rnd.random()
            if op < 0.15 and len(live) < S:
                sid = c.allocate_sequence()
                assert ref.allocate_sequence() == sid
                live.append(sid)
            elif op < 0.25 and live:
                sid = live.pop(rnd.randrange(len(live)))
                c.free_sequence(sid)
                ref.free_sequence(sid)
            elif live:
                ids = [rnd.choice(live) for _ in range(rnd.randint(1, 4))]
                n_tok = rnd.choice([1, 1, 3, 17])
                total_after = {i: ref.seq_lens[i] + n_tok * ids.count(i) for i in set(ids)}
                need = sum(-(-total_after[i] // 16) - -(-ref.seq_lens[i] // 16) for i in set(ids))
                if need > len(ref.free_pages) or max(-(-v // 16) for v in total_after.values()) > MB:
                    with pytest.raises((RuntimeError, IndexError)):
                        c._plan(ids, n_tok)
                    continue
                slots, upd = c._plan(ids, n_tok)
                bt_after(c, upd)
                want = []
                for i in ids:
                    for _ in range(n_tok):
                        pos = ref.seq_lens[i]
                        ref.append_kv(i, 0, np.zeros((2, 8), np.float32), np.zeros((2, 8), np.float32))
                        want.append(int(ref.block_table[i, pos // 16]) * 16 + pos % 16)
                assert slots == want
            assert c.block_table.numpy().tolist() == ref.block_table.tolist()
            assert c._seq_lens == ref.seq_lens and c._free_pages == ref.free_pages


def test_planned_slots_decode_like_dense_attention():
    """Rows stored at the planned slots (oracle store) and read back with the
    oracle's paged addressing give the dense sequences' attention."""
    g = np.random.default_rng(0)
    hkv, d, hq = 2, 16, 8
    c = make(num_pages=12, max_seqs=3, max_blocks=4, layers=1, hkv=hkv, d=d)
    lens = [5, 40, 17]
    sids = [c.allocate_sequence() for _ in lens]
    pool_k = np.zeros((12, hkv, 16, d), np.float16)
    pool_v = np.zeros_like(pool_k)
    dense = []
    for s, L in zip(sids, lens):
        ks = g.standard_normal((L, hkv, d)).astype(np.float16).astype(np.float32)
        vs = g.standard_normal((L, hkv, d)).astype(np.float16).astype(np.float32)
        slots, upd = c._plan([s], L)
        bt_after(c, upd)
        O.paged_write(pool_k, slots, ks, "f16")
        O.paged_write(pool_v, slots, vs, "f16")
        dense.append((ks, vs))
    q = g.standard_normal((3, hq, d))
    bt = c.get_block_table_tensor(sids).numpy()
    got = O.decode_paged(q, pool_k.astype(np.float32), pool_v.astype(np.float32), bt, lens)
    want = np.stack([O.attend(q[i], *dense[i]) for i in range(3)])
    assert np.allclose(got, want, atol=1e-12)


@pytest.mark.parametrize("pool,src", [("f16", "f16"), ("bf16", "bf16"), ("f16", "f32"), ("bf16", "f16"),
                                      ("e4m3", "bf16"), ("e4m3", "f32")])
def test_host_pools_match_reference_cache(pool, src):
    """A cache built in host memory (device="cpu", which the reference's
    cache allows) stores its rows on the host: driven by the same random
    allocate / append / batch-append / reserve+write / free script as the GPU
    test, it ends bit-identical to the oracle's restatement of the reference
    cache (e4m3 pools with fixed scales quantise as the reference's
    quantiser does)."""
    import random
    from tests.test_gpu_kv_write import POOL, SRC, compare, run_cache_script
    rnd = random.Random(6)
    gen = torch.Generator().manual_seed(6)
    L, P, S, MB, hkv, d = 2, 64, 4, 16, 2, 32
    scales = dict(k_scale=0.03, v_scale=0.02) if pool == "e4m3" else {}
    cache = PagedKVCache(L, P, S, MB, hkv, d, POOL[pool], "cpu", **scales)
    ref = O.RefPagedKVCache(L, P, S, MB, hkv, d, pool,
                            np.float32(0.03) if scales else None, np.float32(0.02) if scales else None)
    run_cache_script(cache, ref, rnd, 80, L, SRC[src], gen, dev="cpu")
    compare(cache.k_pool, ref.k_pool, pool, src, "k_pool")
    compare(cache.v_pool, ref.v_pool, pool, src, "v_pool")


def test_host_pools_skip_out_of_range_slots_and_reject_decode():
    """write_kv on host pools follows the write kernel's rule (a negative slot
    or one past the pool is skipped), and the decode entry points refuse host
    pools (no decode runs on the host)."""
    from fskernels.paged_attn import paged_flash_decode
    c = make(num_pages=2)
    x = torch.arange(3 * 2 * 8, dtype=torch.float32).view(3, 2, 8)
    c.write_kv(1, x, -x, torch.tensor([-1, 2 * 16, 17]))
    assert torch.equal(c.k_pool[1, 1, :, 1], x[2].half()) and torch.equal(c.v_pool[1, 1, :, 1], -x[2].half())
    c.k_pool[1, 1, :, 1] = 0
    assert (c.k_pool == 0).all()
    s = c.allocate_sequence()
    c.append_kv(s, 0, torch.ones(1, 2, 1, 8), torch.ones(1, 2, 1, 8))
    q = torch.zeros(1, 4, 8, dtype=torch.float16)
    with pytest.raises(RuntimeError):
        paged_flash_decode(q, c.k_pool[0], c.v_pool[0], c.get_block_table_tensor([s]), c.get_seq_lens_tensor([s]),
                           PAGE_SIZE)


def test_failed_call_restores_only_what_it_touched(monkeypatch):
    """The rollback journal: a failed reservation puts back exactly the pages
    it popped, in free-list order, and the lengths and page lists of the
    sequences it touched, leaving the others alone."""
    c = make(num_pages=8, max_seqs=3, max_blocks=4)
    a, b, z = c.allocate_sequence(), c.allocate_sequence(), c.allocate_sequence()
    c.reserve_slots([a], 20)     # pages 7, 6
    c.reserve_slots([z], 3)      # page 5
    before = _host_state(c)

    def boom(*args, **kw):
        raise RuntimeError("stage failed")
    monkeypatch.setattr(c, "_stage", boom)
    with pytest.raises(RuntimeError, match="stage failed"):
        c.reserve_slots([b, a, b], 13)    # pops 4 (b), 3 (a: 20 -> 33), 2 (b: 13 -> 26)
    after = _host_state(c)
    assert after[:3] == before[:3] and torch.equal(after[3], before[3])
    assert c._journal is None


def _host_state(c):
    return list(c._seq_lens), [list(p) for p in c._pages], list(c._free_pages), c.block_table.clone()


@pytest.mark.parametrize("fail_at", ["_stage", "_write"])
def test_failed_append_leaves_no_trace(monkeypatch, fail_at):
    """An append or reservation whose staging or launch fails restores the
    lengths, page lists and free list (the block-table stores ride the failed
    launch, so the device table is untouched too).  The GPU-only steps are
    stood in for by host functions here; one of them raises."""
    c = make()
    s0, s1 = c.allocate_sequence(), c.allocate_sequence()
    monkeypatch.setattr(c, "_require_gpu", lambda: None)
    monkeypatch.setattr(c, "_stage", lambda slots, upd: (torch.tensor(slots), torch.tensor(upd).view(-1, 2)))
    monkeypatch.setattr(c, "_write", lambda *a: None)
    k = torch.zeros(2, 2, 1, 8, dtype=torch.float16)
    c.append_kv_batch([s0, s1], 0, k, k)          # one page each
    c.reserve_slots([s0], 20)                      # crosses into a second page
    before = _host_state(c)

    def boom(*a, **kw):
        raise RuntimeError("launch failed")
    monkeypatch.setattr(c, fail_at, boom)
    with pytest.raises(RuntimeError, match="launch failed"):
        c.append_kv_batch([s1, s0, s1], 0, torch.zeros(3, 2, 1, 8), torch.zeros(3, 2, 1, 8))
    with pytest.raises(RuntimeError, match="launch failed"):
        c.reserve_slots([s0, s1], 40)
    after = _host_state(c)
    assert after[:3] == before[:3] and torch.equal(after[3], before[3])


def test_rejected_rows_leave_no_trace(monkeypatch):
    """k/v of the wrong shape, head count or dtype raise before any page
    bookkeeping changes."""
    c = make()
    s = c.allocate_sequence()
    monkeypatch.setattr(c, "_require_gpu", lambda: None)
    before = _host_state(c)
    good = torch.zeros(1, 2, 1, 8, dtype=torch.float16)
    for k, err in ((torch.zeros(1, 3, 1, 8, dtype=torch.float16), ValueError),   # Hkv 3, cache has 2
                   (torch.zeros(1, 2, 1, 4, dtype=torch.float16), ValueError),   # head_dim 4
                   (torch.zeros(2, 2, 1, 8, dtype=torch.float16), ValueError),   # two tokens, one sequence
                   (torch.zeros(1, 2, 2, 8, dtype=torch.float16), ValueError),   # two positions
                   (torch.zeros(1, 2, 1, 8, dtype=torch.int32), NotImplementedError)):
        with pytest.raises(err):
            c.append_kv(s, 0, k, good)
        with pytest.raises(err):
            c.append_kv(s, 0, good, k)
    with pytest.raises(ValueError, match="dtypes differ"):
        c.append_kv(s, 0, good, good.float())
    after = _host_state(c)
    assert after[:3] == before[:3] and torch.equal(after[3], before[3])


def test_scales_only_for_e4m3_pools():
    with pytest.raises(ValueError):
        PagedKVCache(1, 2, 1, 1, 1, 8, torch.float16, "cpu", k_scale=0.5, v_scale=0.5)
    with pytest.raises(ValueError):
        PagedKVCache(1, 2, 1, 1, 1, 8, torch.float8_e4m3fn, "cpu", k_scale=0.5)
    c = PagedKVCache(1, 2, 1, 1, 1, 8, torch.float8_e4m3fn, "cpu", k_scale=0.5, v_scale=0.25)
    assert c.k_scale.dtype == torch.float32 and c.k_scale.item() == 0.5 and c.v_scale.item() == 0.25


def test_from_config_uses_bf16():
    cfg = types.SimpleNamespace(num_hidden_layers=3, num_key_value_heads=4, head_dim=64)
    c = PagedKVCache.from_config(cfg, num_pages=5, max_seqs=2, max_blocks_per_seq=3, device="cpu")
    assert c.k_pool.dtype == torch.bfloat16 and c.k_pool.shape == (3, 5, 4, 16, 64)
