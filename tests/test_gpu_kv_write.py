"""GPU parity of the KV write path (fsk_paged_write behind paged_kv_write and
PagedKVCache) against the CPU oracle.

Bar: bit-exact pool bytes, block tables and lengths.  The one exception is
the payload of a NaN produced by a cast between f32/f16/bf16 types, which only
has to be a NaN (same-type stores copy NaN payloads bit for bit; e4m3 NaNs are
bit-exact: 0x7F with the input's sign).
"""
import numpy as np
import pytest
import torch

from fasterkernels_amd import workloads as W
from fskernels.hip import paged_kv_write
from fskernels.paged_attn import PagedKVCache, paged_flash_decode
from fskernels.hip import decode as dec
from oracle import decode_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
POOL = {"f16": torch.float16, "bf16": torch.bfloat16, "e4m3": torch.float8_e4m3fn}
SRC = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}
SENTINEL = {"f16": 0x5A5A, "bf16": 0x5A5A, "e4m3": 0x5A}


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw element bits of a GPU tensor as an unsigned numpy array."""
    if t.element_size() == 1:
        return t.view(torch.uint8).cpu().numpy()
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def oracle_bits(pool_np: np.ndarray) -> np.ndarray:
    return pool_np.view(np.uint16) if pool_np.dtype == np.float16 else pool_np


def sentinel_pools(shape, pool):
    """A GPU pool and its oracle twin filled with the same sentinel pattern."""
    dt = POOL[pool]
    if pool == "e4m3":
        g = torch.full(shape, SENTINEL[pool], dtype=torch.uint8, device=DEV).view(dt)
        o = np.full(shape, SENTINEL[pool], dtype=np.uint8)
    else:
        g = torch.full(shape, SENTINEL[pool], dtype=torch.int16, device=DEV).view(dt)
        o = np.full(shape, SENTINEL[pool], dtype=np.uint16)
        if pool == "f16":
            o = o.view(np.float16)
    return g, o


def source_values(n, hkv, d, src, gen, spread=40.0):
    """[n, hkv, d] values in the source dtype with rounding ties, range edges
    and non-finite values planted among normal draws."""
    x = torch.randn(n, hkv, d, generator=gen) * spread
    flat = x.view(-1)
    special = torch.tensor([0.0, -0.0, 448.0, -448.0, 464.0, -464.0, 470.0, 1e5, -1e5, float("inf"),
                            float("-inf"), float("nan"), -float("nan"), 65504.0, 65520.0, 1e-7, -3e-8])
    idx = torch.randperm(flat.numel(), generator=gen)[:4 * special.numel()]
    flat[idx] = special.repeat(4)[:idx.numel()]   # (small tensors take the first ones)
    if src == "f32":  # f16 and bf16 rounding ties
        u = torch.randint(0, 1 << 15, (512,), generator=gen, dtype=torch.int32)
        ties = ((u << 16) | 0x8000).view(torch.float32)
        h = torch.randint(0, 0x7C00, (512,), generator=gen, dtype=torch.int32).to(torch.int16)
        ties16 = (h.view(torch.float16).float().view(torch.int32) | 0x1000).view(torch.float32)
        idx = torch.randperm(flat.numel(), generator=gen)[:1024]
        flat[idx] = torch.cat([ties, ties16])[:idx.numel()]
    return x.to(SRC[src])


def compare(got_pool, want_np, pool, src, what):
    g = bits(got_pool)
    w = oracle_bits(want_np)
    if pool != "e4m3" and src != pool:
        # NaN payloads of a cast between float types are not pinned
        exp_mask, man_mask = (0x7C00, 0x03FF) if pool == "f16" else (0x7F80, 0x007F)
        nan_w = ((w & exp_mask) == exp_mask) & ((w & man_mask) != 0)
        nan_g = ((g & exp_mask) == exp_mask) & ((g & man_mask) != 0)
        assert np.array_equal(nan_g, nan_w), what
        g = np.where(nan_w, 0, g)
        w = np.where(nan_w, 0, w)
    bad = g != w
    assert not bad.any(), f"{what}: {bad.sum()} elements differ; first at {np.argwhere(bad)[0]}: " \
                          f"got {g[bad][:4]}, want {w[bad][:4]}"


@pytest.mark.parametrize("src", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("pool,scaled", [("f16", False), ("bf16", False), ("e4m3", False), ("e4m3", True)])
def test_write_matches_oracle(src, pool, scaled):
    gen = torch.Generator().manual_seed(11)
    P, hkv, ps, d, n = 37, 8, 16, 128, 200
    kx = source_values(n, hkv, d, src, gen)
    vx = source_values(n, hkv, d, src, gen, spread=3.0)
    slots = torch.randperm(P * ps, generator=gen)[:n].to(torch.int64)
    slots[5], slots[77], slots[150] = -1, P * ps, -(1 << 40)   # skipped tokens
    kg, ko = sentinel_pools((P, hkv, ps, d), pool)
    vg, vo = sentinel_pools((P, hkv, ps, d), pool)
    ks = vs = None
    kso = vso = None
    if scaled:
        kso, vso = np.float32(0.05), np.float32(0.004)
        ks = torch.tensor(kso, device=DEV)
        vs = torch.tensor(vso, device=DEV)
    paged_kv_write(kx.to(DEV), vx.to(DEV), kg, vg, slots.to(DEV), k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    for x, o, sc in ((kx, ko, kso), (vx, vo, vso)):
        if src == pool:   # same element type: a byte copy, NaN payloads included
            O.paged_store_rows(o.view(np.uint16), slots.numpy(), x.view(torch.int16).numpy().view(np.uint16))
        else:
            O.paged_write(o, slots.numpy(), x.float().numpy(), pool, sc)
    compare(kg, ko, pool, src, f"K {src}->{pool} scaled={scaled}")
    compare(vg, vo, pool, src, f"V {src}->{pool} scaled={scaled}")


@pytest.mark.parametrize("ps", [32, 64])
@pytest.mark.parametrize("src,pool,scaled", [("f16", "f16", False), ("bf16", "e4m3", True)])
def test_write_page_sizes(ps, src, pool, scaled):
    """Pages of 32 and 64 rows: slot s goes to page s // ps, row s % ps."""
    gen = torch.Generator().manual_seed(12 + ps)
    P, hkv, d, n = 9, 8, 128, 150
    kx = source_values(n, hkv, d, src, gen)
    vx = source_values(n, hkv, d, src, gen, spread=3.0)
    slots = torch.randperm(P * ps, generator=gen)[:n].to(torch.int64)
    kg, ko = sentinel_pools((P, hkv, ps, d), pool)
    vg, vo = sentinel_pools((P, hkv, ps, d), pool)
    kso, vso = (np.float32(0.05), np.float32(0.004)) if scaled else (None, None)
    ks = None if kso is None else torch.tensor(kso, device=DEV)
    vs = None if vso is None else torch.tensor(vso, device=DEV)
    paged_kv_write(kx.to(DEV), vx.to(DEV), kg, vg, slots.to(DEV), k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    for x, o, sc in ((kx, ko, kso), (vx, vo, vso)):
        if src == pool:
            O.paged_store_rows(o.view(np.uint16), slots.numpy(), x.view(torch.int16).numpy().view(np.uint16))
        else:
            O.paged_write(o, slots.numpy(), x.float().numpy(), pool, sc)
    compare(kg, ko, pool, src, f"K ps={ps} {src}->{pool}")
    compare(vg, vo, pool, src, f"V ps={ps} {src}->{pool}")


def _scales():
    fixed = [1.0, 0.5, 3.0, 1 / 3, 0.1, 0.0123, 4 / 448, 448 / 65504, 1e-3, 7.77e-5, 1e-8, 1e-30, 2.5e30,
             1.0000001, 0.99999994, 1e-40, 2.0 ** -126, 3.4e38]
    g = torch.Generator().manual_seed(77)
    rand = torch.exp(torch.empty(18).uniform_(-14.0, 9.0, generator=g)).tolist()
    return [float(torch.tensor(v, dtype=torch.float32)) for v in fixed + rand]


@pytest.mark.parametrize("src", ["f16", "bf16", "f32"])
def test_quantiser_is_exact_for_every_source_value(src):
    """e4m3 codes of every f16 / bf16 bit pattern (and 2^20 random f32
    patterns) under 36 scales equal torch's evaluation of the reference
    quantiser, (x.float() / scale).clamp(-448, 448).to(float8_e4m3fn)."""
    if src == "f32":
        bits32 = torch.randint(-(1 << 31), 1 << 31, (1 << 20,), generator=torch.Generator().manual_seed(5),
                               dtype=torch.int64).to(torch.int32)
        x = bits32.view(torch.float32)
    else:
        x = torch.arange(-(1 << 15), 1 << 15, dtype=torch.int32).to(torch.int16).view(SRC[src])
    d = 128
    rows = x.reshape(-1, 1, d)
    n = rows.shape[0]
    pool = torch.empty(n, 1, 16, d, dtype=torch.float8_e4m3fn, device=DEV)
    slots = (torch.arange(n) * 16).to(DEV)
    rows_g = rows.to(DEV)
    for scale in _scales():
        st = torch.tensor(scale, dtype=torch.float32)
        paged_kv_write(rows_g, rows_g, pool, pool, slots, k_scale=st.to(DEV), v_scale=st.to(DEV))
        got = pool[:, 0, 0, :].reshape(-1).view(torch.uint8).cpu()
        want = (x.float() / st).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8)
        bad = got != want
        assert not bad.any(), (scale, x[bad][:4].tolist(), got[bad][:4].tolist(), want[bad][:4].tolist())


@pytest.mark.parametrize("d", [64, 128, 256, 136])
def test_head_dims_and_strided_sources(d):
    """HF projections arrive as [1, Hkv, L, D]; the [L, Hkv, D] view of one is
    written without a copy.  Also [n, Hkv, 1, D] inputs and odd head dims."""
    gen = torch.Generator().manual_seed(d)
    P, hkv, ps, L = 11, 4, 16, 150
    hf = torch.randn(1, hkv, L, d, generator=gen).to(torch.bfloat16)
    view = hf[0].transpose(0, 1)                                  # [L, Hkv, D], strides (D, L*D, 1)
    slots = torch.randperm(P * ps, generator=gen)[:L].to(torch.int64)
    kg, ko = sentinel_pools((P, hkv, ps, d), "bf16")
    vg, vo = sentinel_pools((P, hkv, ps, d), "bf16")
    hf_g = hf.to(DEV)
    paged_kv_write(hf_g[0].transpose(0, 1), hf_g[0].transpose(0, 1)[:, :, None, :], kg, vg, slots.to(DEV))
    torch.cuda.synchronize()
    O.paged_write(ko, slots.numpy(), view.float().numpy(), "bf16")
    O.paged_write(vo, slots.numpy(), view.float().numpy(), "bf16")
    compare(kg, ko, "bf16", "bf16", f"strided K d={d}")
    compare(vg, vo, "bf16", "bf16", f"[n,Hkv,1,D] V d={d}")


def test_block_table_updates_in_the_same_launch():
    gen = torch.Generator().manual_seed(3)
    P, hkv, ps, d = 8, 2, 16, 64
    kg, _ = sentinel_pools((P, hkv, ps, d), "f16")
    vg, _ = sentinel_pools((P, hkv, ps, d), "f16")
    bt = torch.full((3, 5), -1, dtype=torch.int32, device=DEV)
    upd = torch.tensor([[0, 7], [6, 3], [14, 1], [15, 99], [-1, 42]], dtype=torch.int64)   # last two skipped
    x = torch.randn(2, hkv, d, generator=gen).half().to(DEV)
    paged_kv_write(x, x, kg, vg, torch.tensor([7 * 16, 3 * 16 + 5], device=DEV), block_table=bt,
                   bt_updates=upd.to(DEV))
    torch.cuda.synchronize()
    want = np.full(15, -1, np.int32)
    want[[0, 6, 14]] = [7, 3, 1]
    assert bt.view(-1).cpu().numpy().tolist() == want.tolist()
    assert torch.equal(kg[7, :, 0].cpu(), x[0].cpu()) and torch.equal(vg[3, :, 5].cpu(), x[1].cpu())


def ref_store(ref, sid, pos, layer, k, v):
    """Row store of the oracle cache at an already allocated position."""
    pp = int(ref.block_table[sid, pos // 16])
    ref.k_pool[layer, pp, :, pos % 16, :] = O.encode_kv(k, ref.pool_dtype, ref.k_scale)
    ref.v_pool[layer, pp, :, pos % 16, :] = O.encode_kv(v, ref.pool_dtype, ref.v_scale)


def fits(ref, ids, n_tok, max_blocks):
    """Whether appending n_tok tokens to each id stays within the pool and rows."""
    after = {i: ref.seq_lens[i] + n_tok * ids.count(i) for i in set(ids)}
    need = sum(-(-after[i] // 16) - -(-ref.seq_lens[i] // 16) for i in after)
    return need <= len(ref.free_pages) and max(-(-a // 16) for a in after.values()) <= max_blocks


def run_cache_script(cache, ref, rnd, steps, layers, src_dt, gen, dev=DEV):
    """Random allocate / append / batch-append / reserve+write / free steps on
    both caches, comparing the full state after every step (the cache's
    pools and new rows on ``dev``)."""
    live = []
    hkv, d = cache.num_kv_heads, cache.head_dim
    mb = cache.max_blocks_per_seq
    for step in range(steps):
        op = rnd.random()
        if (op < 0.15 or not live) and len(live) < cache.max_seqs:
            sid = cache.allocate_sequence()
            assert ref.allocate_sequence() == sid
            live.append(sid)
            continue
        if op < 0.22 and len(live) > 1:
            sid = live.pop(rnd.randrange(len(live)))
            cache.free_sequence(sid)
            ref.free_sequence(sid)
            continue
        layer = rnd.randrange(layers)
        if op < 0.5:        # reference per-token append
            sid = rnd.choice(live)
            if not fits(ref, [sid], 1, mb):
                continue
            x = torch.randn(2, 1, hkv, 1, d, generator=gen).to(src_dt)
            cache.append_kv(sid, layer, x[0].to(dev), x[1].to(dev))
            ref.append_kv(sid, layer, x[0, 0, :, 0].float().numpy(), x[1, 0, :, 0].float().numpy())
        elif op < 0.75:     # one token for several sequences in one launch
            ids = [rnd.choice(live) for _ in range(rnd.randint(1, 5))]
            if not fits(ref, ids, 1, mb):
                continue
            x = torch.randn(2, len(ids), hkv, 1, d, generator=gen).to(src_dt)
            cache.append_kv_batch(ids, layer, x[0].to(dev), x[1].to(dev))
            for j, sid in enumerate(ids):
                ref.append_kv(sid, layer, x[0, j, :, 0].float().numpy(), x[1, j, :, 0].float().numpy())
        else:               # reserve a span once, store it for every layer
            ids = rnd.sample(live, rnd.randint(1, len(live)))
            n_tok = rnd.choice([1, 5, 16, 23])
            if not fits(ref, ids, n_tok, mb):
                continue
            slots = cache.reserve_slots(ids, n_tok)
            xs = [torch.randn(2, len(ids) * n_tok, hkv, d, generator=gen).to(src_dt) for _ in range(layers)]
            for lyr in range(layers):
                cache.write_kv(lyr, xs[lyr][0].to(dev), xs[lyr][1].to(dev), slots)
            for j, sid in enumerate(ids):
                for t in range(n_tok):
                    row = j * n_tok + t
                    pos = ref.seq_lens[sid]
                    ref.append_kv(sid, 0, xs[0][0, row].float().numpy(), xs[0][1, row].float().numpy())
                    for lyr in range(1, layers):
                        ref_store(ref, sid, pos, lyr, xs[lyr][0, row].float().numpy(),
                                  xs[lyr][1, row].float().numpy())
        if torch.device(dev).type == "cuda":
            torch.cuda.synchronize()
        assert cache.block_table.cpu().numpy().tolist() == ref.block_table.tolist(), step
        assert cache._seq_lens == ref.seq_lens and cache._free_pages == ref.free_pages, step
    return live


@pytest.mark.parametrize("pool,src", [("f16", "f16"), ("bf16", "bf16"), ("f16", "f32"), ("e4m3", "bf16")])
def test_cache_matches_reference_cache(pool, src):
    """PagedKVCache driven on the GPU ends bit-identical to the oracle's
    restatement of the reference cache driven with the same calls."""
    import random
    rnd = random.Random(5)
    gen = torch.Generator().manual_seed(5)
    L, P, S, MB, hkv, d = 2, 96, 4, 24, 4, 64
    scales = dict(k_scale=0.03, v_scale=0.02) if pool == "e4m3" else {}
    cache = PagedKVCache(L, P, S, MB, hkv, d, POOL[pool], DEV, **scales)
    ref = O.RefPagedKVCache(L, P, S, MB, hkv, d, pool,
                            np.float32(0.03) if scales else None, np.float32(0.02) if scales else None)
    run_cache_script(cache, ref, rnd, 60, L, SRC[src], gen)
    compare(cache.k_pool, ref.k_pool, pool, src, "k_pool")
    compare(cache.v_pool, ref.v_pool, pool, src, "v_pool")


@pytest.mark.parametrize("pool", ["f16", "e4m3"])
def test_decode_through_the_cache(pool):
    """Prefill spans and single-token appends through the cache, then paged
    decode of the cache equals the oracle's attention over the dense rows."""
    gen = torch.Generator().manual_seed(9)
    hkv, hq, d = 8, 32, 128
    scales = dict(k_scale=0.02, v_scale=0.02) if pool == "e4m3" else {}
    cache = PagedKVCache(1, 200, 4, 64, hkv, d, POOL[pool], DEV, **scales)
    lens = [300, 17, 1000]
    sids = [cache.allocate_sequence() for _ in lens]
    dense = []
    for sid, L in zip(sids, lens):
        kv = torch.randn(2, 1, hkv, L, d, generator=gen).half()
        slots = cache.reserve_slots([sid], L - 1)
        cache.write_kv(0, kv[0, 0].transpose(0, 1)[:L - 1].to(DEV), kv[1, 0].transpose(0, 1)[:L - 1].to(DEV), slots)
        cache.append_kv(sid, 0, kv[0][:, :, L - 1:].to(DEV), kv[1][:, :, L - 1:].to(DEV))
        ks = kv[0, 0].transpose(0, 1).float().numpy()
        vs = kv[1, 0].transpose(0, 1).float().numpy()
        if scales:
            ks = O.dequantize_fp8(O.encode_kv(ks, "e4m3", np.float32(0.02)), np.float32(0.02))
            vs = O.dequantize_fp8(O.encode_kv(vs, "e4m3", np.float32(0.02)), np.float32(0.02))
        dense.append((ks, vs))
    q = torch.randn(len(lens), hq, d, generator=gen).half()
    out = paged_flash_decode(q.to(DEV), cache.k_pool[0], cache.v_pool[0], cache.get_block_table_tensor(sids),
                             cache.get_seq_lens_tensor(sids), 16,
                             k_scale=cache.k_scale, v_scale=cache.v_scale)
    torch.cuda.synchronize()
    want = np.stack([O.attend(q[i].double().numpy(), *dense[i]) for i in range(len(lens))])
    atol = 1e-2 if scales else 2e-3
    err = np.abs(out.double().cpu().numpy() - want)
    tol = atol + 2e-3 * np.abs(want)
    assert (err <= tol).all(), (err / tol).max()


def test_full_size_prefill_write_round_trip():
    """The M0 cache (4 sequences x 32768 tokens, Hkv 8, D 128) written in one
    launch per pool type: f16 reads back bit-exact through the decode kernels'
    page addressing, and the e4m3 quantisation equals torch's expression of
    the reference quantiser on the same device (and the oracle on a sample)."""
    gen = torch.Generator(device=DEV).manual_seed(100)
    B, L, hkv, d, ps = 4, 32768, 8, 128, 16
    n_pages = B * L // ps
    perm = torch.randperm(n_pages, device=DEV, generator=gen).to(torch.int32)
    bt = perm.view(B, L // ps)
    t = torch.arange(L, device=DEV)
    slots = (bt.long()[:, t // ps] * ps + t % ps).reshape(-1)
    k = torch.randn(B * L, hkv, d, device=DEV, generator=gen).half()
    v = torch.randn(B * L, hkv, d, device=DEV, generator=gen).half()
    kp = torch.empty(n_pages, hkv, ps, d, dtype=torch.float16, device=DEV)
    vp = torch.empty_like(kp)
    paged_kv_write(k, v, kp, vp, slots)
    lens = torch.full((B,), L, dtype=torch.int32, device=DEV)
    back = dec.paged_gather(kp, bt, lens)                      # [B, Hkv, L, D]
    assert torch.equal(back.transpose(1, 2).reshape(B * L, hkv, d), k)
    back = dec.paged_gather(vp, bt, lens)
    assert torch.equal(back.transpose(1, 2).reshape(B * L, hkv, d), v)
    del back
    scale = torch.tensor(0.01, device=DEV)
    kq = torch.empty(n_pages, hkv, ps, d, dtype=torch.float8_e4m3fn, device=DEV)
    vq = torch.empty_like(kq)
    paged_kv_write(k, v, kq, vq, slots, k_scale=scale, v_scale=scale)
    want = (k.float() / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    got = dec.paged_gather(kq, bt, lens).transpose(1, 2).reshape(B * L, hkv, d)
    assert torch.equal(got.view(torch.uint8), want.view(torch.uint8))
    rows = torch.randint(0, B * L, (64,), device=DEV, generator=gen)
    o = O.encode_kv(k[rows].float().cpu().numpy(), "e4m3", np.float32(0.01))
    assert np.array_equal(got[rows].view(torch.uint8).cpu().numpy(), o)


def test_write_replays_in_a_hip_graph():
    """With device-resident slots the write is capturable: replays with new
    slot contents and new rows store what eager calls store."""
    gen = torch.Generator().manual_seed(21)
    P, hkv, ps, d, n = 16, 8, 16, 128, 32
    kp = torch.zeros(P, hkv, ps, d, dtype=torch.bfloat16, device=DEV)
    vp = torch.zeros_like(kp)
    k = torch.zeros(n, hkv, d, dtype=torch.bfloat16, device=DEV)
    v = torch.zeros_like(k)
    slots = torch.zeros(n, dtype=torch.int64, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        paged_kv_write(k, v, kp, vp, slots)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        paged_kv_write(k, v, kp, vp, slots)
    ref_k = torch.zeros_like(kp)
    ref_v = torch.zeros_like(vp)
    for rep in range(3):
        kx = torch.randn(n, hkv, d, generator=gen).bfloat16()
        vx = torch.randn(n, hkv, d, generator=gen).bfloat16()
        sl = torch.randperm(P * ps, generator=gen)[:n]
        k.copy_(kx)
        v.copy_(vx)
        slots.copy_(sl)
        g.replay()
        paged_kv_write(kx.to(DEV), vx.to(DEV), ref_k, ref_v, sl.to(DEV))
        torch.cuda.synchronize()
        assert torch.equal(kp, ref_k) and torch.equal(vp, ref_v), rep


@pytest.mark.parametrize("seed", range(20))
def test_randomized_writes(seed):
    """Random pool sizes, page sizes, head counts, head dims, source / pool
    types, scales and slot lists (with skipped and repeated-page slots)."""
    r = np.random.default_rng(3000 + seed)
    src = ["f16", "bf16", "f32"][r.integers(3)]
    pool, scaled = [("f16", False), ("bf16", False), ("e4m3", False), ("e4m3", True)][r.integers(4)]
    ps = int(r.choice([16, 32, 64]))
    P, hkv, d = int(r.integers(1, 40)), int(r.choice([1, 2, 8])), int(r.choice([64, 128, 256]))
    n = int(r.integers(1, min(P * ps, 300) + 1))
    gen = torch.Generator().manual_seed(seed)
    kx = source_values(n, hkv, d, src, gen)
    vx = source_values(n, hkv, d, src, gen, spread=3.0)
    slots = torch.randperm(P * ps, generator=gen)[:n].to(torch.int64)
    if n > 3:
        slots[int(r.integers(n))] = -1   # a skipped token
    kg, ko = sentinel_pools((P, hkv, ps, d), pool)
    vg, vo = sentinel_pools((P, hkv, ps, d), pool)
    kso = vso = None
    if scaled:
        kso, vso = np.float32(r.uniform(1e-3, 1.0)), np.float32(r.uniform(1e-3, 1.0))
    ks = None if kso is None else torch.tensor(kso, device=DEV)
    vs = None if vso is None else torch.tensor(vso, device=DEV)
    paged_kv_write(kx.to(DEV), vx.to(DEV), kg, vg, slots.to(DEV), k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    for x, o, sc in ((kx, ko, kso), (vx, vo, vso)):
        if src == pool:
            O.paged_store_rows(o.view(np.uint16), slots.numpy(), x.view(torch.int16).numpy().view(np.uint16))
        else:
            O.paged_write(o, slots.numpy(), x.float().numpy(), pool, sc)
    what = f"seed {seed}: {src}->{pool} scaled={scaled} P={P} ps={ps} hkv={hkv} d={d} n={n}"
    compare(kg, ko, pool, src, "K " + what)
    compare(vg, vo, pool, src, "V " + what)


def test_rejected_append_leaves_cache_unchanged_and_host_rows_are_copied():
    """A rejected append (wrong head count, wrong dtype) changes neither the
    lengths, the free list nor the device block table; rows given on the CPU
    are stored as the same rows given on the device are (the reference's
    indexed store accepts rows from any device)."""
    gen = torch.Generator().manual_seed(31)
    cache = PagedKVCache(1, 8, 2, 4, 2, 64, torch.float16, DEV)
    twin = PagedKVCache(1, 8, 2, 4, 2, 64, torch.float16, DEV)
    s, t = cache.allocate_sequence(), twin.allocate_sequence()
    rows = [torch.randn(1, 2, 1, 64, generator=gen).half() for _ in range(2 * 17)]
    for j in range(17):                      # 17 tokens: the second page is taken
        cache.append_kv(s, 0, rows[2 * j], rows[2 * j + 1])                  # host rows
        twin.append_kv(t, 0, rows[2 * j].to(DEV), rows[2 * j + 1].to(DEV))    # device rows
    torch.cuda.synchronize()
    lens, free, bt = list(cache._seq_lens), list(cache._free_pages), cache.block_table.clone()
    with pytest.raises(ValueError):
        cache.append_kv(s, 0, torch.zeros(1, 3, 1, 64, dtype=torch.float16, device=DEV),
                        torch.zeros(1, 3, 1, 64, dtype=torch.float16, device=DEV))
    with pytest.raises(NotImplementedError):
        cache.append_kv(s, 0, torch.zeros(1, 2, 1, 64, dtype=torch.int32, device=DEV),
                        torch.zeros(1, 2, 1, 64, dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    assert cache._seq_lens == lens and cache._free_pages == free
    assert torch.equal(cache.block_table, bt)
    assert torch.equal(cache.block_table, twin.block_table) and cache._seq_lens == twin._seq_lens
    assert torch.equal(cache.k_pool.cpu(), twin.k_pool.cpu()) and torch.equal(cache.v_pool.cpu(), twin.v_pool.cpu())


@pytest.mark.parametrize("name", ["W0", "W1", "W2", "W3", "W4"])
def test_bench_write_workloads(name):
    """The bench's KV-write workloads at their bench sizes, bit-exact against
    the oracle: W0 the whole M0 cache (131072 tokens) f16 -> f16, W1 the same
    rows bf16 -> e4m3 with scales, W2 one decode-step append for 64
    sequences (rows into partly filled pages of a zeroed pool), W3 and W4 as
    W0 and W1 on a fresh cache's page order."""
    wl = W.make_write(name, device=DEV)
    cfg = W.WRITE_CONFIGS[name]
    W.run_write(wl)
    torch.cuda.synchronize()
    slots = wl.slots.cpu().numpy()
    for x, got, sc, kv in ((wl.k, wl.k_pool, wl.k_scale, "K"), (wl.v, wl.v_pool, wl.v_scale, "V")):
        if cfg["pool"] == "e4m3":
            o = np.zeros(tuple(got.shape), np.uint8)
            O.paged_write(o, slots, x.float().cpu().numpy(), "e4m3", None if sc is None else np.float32(sc.item()))
        else:
            o = np.zeros(tuple(got.shape), np.float16)
            O.paged_store_rows(o.view(np.uint16), slots, x.view(torch.int16).cpu().numpy().view(np.uint16))
        compare(got, o, cfg["pool"], cfg["src"], f"{kv} {name}")
