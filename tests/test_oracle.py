"""Pins the CPU oracle (oracle/decode_oracle.py) before it is trusted.

Every oracle function is checked against something it does not share code
with: torch's scaled_dot_product_attention and logsumexp (library routines),
torch's float8_e4m3fn casts, the brute-force golden vectors in tests/golden/
(pure-Python loops written from the definitions), closed forms and
invariants.  The last test plants plausible mistakes in the oracle (wrong
head mapping, dropped scale, swapped sink semantics, K/V swapped, transposed
page addressing, off-by-one varlen slicing, dropped LSE weight, transposed
write slots, truncating bf16, a wrong e4m3 tie, a quantiser without clamp, a
FIFO free list) and requires that at least one pin fails for each.
"""
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import decode_oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
rng = np.random.default_rng(1234)


def sdpa(q, k, v, sink=None):
    """torch SDPA reference for one sequence: q [Hq, D], k/v [L, Hkv, D].
    An exp-mode sink is an extra key whose logit is the sink (additive mask)
    and whose value is zero."""
    Hq, D = q.shape
    L, Hkv, _ = k.shape
    G = Hq // Hkv
    Q = torch.tensor(q)[:, None, :]                                    # [Hq, 1, D]
    K = torch.tensor(k).permute(1, 0, 2).repeat_interleave(G, 0)       # [Hq, L, D]
    V = torch.tensor(v).permute(1, 0, 2).repeat_interleave(G, 0)
    mask = torch.zeros(Hq, 1, L, dtype=torch.float64)
    if sink is not None:
        K = torch.cat([K, torch.zeros(Hq, 1, D, dtype=K.dtype)], 1)
        V = torch.cat([V, torch.zeros(Hq, 1, D, dtype=V.dtype)], 1)
        mask = torch.cat([mask, torch.tensor(sink, dtype=torch.float64).view(Hq, 1, 1)], 2)
    return F.scaled_dot_product_attention(Q, K, V, attn_mask=mask)[:, 0, :].numpy()


def rand_case(Hq=8, Hkv=2, D=32, L=37):
    return rng.standard_normal((Hq, D)), rng.standard_normal((L, Hkv, D)), rng.standard_normal((L, Hkv, D))


# ---------------------------------------------------------------------------
# pins, written as predicates so the planted-mistake test can reuse them
# ---------------------------------------------------------------------------
def pin_sdpa(ora):
    for Hq, Hkv, D, L in [(8, 8, 16, 5), (8, 2, 32, 37), (32, 8, 128, 300), (6, 3, 64, 1)]:
        q, k, v = rand_case(Hq, Hkv, D, L)
        if not np.allclose(ora.attend(q, k, v), sdpa(q, k, v), atol=1e-12, rtol=1e-10):
            return False
    return True


def pin_exp_sink(ora):
    for L in (1, 9, 200):
        q, k, v = rand_case(L=L)
        z = rng.standard_normal(8) * 2
        if not np.allclose(ora.attend(q, k, v, z, "exp"), sdpa(q, k, v, z), atol=1e-12, rtol=1e-10):
            return False
    return True


def pin_linear_sink(ora):
    """out_lin = out_plain * S / (S + z) with S = sum_t e^{s_t - max s} = e^{lse - max}."""
    for L in (1, 9, 200):
        q, k, v = rand_case(L=L)
        z = np.abs(rng.standard_normal(8)) + 0.1
        G = 4
        s = torch.einsum("hd,lhd->hl", torch.tensor(q),
                         torch.tensor(k).repeat_interleave(G, 1)) / math.sqrt(q.shape[1])
        S = torch.exp(torch.logsumexp(s, 1) - s.max(1).values).numpy()
        want = sdpa(q, k, v) * (S / (S + z))[:, None]
        if not np.allclose(ora.attend(q, k, v, z, "linear"), want, atol=1e-12, rtol=1e-10):
            return False
    return True


def pin_golden_varlen(ora):
    g = np.load(os.path.join(GOLD, "varlen_small.npz"))
    for mode, key in (("exp", "out_none"), ("exp", "out_exp"), ("linear", "out_linear")):
        sink = None if key == "out_none" else g["s_aux"]
        got = ora.decode_varlen(g["q"], g["k"], g["v"], g["cu_seqlens"], sink, mode)
        if not np.allclose(got, g[key], atol=1e-12, rtol=1e-10):
            return False
    return True


def pin_golden_paged(ora):
    g = np.load(os.path.join(GOLD, "paged_small.npz"))
    got = ora.decode_paged(g["q"], g["k_pool"], g["v_pool"], g["block_table"], g["seq_lens"])
    if not np.allclose(got, g["out"], atol=1e-12, rtol=1e-10):
        return False
    f = np.load(os.path.join(GOLD, "paged_fp8_small.npz"))
    got = ora.decode_paged(f["q"], f["k_codes"], f["v_codes"], f["block_table"], f["seq_lens"],
                           f["s_aux"], "exp", float(f["k_scale"]), float(f["v_scale"]))
    return bool(np.allclose(got, f["out"], atol=1e-10, rtol=1e-9))


def pin_split_merge(ora):
    for L in (1, 5, 64, 257):
        q, k, v = rand_case(L=L)
        z = rng.standard_normal(8)
        full = ora.attend(q, k, v)
        for n in (1, 2, 3, 8, L + 5):
            acc, m, l = ora.partials(q, k, v, n)
            if not np.allclose(ora.merge_partials(acc, m, l), full, atol=1e-12, rtol=1e-10):
                return False
            for mode in ("exp", "linear"):
                zz = np.abs(z) if mode == "linear" else z
                want = ora.attend(q, k, v, zz, mode)
                if not np.allclose(ora.merge_partials(acc, m, l, zz, mode), want, atol=1e-12, rtol=1e-10):
                    return False
    return True


def pin_closed_forms(ora):
    q, k, v = rand_case(L=1)
    if not np.allclose(ora.attend(q, k, v), np.repeat(v[0], 4, axis=0), atol=1e-14):
        return False  # one token: the output is that token's value row
    q, k, v = rand_case(L=23)
    k[:] = k[:1]  # identical keys: uniform weights -> mean of the values
    if not np.allclose(ora.attend(q, k, v), np.repeat(v.mean(0), 4, axis=0), atol=1e-12):
        return False
    q, k, v = rand_case(L=11)
    if not np.allclose(ora.attend(q, k, v, np.full(8, -np.inf), "exp"), ora.attend(q, k, v), atol=1e-14):
        return False
    if not np.allclose(ora.attend(q, k, v, np.zeros(8), "linear"), ora.attend(q, k, v), atol=1e-14):
        return False
    # scores scale with sm_scale: doubling q equals doubling sm_scale
    return bool(np.allclose(ora.attend(2 * q, k, v), ora.attend(q, k, v, sm_scale=2 / math.sqrt(32)), atol=1e-12))


def pin_layouts(ora):
    """Varlen, paged and dense entry points agree on the same logical sequences."""
    Hq, Hkv, D = 8, 2, 16
    lens = [3, 16, 33]
    T = sum(lens)
    q = rng.standard_normal((3, Hq, D))
    k = rng.standard_normal((T, Hkv, D))
    v = rng.standard_normal((T, Hkv, D))
    cu = np.concatenate([[0], np.cumsum(lens)])
    ref = np.stack([ora.attend(q[b], k[cu[b]:cu[b + 1]], v[cu[b]:cu[b + 1]]) for b in range(3)])
    if not np.allclose(ora.decode_varlen(q, k, v, cu), ref, atol=1e-13):
        return False
    # paged: build a shuffled pool like tests/test_triton_paged_gqa_decode.py:65-87
    npg = [(L + 15) // 16 for L in lens]
    P = sum(npg) + 3
    perm = rng.permutation(P)
    bt = -np.ones((3, max(npg)), dtype=np.int32)
    kp = rng.standard_normal((P, Hkv, 16, D))
    vp = rng.standard_normal((P, Hkv, 16, D))
    o = 0
    for b, L in enumerate(lens):
        for j in range(npg[b]):
            pg = perm[o]
            o += 1
            bt[b, j] = pg
            n = min(16, L - 16 * j)
            kp[pg, :, :n] = k[cu[b] + 16 * j: cu[b] + 16 * j + n].transpose(1, 0, 2)
            vp[pg, :, :n] = v[cu[b] + 16 * j: cu[b] + 16 * j + n].transpose(1, 0, 2)
    if not np.allclose(ora.decode_paged(q, kp, vp, bt, lens), ref, atol=1e-13):
        return False
    # dense with start offsets: pad each sequence behind 4 junk rows
    S = max(lens) + 4
    kd = rng.standard_normal((3, Hkv, S, D))
    vd = rng.standard_normal((3, Hkv, S, D))
    for b, L in enumerate(lens):
        kd[b, :, 4:4 + L] = k[cu[b]:cu[b + 1]].transpose(1, 0, 2)
        vd[b, :, 4:4 + L] = v[cu[b]:cu[b + 1]].transpose(1, 0, 2)
    got = ora.decode_dense(q, kd, vd, np.array(lens) + 4, np.full(3, 4))
    return bool(np.allclose(got, ref, atol=1e-13))


def pin_gather(ora):
    g = np.load(os.path.join(GOLD, "paged_small.npz"))
    dense = ora.paged_gather(g["k_pool"], g["block_table"], g["seq_lens"])
    for b, L in enumerate(g["seq_lens"]):
        for t in range(dense.shape[2]):
            want = g["k_pool"][g["block_table"][b, t // 16], :, t % 16] if t < L else 0.0
            if not np.array_equal(dense[b, :, t], np.broadcast_to(want, dense[b, :, t].shape)):
                return False
    return True


def _encode_values():
    """Values that exercise every rounding and range rule of the pool encodings."""
    u = rng.integers(0, 1 << 15, 4000).astype(np.uint32)
    bf16_ties = ((u << 16) | 0x8000).view(np.float32)           # halfway between bf16 neighbours
    h = rng.integers(0, 0x7C00, 4000).astype(np.uint16)
    f16_ties = (h.view(np.float16).astype(np.float32).view(np.uint32) | 0x1000).view(np.float32)
    codes = np.arange(0, 127, dtype=np.uint8)
    e4m3_mid = (O.e4m3_decode(codes[:-1]).astype(np.float64) + O.e4m3_decode(codes[1:])) / 2
    special = [0.0, -0.0, 448.0, -448.0, 449.0, 463.99, 464.0, -464.0, 464.01, 470.0, 480.0, 1e6, -1e6,
               np.inf, -np.inf, 65504.0, 65520.0, 1e-8, -1e-8, 2.0 ** -24, 2.0 ** -25, 3e38, -3e38]
    v = np.concatenate([rng.standard_normal(20000) * 40, rng.standard_normal(4000) * 1e-3,
                        bf16_ties, -bf16_ties, f16_ties, -f16_ties, e4m3_mid, -e4m3_mid, special])
    with np.errstate(over="ignore", invalid="ignore"):
        v = v.astype(np.float32)
    return v[~np.isnan(v)]


def pin_kv_encode(ora):
    """Pool encodings against torch's casts (library routines) of the same fp32 values."""
    x = _encode_values()
    t = torch.from_numpy(x)
    if not np.array_equal(ora.encode_kv(x, "f16").view(np.uint16), t.to(torch.float16).view(torch.int16).numpy().view(np.uint16)):
        return False
    if not np.array_equal(ora.encode_kv(x, "bf16"), t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)):
        return False
    xn = np.concatenate([x, np.array([np.nan, -np.nan], dtype=np.float32)])
    tn = torch.from_numpy(xn)
    if not np.array_equal(ora.encode_kv(xn, "e4m3"), tn.to(torch.float8_e4m3fn).view(torch.uint8).numpy()):
        return False
    for scale in (np.float32(0.0123), np.float32(2.5), np.float32(1.0)):
        want = (tn / torch.tensor(scale)).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        if not np.array_equal(ora.encode_kv(xn, "e4m3", scale), want):
            return False
    return True


def pin_paged_write(ora):
    """Rows written through block-table slots read back through paged_rows
    (pinned above on the golden gather) as the encoded rows; other rows stay."""
    P, Hkv, ps, D = 9, 3, 16, 8
    for dt in ("f16", "bf16", "e4m3"):
        pool = np.full((P, Hkv, ps, D), 7, dtype=ora._POOL_NP[dt])
        bt = rng.permutation(P)[:4].reshape(2, 2)
        lens = [21, 32]
        x = [rng.standard_normal((L, Hkv, D)).astype(np.float32) for L in lens]
        for b, L in enumerate(lens):
            t = np.arange(L)
            slots = bt[b, t // ps] * ps + t % ps
            ora.paged_write(pool, slots, x[b], dt, 0.01 if dt == "e4m3" else None)
            if not np.array_equal(ora.paged_rows(pool, bt, b, L), ora.encode_kv(x[b], dt, 0.01 if dt == "e4m3" else None)):
                return False
        # a skipped slot and an out-of-range slot leave the pool alone
        before = pool.copy()
        ora.paged_write(pool, [-1, P * ps], np.zeros((2, Hkv, D), np.float32), dt)
        if not np.array_equal(pool, before):
            return False
        # rows past sequence 0's length in its last page keep the fill value
        if not (pool[bt[0, 1], :, 21 - ps:, :] == 7).all():
            return False
    return True


def pin_ref_cache(ora):
    """Page bookkeeping facts of fskernels/paged_attn/paged_kv_cache.py: lowest
    free slot (:85-91), pages popped from the end of [0..P-1] (:61, :106),
    freed pages appended in logical order (:93-101), a new page at each
    16-token boundary (:122-124), "Out of KV pages" (:104-105)."""
    c = ora.RefPagedKVCache(1, 8, 3, 4, 2, 8, "f16")
    if [c.allocate_sequence() for _ in range(3)] != [0, 1, 2]:
        return False
    for pos in range(33):
        c.append_kv(0, 0, np.full((2, 8), pos + 1.0, np.float32), np.full((2, 8), -(pos + 1.0), np.float32))
    if c.block_table[0].tolist() != [7, 6, 5, -1] or c.seq_lens[0] != 33:
        return False
    if not (c.k_pool[0, 6, :, 1, :] == 18.0).all() or not (c.v_pool[0, 5, :, 0, :] == -33.0).all():
        return False
    c.free_sequence(0)
    if c.free_pages != [0, 1, 2, 3, 4, 7, 6, 5] or c.allocate_sequence() != 0:
        return False
    c.append_kv(1, 0, np.zeros((2, 8), np.float32), np.zeros((2, 8), np.float32))
    if c.block_table[1, 0] != 5:
        return False
    c2 = ora.RefPagedKVCache(1, 1, 1, 4, 1, 8, "f16")
    c2.allocate_sequence()
    for _ in range(16):
        c2.append_kv(0, 0, np.zeros((1, 8), np.float32), np.zeros((1, 8), np.float32))
    try:
        c2.append_kv(0, 0, np.zeros((1, 8), np.float32), np.zeros((1, 8), np.float32))
        return False
    except RuntimeError as e:
        return "Out of KV pages" in str(e)


def _torch_probs(q, k, sink=None):
    """Softmax weights from torch.softmax (exp sink = extra logit, then dropped)."""
    Hq, D = q.shape
    L, Hkv, _ = k.shape
    G = Hq // Hkv
    K = torch.tensor(k).permute(1, 0, 2).repeat_interleave(G, 0)           # [Hq, L, D]
    s = torch.einsum("hd,hld->hl", torch.tensor(q), K) / math.sqrt(D)
    if sink is not None:
        s = torch.cat([s, torch.tensor(sink, dtype=s.dtype)[:, None]], 1)
        return torch.softmax(s, 1)[:, :L].numpy()
    return torch.softmax(s, 1).numpy()


def pin_block_scores(ora):
    for L in (1, 127, 128, 129, 300, 1000):
        q, k, _ = rand_case(8, 2, 32, L)
        z = rng.standard_normal(8)
        for sink in (None, z):
            p = _torch_probs(q, k, sink)
            want = np.zeros((8, 10))
            for j in range(min(10, -(-L // 128))):                          # brute-force block maxima
                for h in range(8):
                    want[h, j] = max(p[h, t] for t in range(128 * j, min(128 * j + 128, L)))
            if not np.allclose(ora.block_scores(q, k, sink, "exp", n_blocks=10), want, atol=1e-14, rtol=1e-12):
                return False
        # linear sink: every probability scales by l / (l + z), l = sum e^{s - max} (logsumexp)
        zl = np.abs(z) + 0.5
        s = torch.tensor(np.stack([k[:, h // 4, :] @ q[h] for h in range(8)]) / math.sqrt(32))
        l = torch.exp(torch.logsumexp(s, 1) - s.max(1).values).numpy()
        plain = ora.block_scores(q, k, None, n_blocks=10)
        if not np.allclose(ora.block_scores(q, k, zl, "linear", n_blocks=10), plain * (l / (l + zl))[:, None],
                           atol=1e-14, rtol=1e-12):
            return False
    if ora.block_scores(np.ones((2, 8)), np.ones((1, 1, 8)), n_blocks=3).tolist() != [[1, 0, 0], [1, 0, 0]]:
        return False
    return ora.block_scores(np.ones((2, 8)), np.zeros((0, 1, 8)), n_blocks=2).tolist() == [[0, 0], [0, 0]]


PINS = [pin_sdpa, pin_exp_sink, pin_linear_sink, pin_golden_varlen, pin_golden_paged,
        pin_split_merge, pin_closed_forms, pin_layouts, pin_gather, pin_kv_encode, pin_paged_write,
        pin_ref_cache, pin_block_scores]


@pytest.mark.parametrize("pin", PINS, ids=lambda f: f.__name__)
def test_oracle_pinned(pin):
    assert pin(O)


# ---------------------------------------------------------------------------
# e4m3 codec against torch's float8_e4m3fn and the golden table
# ---------------------------------------------------------------------------
def test_e4m3_decode_matches_torch_and_definition():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    got = O.e4m3_decode(codes)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin].view(np.int32), want[fin].view(np.int32))
    gold = np.load(os.path.join(GOLD, "e4m3_table.npz"))["values"]
    assert np.array_equal(np.isnan(gold), np.isnan(got))
    assert np.array_equal(gold[fin], got[fin].astype(np.float64))


def test_e4m3_encode_matches_torch_cast():
    vals = np.concatenate([
        rng.standard_normal(20000) * 50,
        rng.standard_normal(5000) * 1e-2,        # subnormal range
        O.e4m3_decode(np.arange(256, dtype=np.uint8)),
        # exact midpoints between neighbouring codes (ties to even)
        (O.e4m3_decode(np.arange(0, 126, dtype=np.uint8)).astype(np.float64)
         + O.e4m3_decode(np.arange(1, 127, dtype=np.uint8))) / 2,
        [0.0, -0.0, 448.0, -448.0, 449.0, 463.9, 1e-9, -1e-9, 2.0 ** -10, 3 * 2.0 ** -11],
    ]).astype(np.float32)
    vals = vals[~np.isnan(vals)]
    want = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = O.e4m3_encode(vals)
    bad = got != want
    assert not bad.any(), (vals[bad][:5], got[bad][:5], want[bad][:5])


def test_quantize_to_fp8_matches_reference_formula():
    # restated formula: fskernels/triton/triton_gqa_decode_hf_fp8.py:13-16, via torch ops
    for x in (rng.standard_normal((4, 8, 64)) * 3, np.zeros((3, 5)), rng.standard_normal(7) * 1e-20):
        x = x.astype(np.float32)
        t = torch.from_numpy(x)
        scale = t.abs().max().clamp(min=1e-12) / 448.0
        codes = (t / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        got_codes, got_scale = O.quantize_to_fp8(x)
        assert np.float32(got_scale) == np.float32(scale.item())
        assert np.array_equal(got_codes, codes)


# ---------------------------------------------------------------------------
# planted mistakes: every mutant must fail at least one pin
# ---------------------------------------------------------------------------
class Mutant:
    """The oracle with one function replaced by a plausibly wrong variant."""

    def __init__(self, **over):
        self.__dict__.update({k: getattr(O, k) for k in dir(O) if not k.startswith("__")})
        self.__dict__.update(over)


def _attend_variant(kind):
    def attend(q, k, v, sink=None, sink_mode="exp", sm_scale=None):
        q = np.asarray(q, dtype=np.float64)
        k = np.asarray(k, dtype=np.float64)
        v = np.asarray(v, dtype=np.float64)
        Hq, D = q.shape
        L, Hkv, _ = k.shape
        G = Hq // Hkv
        scale = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
        if kind == "noscale":
            scale = 1.0
        if kind == "kv_swap":
            k, v = v, k
        out = np.empty((Hq, D))
        for h in range(Hq):
            kv = h % Hkv if kind == "headmap" else h // G
            s = k[:, kv, :] @ q[h] * scale
            m = s.max() if L else -np.inf
            mode = sink_mode
            if kind == "sinkswap" and sink is not None:
                mode = "linear" if sink_mode == "exp" else "exp"
            if sink is not None and mode == "exp":
                M = max(m, sink[h])
                e = np.exp(s - M)
                den = e.sum() + np.exp(sink[h] - M)
            else:
                e = np.exp(s - m)
                den = e.sum() + (sink[h] if sink is not None else 0.0)
            out[h] = e @ v[:, kv, :] / den
        return out
    return attend


def _paged_rows_transposed(pool, block_table, b, length):
    pool = np.asarray(pool)
    ps = pool.shape[2]
    t = np.arange(length)
    return pool[np.asarray(block_table)[b, t % ps], :, t // ps, :]


def _varlen_off_by_one(q, k, v, cu, s_aux=None, sink_mode="exp", sm_scale=None):
    cu = np.asarray(cu)
    return np.stack([O.attend(q[b], k[cu[b]:max(cu[b + 1] - 1, cu[b] + 1)], v[cu[b]:max(cu[b + 1] - 1, cu[b] + 1)],
                              s_aux, sink_mode, sm_scale) for b in range(len(q))])


def _merge_no_weight(acc, m, l, sink=None, sink_mode="exp"):
    num = np.asarray(acc).sum(0)
    den = np.asarray(l).sum(0)
    return num / den[:, None]


def _store_rows_transposed(pool, slots, rows):
    P, Hkv, ps, D = pool.shape
    rows = np.asarray(rows).reshape(-1, Hkv, D)
    for i, s in enumerate(np.asarray(slots, dtype=np.int64).reshape(-1)):
        if 0 <= s < P * ps:
            pool[s % P, :, s // P % ps, :] = rows[i]
    return pool


def _bf16_truncate(x):
    return (np.asarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


_e4m3_encode_orig = O.e4m3_encode
_encode_kv_orig = O.encode_kv


def _e4m3_encode_tie_to_nan(x):
    x = np.asarray(x, dtype=np.float64)
    codes = _e4m3_encode_orig(x)
    return np.where(np.abs(x) == 464.0, codes | 0x7F, codes).astype(np.uint8)


def _encode_kv_no_clamp(x, pool_dtype, scale=None):
    if pool_dtype == "e4m3" and scale is not None:
        return _e4m3_encode_orig(np.asarray(x, dtype=np.float32) / np.float32(scale))
    return _encode_kv_orig(x, pool_dtype, scale)


class _FifoCache(O.RefPagedKVCache):
    def append_kv(self, sid, layer, k, v):
        if self.seq_lens[sid] % self.page_size == 0 and self.free_pages:
            self.free_pages.insert(len(self.free_pages), self.free_pages.pop(0))
        super().append_kv(sid, layer, k, v)


_block_scores_orig = O.block_scores


def _block_scores_block64(q, k, sink=None, sink_mode="exp", sm_scale=None, n_blocks=None, block=128):
    return _block_scores_orig(q, k, sink, sink_mode, sm_scale, n_blocks, block=64)


def _block_scores_no_sink(q, k, sink=None, sink_mode="exp", sm_scale=None, n_blocks=None, block=128):
    return _block_scores_orig(q, k, None, sink_mode, sm_scale, n_blocks, block)


def _block_scores_sum(q, k, sink=None, sink_mode="exp", sm_scale=None, n_blocks=None, block=128):
    # block sum instead of block max
    full = _block_scores_orig(q, k, sink, sink_mode, sm_scale, None, 1)   # per-token probabilities
    L = full.shape[1]
    n = -(-L // block) if n_blocks is None else n_blocks
    out = np.zeros((full.shape[0], n))
    for j in range(min(n, -(-L // block))):
        out[:, j] = full[:, j * block:(j + 1) * block].sum(1)
    return out


MUTANTS = {
    "head mapping h % Hkv": Mutant(attend=_attend_variant("headmap")),
    "sm_scale dropped": Mutant(attend=_attend_variant("noscale")),
    "K and V swapped": Mutant(attend=_attend_variant("kv_swap")),
    "sink semantics swapped": Mutant(attend=_attend_variant("sinkswap")),
    "page index transposed": Mutant(paged_rows=_paged_rows_transposed),
    "varlen off by one": Mutant(decode_varlen=_varlen_off_by_one),
    "LSE weight dropped": Mutant(merge_partials=_merge_no_weight),
    "write slot transposed": Mutant(paged_store_rows=_store_rows_transposed),
    "bf16 truncated": Mutant(bf16_bits=_bf16_truncate),
    "e4m3 tie at 464 encodes NaN": Mutant(e4m3_encode=_e4m3_encode_tie_to_nan),
    "quantiser without clamp": Mutant(encode_kv=_encode_kv_no_clamp),
    "free list FIFO": Mutant(RefPagedKVCache=_FifoCache),
    "score block of 64": Mutant(block_scores=_block_scores_block64),
    "scores ignore the sink": Mutant(block_scores=_block_scores_no_sink),
    "scores pool by sum": Mutant(block_scores=_block_scores_sum),
}


@pytest.mark.parametrize("name", list(MUTANTS))
def test_planted_mistake_is_caught(name, monkeypatch):
    mut = MUTANTS[name]
    # functions that call each other inside the oracle module see the mutant too
    for k, val in mut.__dict__.items():
        if callable(val) and getattr(O, k, None) is not val:
            monkeypatch.setattr(O, k, val)
    def holds(pin):
        try:
            return pin(O)
        except (IndexError, ValueError, FloatingPointError):
            return False  # the mistake broke the oracle outright: caught

    failed = [p.__name__ for p in PINS if not holds(p)]
    assert failed, f"no pin caught the planted mistake: {name}"


# ---------------------------------------------------------------------------
# the host torch restatement timed as the CPU baseline (oracle/torch_ref.py)
# ---------------------------------------------------------------------------
from oracle import torch_ref as R  # noqa: E402


def _torch_ref_case(layout, fp8, sinks, seed):
    """A small seeded batch in both forms: torch tensors for torch_ref, numpy
    for the float64 oracle (pools of 16-token pages scattered by a
    permutation, or packed rows with cu_seqlens)."""
    g = np.random.default_rng(seed)
    Hq, Hkv, D, lens = 8, 2, 32, [1, 17, 40, 5]
    B = len(lens)
    q = g.standard_normal((B, Hq, D)).astype(np.float32)
    s_aux = g.standard_normal(Hq).astype(np.float32) if sinks else None
    case = dict(q=q, lens=lens, s_aux=s_aux)
    if layout == "paged":
        npg = [(L + 15) // 16 for L in lens]
        P = sum(npg) + 2
        perm = g.permutation(P)
        bt = np.full((B, max(npg)), -1, np.int32)
        off = 0
        for b, n in enumerate(npg):
            bt[b, :n] = perm[off:off + n]
            off += n
        shape = (P, Hkv, 16, D)
        case.update(block_table=bt)
    else:
        cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        shape = (int(cu[-1]), Hkv, D)
        case.update(cu_seqlens=cu)
    k = g.standard_normal(shape).astype(np.float32)
    v = g.standard_normal(shape).astype(np.float32)
    if fp8:
        k8, ks = O.quantize_to_fp8(k)
        v8, vs = O.quantize_to_fp8(v)
        case.update(k=k8, v=v8, k_scale=float(ks), v_scale=float(vs))
    else:
        case.update(k=k, v=v)
    return case


def _run_torch_ref(case, sink_mode, compute_dtype):
    fp8 = "k_scale" in case
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a))  # noqa: E731
    k, v = t(case["k"]), t(case["v"])
    if fp8:
        k, v = k.view(torch.float8_e4m3fn), v.view(torch.float8_e4m3fn)
    return R.decode(t(case["q"]).to(compute_dtype), k, v, case["lens"],
                    block_table=t(case.get("block_table")), cu_seqlens=t(case.get("cu_seqlens")),
                    s_aux=t(case["s_aux"]), sink_mode=sink_mode,
                    k_scale=torch.tensor(case["k_scale"]) if fp8 else None,
                    v_scale=torch.tensor(case["v_scale"]) if fp8 else None,
                    compute_dtype=compute_dtype)


def _numpy_oracle(case, sink_mode):
    q = case["q"].astype(np.float64)
    s_aux = case["s_aux"]
    ks, vs = case.get("k_scale"), case.get("v_scale")
    if "block_table" in case:
        return O.decode_paged(q, case["k"], case["v"], case["block_table"], case["lens"], s_aux, sink_mode, ks, vs)
    k, v = case["k"], case["v"]
    if ks is not None:
        k, v = O.dequantize_fp8(k, ks), O.dequantize_fp8(v, vs)
    return O.decode_varlen(q, k, v, case["cu_seqlens"], s_aux, sink_mode)


@pytest.mark.parametrize("layout", ["paged", "varlen"])
@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("sink_mode", [None, "exp", "linear"])
def test_torch_ref_matches_oracle(layout, fp8, sink_mode):
    """The CPU baseline's torch path computes the oracle's attention: to fp32
    rounding in float32, and to f16 / bf16 rounding in the inputs' dtypes."""
    case = _torch_ref_case(layout, fp8, sink_mode is not None, seed=3 + 2 * fp8)
    if sink_mode == "linear":
        # den = sum + z: a negative z can cancel most of a short sequence's
        # sum and amplify any rounding, so the half-precision comparison
        # uses non-negative sinks (float32 has the margin either way)
        case["s_aux"] = np.abs(case["s_aux"])
    mode = sink_mode or "exp"
    want = _numpy_oracle(case, mode)
    for dt, tol in ((torch.float32, 1e-5), (torch.float16, 4e-3), (torch.bfloat16, 3e-2)):
        got = _run_torch_ref(case, mode, dt).double().numpy()
        assert np.allclose(got, want, atol=tol, rtol=tol), (dt, np.abs(got - want).max())


def test_torch_ref_repeat_kv_and_mistakes_are_caught(monkeypatch):
    """repeat_kv maps query head h to KV head h // G (a planted h % Hkv map
    and a transposed page index fail the comparison above)."""
    x = torch.arange(2 * 3 * 4, dtype=torch.float32).view(2, 3, 4)
    r = R.repeat_kv(x, 3)
    assert r.shape == (6, 3, 4) and all(torch.equal(r[h], x[h // 3]) for h in range(6))
    case = _torch_ref_case("paged", False, True, seed=11)
    want = _numpy_oracle(case, "exp")
    good = _run_torch_ref(case, "exp", torch.float32).double().numpy()
    assert np.allclose(good, want, atol=1e-5)
    monkeypatch.setattr(R, "repeat_kv", lambda t, n: t.repeat(n, 1, 1))          # h % Hkv
    assert not np.allclose(_run_torch_ref(case, "exp", torch.float32).double().numpy(), want, atol=1e-3)
    monkeypatch.undo()

    def transposed_rows(k, b, length, *, block_table=None, cu_seqlens=None):
        n = (length + 15) // 16
        rows = k[block_table[b, :n].long()]
        return rows.permute(1, 2, 0, 3).reshape(rows.shape[1], n * 16, rows.shape[3])[:, :length]
    monkeypatch.setattr(R, "sequence_rows", transposed_rows)                       # t % 16 / t // 16 swapped
    assert not np.allclose(_run_torch_ref(case, "exp", torch.float32).double().numpy(), want, atol=1e-3)
