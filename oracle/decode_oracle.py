"""CPU oracle for the GQA flash-decode hot path (numpy, float64).

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the checker or the timed
CPU baseline.  The product path (fskernels, fasterkernels_amd) never imports it and has no
CPU fallback.

It restates, in plain numpy, what the reference computes on the decode path:

* GQA attention for one query token per sequence: query head h reads KV head
  h // (Hq / Hkv) (repeat_kv, tests/test_triton_fd_gqa.py:8-13; head mapping
  fskernels/triton/triton_gqa_decode.py:53-56), scores q.k * sm_scale with
  sm_scale = 1/sqrt(D) (:70-71, :86-87), softmax over the valid tokens.
* Sinks, two semantics (a per-query-head value z):
    "exp"    -- z is an extra logit with a zero value vector:
                p_t = e^{s_t - M} / (sum e^{s - M} + e^{z - M}), M = max(max s, z)
                (tests/test_triton_fd_gqa.py:117-132, :27-33)
    "linear" -- z is added to the softmax denominator relative to m = max s:
                den = sum e^{s - m} + z
                (fskernels/triton/triton_gqa_decode.py:111-118;
                 fskernels/cuda/flash_decode_cuda.cu:151-153)
* Varlen packing through cu_seqlens (triton_gqa_decode.py:66-68, :81).
* Paged addressing: token t of sequence b is pool[block_table[b, t // ps], h,
  t % ps] (fskernels/paged_attn/triton_paged_attn.py:57-69), tokens >= seq_len
  masked (:71-79).
* Dense HF cache: tokens [start_k_offsets[b], cache_lens[b]) of
  k[b, h, :, :] (fskernels/triton/triton_gqa_decode_hf.py:46-54, :62-64).
* Split-KV partials and their log-sum-exp merge
  (triton_gqa_decode_hf.py:52-54, :90-99, :103-137).
* Pooled block scores (the TileLang kernel's S output): the largest
  attention probability within each 128-token block.
* The KV write path: PagedKVCache's page bookkeeping and row stores
  (fskernels/paged_attn/paged_kv_cache.py:44-141) restated as
  RefPagedKVCache, and the slot-addressed batch store paged_write with the
  element encodings a pool can hold (f16 / bf16 round to nearest even, e4m3
  plain cast or fixed-scale quantisation).
* e4m3fn (OCP FP8, torch.float8_e4m3fn) decoding from the format definition,
  encoding with round-to-nearest-even, and the per-tensor quantiser
  scale = max|x|.clamp(1e-12) / 448, x8 = e4m3(clamp(x / scale, +-448))
  (fskernels/triton/triton_gqa_decode_hf_fp8.py:9-16); dequantised values are
  fp32(code) * scale (:47-50, :71-73, :90-92).

Every function is pinned by tests/test_oracle.py (closed forms, a library
routine -- torch's scaled_dot_product_attention and its float8 cast --,
brute-force loops on tiny inputs, committed golden vectors and planted
mistakes that must be caught).
"""
from __future__ import annotations

import math

import numpy as np

E4M3_MAX = 448.0


# ---------------------------------------------------------------------------
# e4m3fn codec (OCP OFP8 E4M3: bias 7, no infinities, S.1111.111 = NaN)
# ---------------------------------------------------------------------------
def e4m3_decode(codes) -> np.ndarray:
    """uint8 codes -> float32 values, from the bit-level definition."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    exp = (c >> 3) & 0xF
    man = c & 0x7
    normal = (1.0 + man / 8.0) * np.power(2.0, exp - 7.0)
    subnormal = (man / 8.0) * 2.0 ** -6
    val = sign * np.where(exp == 0, subnormal, normal)
    val = np.where((c & 0x7F) == 0x7F, np.nan, val)
    return val.astype(np.float32)


_E4M3_POS = e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)  # codes 0..126


def e4m3_encode(x) -> np.ndarray:
    """float -> uint8 code, round to nearest (ties to even code), NaN -> 0x7F.

    Magnitudes above 448 are not clamped here (the quantiser clamps first,
    triton_gqa_decode_hf_fp8.py:15); they round to 448 up to the 464 midpoint
    (the tie goes to the even code 448), beyond it they encode NaN, as torch's
    float8_e4m3fn cast does.
    """
    x = np.asarray(x, dtype=np.float64)
    a = np.abs(x)
    idx = np.searchsorted(_E4M3_POS, a, side="left")
    idx = np.clip(idx, 1, len(_E4M3_POS) - 1)
    lo = _E4M3_POS[idx - 1]
    hi = _E4M3_POS[idx]
    pick_hi = (a - lo > hi - a) | ((a - lo == hi - a) & ((idx % 2) == 0))
    code = np.where(pick_hi, idx, idx - 1)
    code = np.where(a <= _E4M3_POS[0], 0, code)
    code = np.where(a > 464.0, 0x7F, code)  # past the last midpoint (464 ties to 448): NaN
    code = np.where(np.isnan(a), 0x7F, code)
    sign = np.where(np.signbit(x), 0x80, 0)
    return (code | sign).astype(np.uint8)


def quantize_to_fp8(x):
    """(codes uint8, scale float32) as the reference quantiser computes them."""
    x32 = np.asarray(x, dtype=np.float32)
    amax = np.float32(np.abs(x32).max()) if x32.size else np.float32(0)
    scale = np.float32(max(amax, np.float32(1e-12)) / np.float32(E4M3_MAX))
    y = np.clip(x32 / scale, -E4M3_MAX, E4M3_MAX).astype(np.float32)
    return e4m3_encode(y), scale


# e4m3_decode of every code, indexed by code (dequantising a large pool is a
# table lookup; the values are e4m3_decode's own)
_E4M3_TABLE = e4m3_decode(np.arange(256, dtype=np.uint8))


def dequantize_fp8(codes, scale) -> np.ndarray:
    return (_E4M3_TABLE[np.asarray(codes, dtype=np.uint8)] * np.float32(scale)).astype(np.float32)


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------
def attend(q, k, v, sink=None, sink_mode: str = "exp", sm_scale: float | None = None):
    """One decode step of one sequence.

    q [Hq, D]; k, v [L, Hkv, D]; sink [Hq] or None.  Returns [Hq, D] float64.
    Query head h uses KV head h // (Hq // Hkv).  L = 0 gives NaN without a sink
    (0/0, as the reference kernels produce) and the sink-only result with one.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    Hq, D = q.shape
    L, Hkv, _ = k.shape
    G = Hq // Hkv
    scale = 1.0 / math.sqrt(D) if sm_scale is None else float(sm_scale)
    out = np.empty((Hq, D), dtype=np.float64)
    for kvh in range(Hkv):
        qs = q[kvh * G:(kvh + 1) * G]                  # [G, D]
        s = (qs @ k[:, kvh, :].T) * scale              # [G, L]
        m = s.max(axis=1, keepdims=True) if L else np.full((G, 1), -np.inf)
        if sink is not None and sink_mode == "exp":
            z = np.asarray(sink, dtype=np.float64)[kvh * G:(kvh + 1) * G, None]
            M = np.maximum(m, z)
            e = np.exp(s - M)
            den = e.sum(axis=1, keepdims=True) + np.exp(z - M)
        else:
            with np.errstate(invalid="ignore"):
                e = np.exp(s - m)
            den = e.sum(axis=1, keepdims=True)
            if sink is not None:
                if sink_mode != "linear":
                    raise ValueError(f"unknown sink_mode {sink_mode!r}")
                den = den + np.asarray(sink, dtype=np.float64)[kvh * G:(kvh + 1) * G, None]
        with np.errstate(invalid="ignore", divide="ignore"):
            out[kvh * G:(kvh + 1) * G] = (e @ v[:, kvh, :]) / den
    return out


def decode_varlen(q, k, v, cu_seqlens, s_aux=None, sink_mode="exp", sm_scale=None):
    """q [B, Hq, D]; k, v [T, Hkv, D]; cu_seqlens [B+1] -> [B, Hq, D]."""
    q = np.asarray(q)
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    return np.stack([attend(q[b], k[cu[b]:cu[b + 1]], v[cu[b]:cu[b + 1]], s_aux, sink_mode, sm_scale)
                     for b in range(q.shape[0])])


def paged_rows(pool, block_table, b: int, length: int):
    """Rows [0, length) of sequence b gathered from pool [P, Hkv, ps, D] -> [L, Hkv, D]."""
    pool = np.asarray(pool)
    ps = pool.shape[2]
    t = np.arange(length)
    pages = np.asarray(block_table)[b, t // ps]
    return pool[pages, :, t % ps, :]


def paged_gather(pool, block_table, seq_lens):
    """Dense [B, Hkv, max_blocks*ps, D] copy of a pool; rows >= seq_len are zero."""
    pool = np.asarray(pool)
    bt = np.asarray(block_table)
    B, MB = bt.shape
    P, Hkv, ps, D = pool.shape
    out = np.zeros((B, Hkv, MB * ps, D), dtype=pool.dtype)
    for b in range(B):
        L = int(seq_lens[b])
        out[b, :, :L, :] = paged_rows(pool, bt, b, L).transpose(1, 0, 2)
    return out


def decode_paged(q, k_pool, v_pool, block_table, seq_lens, s_aux=None, sink_mode="exp",
                 k_scale=None, v_scale=None, sm_scale=None):
    """q [B, Hq, D]; pools [P, Hkv, ps, D] (float values, or uint8 e4m3 codes when
    k_scale / v_scale are given) -> [B, Hq, D]."""
    q = np.asarray(q)
    outs = []
    for b in range(q.shape[0]):
        L = int(seq_lens[b])
        k = paged_rows(k_pool, block_table, b, L)
        v = paged_rows(v_pool, block_table, b, L)
        if k_scale is not None:
            k = dequantize_fp8(k, k_scale)
        if v_scale is not None:
            v = dequantize_fp8(v, v_scale)
        outs.append(attend(q[b], k, v, s_aux, sink_mode, sm_scale))
    return np.stack(outs)


def decode_dense(q, k, v, cache_lens, start_offsets=None, s_aux=None, sink_mode="exp",
                 k_scale=None, v_scale=None, sm_scale=None):
    """q [B, Hq, D]; k, v [B, Hkv, S, D] -> [B, Hq, D] over rows [start, len)."""
    q = np.asarray(q)
    outs = []
    for b in range(q.shape[0]):
        e = int(cache_lens[b])
        s = 0 if start_offsets is None else int(start_offsets[b])
        kb = np.asarray(k)[b, :, s:e, :].transpose(1, 0, 2)
        vb = np.asarray(v)[b, :, s:e, :].transpose(1, 0, 2)
        if k_scale is not None:
            kb = dequantize_fp8(kb, k_scale)
        if v_scale is not None:
            vb = dequantize_fp8(vb, v_scale)
        outs.append(attend(q[b], kb, vb, s_aux, sink_mode, sm_scale))
    return np.stack(outs)


# ---------------------------------------------------------------------------
# pooled block scores
# ---------------------------------------------------------------------------
SCORE_BLOCK = 128


def block_scores(q, k, sink=None, sink_mode: str = "exp", sm_scale=None, n_blocks=None,
                 block: int = SCORE_BLOCK):
    """[Hq, n_blocks]: for each 128-token block of one sequence, the largest
    final attention probability of its tokens (0 for blocks past the end).

    Restates the S output of fskernels/tilelang/tilelang_gqa_decode.py:
    block maxima of the scores (:102-103) turned into probabilities with the
    final maximum and denominator (:123-124), the sink folded into the
    denominator (:117-120; "exp" mode adds e^z instead).  q [Hq, D];
    k [L, Hkv, D]."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    Hq, D = q.shape
    L, Hkv, _ = k.shape
    G = Hq // Hkv
    nb = -(-L // block)
    n_blocks = nb if n_blocks is None else int(n_blocks)
    out = np.zeros((Hq, n_blocks))
    if L == 0:
        return out
    scale = 1.0 / math.sqrt(D) if sm_scale is None else float(sm_scale)
    s = np.stack([k[:, h // G, :] @ q[h] for h in range(Hq)]) * scale      # [Hq, L]
    m = s.max(axis=1, keepdims=True)
    if sink is not None and sink_mode == "exp":
        z = np.asarray(sink, dtype=np.float64)[:, None]
        M = np.maximum(m, z)
        e = np.exp(s - M)
        den = e.sum(axis=1, keepdims=True) + np.exp(z - M)
    else:
        e = np.exp(s - m)
        den = e.sum(axis=1, keepdims=True)
        if sink is not None:
            den = den + np.asarray(sink, dtype=np.float64)[:, None]
    p = e / den
    for j in range(min(nb, n_blocks)):
        out[:, j] = p[:, j * block:(j + 1) * block].max(axis=1)
    return out


def block_scores_varlen(q, k, cu_seqlens, s_aux=None, sink_mode="exp", sm_scale=None, n_blocks=1):
    """[B, Hq, n_blocks] block scores of varlen-packed sequences."""
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    return np.stack([block_scores(q[b], k[cu[b]:cu[b + 1]], s_aux, sink_mode, sm_scale, n_blocks)
                     for b in range(len(q))])


def block_scores_paged(q, k_pool, block_table, seq_lens, s_aux=None, sink_mode="exp", sm_scale=None,
                       n_blocks=1, k_scale=None):
    """[B, Hq, n_blocks] block scores through the paged addressing."""
    outs = []
    for b in range(len(q)):
        k = paged_rows(k_pool, block_table, b, int(seq_lens[b]))
        if k_scale is not None:
            k = dequantize_fp8(k, k_scale)
        outs.append(block_scores(q[b], k, s_aux, sink_mode, sm_scale, n_blocks))
    return np.stack(outs)


# ---------------------------------------------------------------------------
# split-KV partials and their merge
# ---------------------------------------------------------------------------
def partials(q, k, v, n_splits: int, sm_scale=None):
    """Split the L tokens into n_splits ranges of ceil(L/n) tokens and return
    (acc [n, Hq, D] unnormalised, m [n, Hq], l [n, Hq]) per range, as the
    dense split kernel produces them (triton_gqa_decode_hf.py:52-54, :90-99).
    Empty ranges give m = -inf, l = 0, acc = 0."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    Hq, D = q.shape
    L, Hkv, _ = k.shape
    G = Hq // Hkv
    scale = 1.0 / math.sqrt(D) if sm_scale is None else float(sm_scale)
    tps = -(-L // n_splits) if L else 0
    acc = np.zeros((n_splits, Hq, D))
    m = np.full((n_splits, Hq), -np.inf)
    l = np.zeros((n_splits, Hq))
    for i in range(n_splits):
        lo, hi = i * tps, min((i + 1) * tps, L)
        if lo >= hi:
            continue
        for h in range(Hq):
            s = (k[lo:hi, h // G, :] @ q[h]) * scale
            m[i, h] = s.max()
            e = np.exp(s - m[i, h])
            l[i, h] = e.sum()
            acc[i, h] = e @ v[lo:hi, h // G, :]
    return acc, m, l


def merge_partials(acc, m, l, sink=None, sink_mode="exp"):
    """Log-sum-exp merge (triton_gqa_decode_hf.py:117-135) plus the sink fold."""
    acc = np.asarray(acc, dtype=np.float64)
    m = np.asarray(m, dtype=np.float64)
    l = np.asarray(l, dtype=np.float64)
    M = m.max(axis=0)                                   # [Hq]
    Mu = np.where(np.isneginf(M), 0.0, M)
    w = np.exp(m - Mu)                                  # [n, Hq]
    den = (l * w).sum(axis=0)
    num = (acc * w[:, :, None]).sum(axis=0)
    if sink is not None:
        z = np.asarray(sink, dtype=np.float64)
        if sink_mode == "exp":
            Mn = np.maximum(M, z)
            f = np.exp(Mu - Mn)
            den = den * f + np.exp(z - Mn)
            num = num * f[:, None]
        else:
            den = den + z
    with np.errstate(invalid="ignore", divide="ignore"):
        return num / den[:, None]


# ---------------------------------------------------------------------------
# KV write path
# ---------------------------------------------------------------------------
def bf16_bits(x) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16), round to nearest, ties to even.

    NaN maps to 0x7FC0 here; the write kernels keep NaN a NaN but its payload
    is not pinned."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), r)


def bf16_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def encode_kv(x, pool_dtype: str, scale=None) -> np.ndarray:
    """Pool elements for float32 values x.

    'f16'  -> float16, round to nearest even (numpy's conversion);
    'bf16' -> uint16 bfloat16 bits (bf16_bits);
    'e4m3' -> uint8 codes: with a scale, e4m3(clamp(x / scale, -448, 448)) in
              fp32 -- the quantiser of triton_gqa_decode_hf_fp8.py:13-16 with a
              fixed scale; without one, the plain e4m3fn cast that a torch copy
              into an e4m3 pool performs (paged_kv_cache.py:129-130).
    """
    x = np.asarray(x, dtype=np.float32)
    if pool_dtype == "f16":
        with np.errstate(over="ignore"):
            return x.astype(np.float16)
    if pool_dtype == "bf16":
        return bf16_bits(x)
    if pool_dtype == "e4m3":
        if scale is not None:
            with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
                x = np.clip(x / np.float32(scale), -E4M3_MAX, E4M3_MAX).astype(np.float32)
        return e4m3_encode(x)
    raise ValueError(f"unknown pool dtype {pool_dtype!r}")


def paged_store_rows(pool, slots, rows):
    """Stores row i of rows [n, Hkv, D] (already in the pool's element type) at
    page slots[i] // ps, row slots[i] % ps of every head of pool [P, Hkv, ps, D]
    (in place, returned).  Slots outside [0, P * ps) are skipped.  Restates the
    per-token row store of paged_kv_cache.py:117-130 for a batch of slots; a
    store between equal element types is this byte copy."""
    P, Hkv, ps, D = pool.shape
    rows = np.asarray(rows).reshape(-1, Hkv, D)
    for i, s in enumerate(np.asarray(slots, dtype=np.int64).reshape(-1)):
        if 0 <= s < P * ps:
            pool[s // ps, :, s % ps, :] = rows[i]
    return pool


def paged_write(pool, slots, x, pool_dtype: str, scale=None):
    """paged_store_rows of float32 values x [n, Hkv, D] encoded for the pool."""
    Hkv, D = pool.shape[1], pool.shape[3]
    enc = encode_kv(np.asarray(x, dtype=np.float32).reshape(-1, Hkv, D), pool_dtype, scale)
    return paged_store_rows(pool, slots, enc)


_POOL_NP = {"f16": np.float16, "bf16": np.uint16, "e4m3": np.uint8}


class RefPagedKVCache:
    """Restatement of fskernels/paged_attn/paged_kv_cache.py:44-141 in numpy.

    Pools [L, P, Hkv, 16, D] hold encoded elements (encode_kv), zero-filled
    (:46-50); block_table [max_seqs, max_blocks] int32 starts at -1 (:53-56);
    the free list starts as [0, 1, ..., P-1] and pages are popped from its end
    (:61, :103-106); allocate_sequence takes the lowest inactive slot (:85-91);
    free_sequence returns a sequence's pages in logical order (:93-101);
    append_kv stores token pos at page block_table[s, pos // 16], row pos % 16,
    taking a new page when pos % 16 == 0, and advances the length (:109-132).
    """

    page_size = 16

    def __init__(self, num_layers, num_pages, max_seqs, max_blocks, num_kv_heads, head_dim,
                 pool_dtype="f16", k_scale=None, v_scale=None):
        shape = (num_layers, num_pages, num_kv_heads, self.page_size, head_dim)
        self.k_pool = np.zeros(shape, dtype=_POOL_NP[pool_dtype])
        self.v_pool = np.zeros(shape, dtype=_POOL_NP[pool_dtype])
        self.block_table = np.full((max_seqs, max_blocks), -1, dtype=np.int32)
        self.seq_lens = [0] * max_seqs
        self.active = [False] * max_seqs
        self.free_pages = list(range(num_pages))
        self.pool_dtype, self.k_scale, self.v_scale = pool_dtype, k_scale, v_scale

    def allocate_sequence(self) -> int:
        for sid, on in enumerate(self.active):
            if not on:
                self.active[sid] = True
                self.seq_lens[sid] = 0
                return sid
        raise RuntimeError("All sequence slots are occupied")

    def free_sequence(self, sid: int) -> None:
        n_pages = -(-self.seq_lens[sid] // self.page_size)
        for lp in range(n_pages):
            pp = int(self.block_table[sid, lp])
            if pp >= 0:
                self.free_pages.append(pp)
                self.block_table[sid, lp] = -1
        self.active[sid] = False
        self.seq_lens[sid] = 0

    def append_kv(self, sid: int, layer: int, k, v) -> None:
        """k, v: [Hkv, D] float32 values of one token."""
        pos = self.seq_lens[sid]
        lp, off = divmod(pos, self.page_size)
        if off == 0:
            if not self.free_pages:
                raise RuntimeError("Out of KV pages")
            pp = self.free_pages.pop()
            self.block_table[sid, lp] = pp
        else:
            pp = int(self.block_table[sid, lp])
        self.k_pool[layer, pp, :, off, :] = encode_kv(k, self.pool_dtype, self.k_scale)
        self.v_pool[layer, pp, :, off, :] = encode_kv(v, self.pool_dtype, self.v_scale)
        self.seq_lens[sid] = pos + 1
