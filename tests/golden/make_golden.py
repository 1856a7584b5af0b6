"""Writes the golden decode vectors in tests/golden/ (run: python tests/golden/make_golden.py).

The expected outputs are computed by brute force in pure Python (math.exp,
explicit loops over heads, tokens and head_dim), directly from the
definitions the reference's test oracles use:

* query head h reads KV head h // (Hq // Hkv)        (tests/test_triton_fd_gqa.py:8-13)
* s_t = sum_d q[h,d] k[t,kv,d] / sqrt(D)               (:22, :110-115)
* no sink:     p_t = e^{s_t - m} / sum_u e^{s_u - m}   (:28, :118)
* exp sink z:  p_t = e^{s_t - M} / (sum_u e^{s_u - M} + e^{z - M}), M = max(m, z)  (:117-132)
* linear sink: p_t = e^{s_t - m} / (sum_u e^{s_u - m} + z)  (the reference kernels'
  fold, fskernels/triton/triton_gqa_decode.py:111-118)
* out[h] = sum_t p_t v[t,kv]
* paged: token t of sequence b is pool[block_table[b, t // 16], kv, t % 16]
  (fskernels/paged_attn/triton_paged_attn.py:57-69)
* e4m3 dequant: sign * 2^(e-7) * (1 + m/8), subnormal 2^-6 * m/8, code*scale
  (OCP FP8 E4M3; fskernels/triton/triton_gqa_decode_hf_fp8.py:71-73, :90-92)

Inputs are small (so the loops finish in seconds), seeded, and rounded to
fp16-representable values.  It does not import the oracle or the product.
"""
from __future__ import annotations

import math
import os
import random

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def f16(x: float) -> float:
    return float(np.float16(x))


def brute_attend(q, k, v, sink=None, mode="none"):
    """q: [Hq][D]; k, v: [L][Hkv][D] nested lists -> [Hq][D]."""
    Hq, D = len(q), len(q[0])
    L = len(k)
    Hkv = len(k[0]) if L else 1
    G = Hq // Hkv
    out = []
    for h in range(Hq):
        kv = h // G
        s = [sum(q[h][d] * k[t][kv][d] for d in range(D)) / math.sqrt(D) for t in range(L)]
        m = max(s) if s else -math.inf
        if mode == "exp":
            M = max(m, sink[h])
            e = [math.exp(x - M) for x in s]
            den = sum(e) + math.exp(sink[h] - M)
        else:
            e = [math.exp(x - m) for x in s]
            den = sum(e) + (sink[h] if mode == "linear" else 0.0)
        out.append([sum(e[t] * v[t][kv][d] for t in range(L)) / den for d in range(D)])
    return out


def e4m3_value(code: int) -> float:
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 0x7
    if e == 0xF and m == 0x7:
        return math.nan
    if e == 0:
        return s * (m / 8.0) * 2.0 ** -6
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def main():
    rng = random.Random(20261201)

    def rnd(*shape):
        if len(shape) == 1:
            return [f16(rng.gauss(0, 1)) for _ in range(shape[0])]
        return [rnd(*shape[1:]) for _ in range(shape[0])]

    # ---- varlen: B=3, Hq=8, Hkv=2 (G=4), D=16, lens 1, 5, 19
    Hq, Hkv, D = 8, 2, 16
    lens = [1, 5, 19]
    T = sum(lens)
    q = rnd(3, Hq, D)
    k = rnd(T, Hkv, D)
    v = rnd(T, Hkv, D)
    sink = [f16(rng.gauss(0, 1)) for _ in range(Hq)]
    cu = [0]
    for L in lens:
        cu.append(cu[-1] + L)
    outs = {}
    for mode in ("none", "exp", "linear"):
        outs[mode] = [brute_attend(q[b], k[cu[b]:cu[b + 1]], v[cu[b]:cu[b + 1]], sink, mode)
                      for b in range(3)]
    np.savez_compressed(os.path.join(HERE, "varlen_small.npz"), q=np.array(q), k=np.array(k),
                        v=np.array(v), cu_seqlens=np.array(cu, dtype=np.int32),
                        s_aux=np.array(sink), out_none=np.array(outs["none"]),
                        out_exp=np.array(outs["exp"]), out_linear=np.array(outs["linear"]))

    # ---- paged: B=2, lens 17, 40, page size 16, pool of 7 pages (2 spare), shuffled
    lens = [17, 40]
    npages = [(L + 15) // 16 for L in lens]
    P = sum(npages) + 2
    pool_k = rnd(P, Hkv, 16, D)
    pool_v = rnd(P, Hkv, 16, D)
    ids = list(range(P))
    rng.shuffle(ids)
    bt = [[-1] * max(npages) for _ in lens]
    for b, n in enumerate(npages):
        for j in range(n):
            bt[b][j] = ids.pop()
    qp = rnd(2, Hq, D)
    outp = []
    for b, L in enumerate(lens):
        kk = [[pool_k[bt[b][t // 16]][kv][t % 16] for kv in range(Hkv)] for t in range(L)]
        vv = [[pool_v[bt[b][t // 16]][kv][t % 16] for kv in range(Hkv)] for t in range(L)]
        outp.append(brute_attend(qp[b], kk, vv))
    np.savez_compressed(os.path.join(HERE, "paged_small.npz"), q=qp, k_pool=np.array(pool_k),
                        v_pool=np.array(pool_v), block_table=np.array(bt, dtype=np.int32),
                        seq_lens=np.array(lens, dtype=np.int32), out=np.array(outp))

    # ---- fp8 paged: codes drawn uniformly from the finite e4m3 codes, power-of-two scales
    finite = [c for c in range(256) if (c & 0x7F) != 0x7F]
    kc = [[[[rng.choice(finite) for _ in range(D)] for _ in range(16)] for _ in range(Hkv)] for _ in range(P)]
    vc = [[[[rng.choice(finite) for _ in range(D)] for _ in range(16)] for _ in range(Hkv)] for _ in range(P)]
    sk, sv = 1.0 / 64, 1.0 / 32  # exact in fp32
    outf = []
    for b, L in enumerate(lens):
        kk = [[[e4m3_value(x) * sk for x in kc[bt[b][t // 16]][kv][t % 16]] for kv in range(Hkv)]
              for t in range(L)]
        vv = [[[e4m3_value(x) * sv for x in vc[bt[b][t // 16]][kv][t % 16]] for kv in range(Hkv)]
              for t in range(L)]
        outf.append(brute_attend(qp[b], kk, vv, sink, "exp"))
    np.savez_compressed(os.path.join(HERE, "paged_fp8_small.npz"), q=qp,
                        k_codes=np.array(kc, dtype=np.uint8), v_codes=np.array(vc, dtype=np.uint8),
                        k_scale=np.float32(sk), v_scale=np.float32(sv), s_aux=np.array(sink),
                        block_table=np.array(bt, dtype=np.int32),
                        seq_lens=np.array(lens, dtype=np.int32), out=np.array(outf))

    # ---- e4m3 decode table from the bit-level definition
    np.savez_compressed(os.path.join(HERE, "e4m3_table.npz"),
                        values=np.array([e4m3_value(c) for c in range(256)]))
    print("golden vectors written to", HERE)


if __name__ == "__main__":
    main()
