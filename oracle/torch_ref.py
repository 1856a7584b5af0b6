"""Host (CPU) torch restatement of the reference's PyTorch decode path.

TEST INFRASTRUCTURE ONLY, like decode_oracle.py: bench.py's cpu_baseline leg
times it as the CPU baseline, and tests/test_oracle.py checks it against the
float64 numpy oracle.  The product path never imports it.

It is the form the reference's own tests compute attention in, on the host:
per sequence, gather the sequence's K/V rows (pages through the block table,
or the cu_seqlens slice), widen fp8 codes as ``fp32(code) * scale`` and cast
to the compute dtype, expand the KV heads to the query heads with
``repeat_kv``, then ``matmul`` -> softmax -> ``matmul``, all in the inputs'
dtype (fp16 / bf16) unless ``compute_dtype`` says otherwise.

* repeat_kv: tests/test_triton_fd_gqa.py:8-13 (tests/test_triton_paged_gqa_decode.py:9-14)
* logits, softmax and the exp-form sink: tests/test_triton_fd_gqa.py:16-37
* per-sequence loop over the valid rows: tests/test_triton_paged_gqa_decode.py:17-38
* fp8 dequantisation ``code.to(fp32) * scale`` then the compute dtype:
  tests/test_triton_gqa_decode_fp8.py:50-53
* the linear sink (``den += sink``): fskernels/triton/triton_gqa_decode.py:111-118
"""
from __future__ import annotations

import math

import torch

PAGE = 16


def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """[Hkv, L, D] -> [Hkv * n_rep, L, D]: KV head j serves query heads j*n_rep .. j*n_rep+n_rep-1."""
    if n_rep == 1:
        return x
    hkv, length, d = x.shape
    return x[:, None, :, :].expand(hkv, n_rep, length, d).reshape(hkv * n_rep, length, d)


def sequence_rows(k, b: int, length: int, *, block_table=None, cu_seqlens=None) -> torch.Tensor:
    """Rows [0, length) of sequence b as [Hkv, L, D]: from a paged pool
    [P, Hkv, 16, D] through block_table[b], or from packed [T, Hkv, D] rows
    starting at cu_seqlens[b]."""
    if block_table is not None:
        n = (length + PAGE - 1) // PAGE
        pages = block_table[b, :n].long()
        rows = k[pages]                                   # [n, Hkv, 16, D]
        hkv, d = rows.shape[1], rows.shape[3]
        return rows.permute(1, 0, 2, 3).reshape(hkv, n * PAGE, d)[:, :length]
    start = int(cu_seqlens[b])
    return k[start:start + length].transpose(0, 1)


def attend(q, k, v, sink=None, sink_mode: str = "exp", sm_scale=None) -> torch.Tensor:
    """q [Hq, D], k/v [Hkv, L, D] in one dtype -> [Hq, D] in that dtype."""
    hq, d = q.shape
    scale = 1.0 / math.sqrt(d) if sm_scale is None else float(sm_scale)
    k = repeat_kv(k, hq // k.shape[0])
    v = repeat_kv(v, hq // v.shape[0])
    logits = torch.matmul(q.unsqueeze(1), k.transpose(-2, -1)) * scale      # [Hq, 1, L]
    if sink is None:
        probs = logits.softmax(dim=-1)
    elif sink_mode == "exp":
        z = sink.view(hq, 1, 1).to(logits.dtype)
        m = torch.maximum(logits.max(dim=-1, keepdim=True).values, z)
        e = torch.exp(logits - m)
        probs = e / (e.sum(dim=-1, keepdim=True) + torch.exp(z - m))
    elif sink_mode == "linear":
        z = sink.view(hq, 1, 1).to(logits.dtype)
        m = logits.max(dim=-1, keepdim=True).values
        e = torch.exp(logits - m)
        probs = e / (e.sum(dim=-1, keepdim=True) + z)
    else:
        raise ValueError(f"unknown sink_mode {sink_mode!r}")
    return torch.matmul(probs.to(v.dtype), v).squeeze(1)


def decode(q, k, v, lens, *, block_table=None, cu_seqlens=None, s_aux=None, sink_mode="exp",
           k_scale=None, v_scale=None, compute_dtype=None, seqs=None) -> torch.Tensor:
    """One decode step on the host: out[b] for b in ``seqs`` (default: all),
    [len(seqs), Hq, D] in the compute dtype (default q's).  fp8 pools are
    given as float8_e4m3fn tensors with k_scale / v_scale."""
    cdt = compute_dtype or q.dtype
    seqs = range(q.shape[0]) if seqs is None else seqs
    outs = []
    for b in seqs:
        length = int(lens[b])
        kb = sequence_rows(k, b, length, block_table=block_table, cu_seqlens=cu_seqlens)
        vb = sequence_rows(v, b, length, block_table=block_table, cu_seqlens=cu_seqlens)
        if k_scale is not None:
            kb = kb.to(torch.float32) * k_scale
            vb = vb.to(torch.float32) * v_scale
        outs.append(attend(q[b].to(cdt), kb.to(cdt), vb.to(cdt), s_aux, sink_mode))
    return torch.stack(outs)
