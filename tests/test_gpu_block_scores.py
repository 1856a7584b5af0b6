"""GPU parity of the pooled block scores (the TileLang kernel's S output)
against the float64 oracle: varlen and paged, f16 / bf16 / e4m3 KV, both sink
modes, lengths around block boundaries and zero, truncated and padded score
widths, fixed and automatic split sizes.  Bar: atol = rtol = 2e-3 (plus half
an ulp for bf16 scores, the final cast's own rounding); blocks past a
sequence are exactly 0.
"""
import numpy as np
import pytest
import torch

from fskernels.hip import flash_decode_gqa_varlen, paged_flash_decode
from fasterkernels_amd import workloads as W
from oracle import decode_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def close(got, want, what):
    g = got.double().cpu().numpy()
    half_ulp = np.abs(want) * (2.0 ** -8 if got.dtype == torch.bfloat16 else 0.0)  # bf16 scores only
    tol = 2e-3 + 2e-3 * np.abs(want) + half_ulp
    bad = ~(np.abs(g - want) <= tol)
    assert not bad.any(), f"{what}: {bad.sum()} bad, first {np.argwhere(bad)[0]}, got {g[bad][:3]}, want {want[bad][:3]}"
    assert (g[want == 0] == 0).all(), f"{what}: blocks past the end must be 0"


def varlen_case(lens, dtype=torch.float16, seed=0, Hq=32, Hkv=8, D=128):
    g = torch.Generator().manual_seed(seed)
    T = sum(lens)
    q = torch.randn(len(lens), Hq, D, generator=g).to(dtype)
    k = torch.randn(max(T, 1), Hkv, D, generator=g).to(dtype)
    v = torch.randn(max(T, 1), Hkv, D, generator=g).to(dtype)
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens), 0)
    sinks = torch.randn(Hq, generator=g)
    return q, k, v, cu, sinks


@pytest.mark.parametrize("sink_mode", [None, "exp", "linear"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_varlen_block_scores(sink_mode, dtype):
    lens = [0, 1, 127, 128, 129, 1000, 3000]
    q, k, v, cu, sinks = varlen_case(lens, dtype, seed=3)
    s_aux = None if sink_mode is None else (sinks.abs() + 0.5 if sink_mode == "linear" else sinks)
    out, S = flash_decode_gqa_varlen(q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV),
                                     None if s_aux is None else s_aux.to(DEV), sink_mode=sink_mode or "exp",
                                     return_block_scores=True)
    torch.cuda.synchronize()
    T = sum(lens)
    assert S.shape == (7, 32, -(-T // 128)) and S.dtype == dtype
    want = O.block_scores_varlen(q.double().numpy(), k.double().numpy(), cu.numpy(),
                                 None if s_aux is None else s_aux.double().numpy(), sink_mode or "exp",
                                 n_blocks=S.shape[2])
    close(S, want, f"varlen {dtype} sink={sink_mode}")
    # the attention output itself is unchanged by asking for scores
    plain = flash_decode_gqa_varlen(q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV),
                                    None if s_aux is None else s_aux.to(DEV), sink_mode=sink_mode or "exp")
    torch.cuda.synchronize()
    o, p = out.double().cpu(), plain.double().cpu()
    both = torch.isnan(o) & torch.isnan(p)
    assert torch.equal(torch.isnan(o), torch.isnan(p))
    assert ((o - p).abs()[~both] <= 2e-3 + 2e-3 * p.abs()[~both]).all()


@pytest.mark.parametrize("kv", ["f16", "e4m3"])
def test_paged_block_scores(kv):
    name = "C3" if kv == "f16" else "C5"
    wl = W.make(name, overrides=dict(B=6, lens=("list", [5, 128, 300, 2000, 4097, 0])), seed=7)
    d = wl.to(DEV)
    out, S = paged_flash_decode(d.q, d.k, d.v, d.block_table, d.seq_lens, 16, s_aux=d.s_aux, k_scale=d.k_scale,
                                v_scale=d.v_scale, out_dtype=d.out_dtype, sink_mode="exp",
                                return_block_scores=True)
    torch.cuda.synchronize()
    assert S.shape == (6, 32, -(-wl.block_table.shape[1] * 16 // 128))
    if kv == "e4m3":
        kp = wl.k.view(torch.uint8).numpy()
        want = O.block_scores_paged(wl.q.double().numpy(), kp, wl.block_table.numpy(), wl.lens,
                                    wl.s_aux.double().numpy(), "exp", n_blocks=S.shape[2],
                                    k_scale=np.float32(wl.k_scale))
    else:
        want = O.block_scores_paged(wl.q.double().numpy(), wl.k.double().numpy(), wl.block_table.numpy(),
                                    wl.lens, None, "exp", n_blocks=S.shape[2])
    close(S, want, f"paged {kv}")


def test_score_width_chunks_and_errors():
    lens = [700, 1, 2100]
    q, k, v, cu, _ = varlen_case(lens, seed=5)
    args = (q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV))
    qd, kd = q.double().numpy(), k.double().numpy()
    for width in (3, 40):             # truncated (longer sequences lose blocks) and padded with zeros
        for chunk in (0, 128, 384):
            _, S = flash_decode_gqa_varlen(*args, return_block_scores=True, score_blocks=width, chunk_tokens=chunk,
                                           out_dtype=torch.float32)
            torch.cuda.synchronize()
            close(S, O.block_scores_varlen(qd, kd, cu.numpy(), n_blocks=width), f"width {width} chunk {chunk}")
    with pytest.raises(ValueError, match="multiple of 128"):
        flash_decode_gqa_varlen(*args, return_block_scores=True, chunk_tokens=96)
    with pytest.raises(ValueError):
        flash_decode_gqa_varlen(*args, return_block_scores=True, score_blocks=0)


def test_binding_rejects_bad_score_tensors():
    """The torch binding checks the score tensor it is handed (the reduce
    kernel writes a contiguous [B, Hq, n] array in the output dtype)."""
    from fasterkernels_amd import native as nat

    q, k, v, cu, _ = varlen_case([300, 5], seed=6)
    q, k, v, cu = q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV)
    stream = nat.raw_stream(q.get_device())
    ext = nat.ext()
    bad = [torch.empty(2, 32, dtype=torch.float16, device=DEV),                    # rank 2
           torch.empty(3, 32, 4, dtype=torch.float16, device=DEV),                 # batch 3 for 2
           torch.empty(2, 16, 4, dtype=torch.float16, device=DEV),                 # 16 heads for 32
           torch.empty(2, 32, 4, dtype=torch.float32, device=DEV),                 # not the output dtype
           torch.empty(2, 32, 8, dtype=torch.float16, device=DEV)[:, :, ::2]]      # not contiguous
    for s in bad:
        with pytest.raises(ValueError, match="scores must be"):
            ext.varlen(q, k, v, cu, None, None, None, -1, 0, None, 0, s, stream)
    good = torch.empty(2, 32, 4, dtype=torch.float16, device=DEV)
    out = ext.varlen(q, k, v, cu, None, None, None, -1, 0, None, 0, good, stream)
    torch.cuda.synchronize()
    assert out.shape == (2, 32, 128) and torch.isfinite(good.float()).all()


@pytest.mark.parametrize("name", ["M0", "C2"])
def test_block_scores_bench_sizes(name):
    """The `--block-scores` bench workloads at their sizes: M0 (paged, 4 x
    32768 tokens: 128-token-rounded chunk pairs of the XCD skew) and C2
    (varlen with exp sinks), scores and output against the oracle."""
    wl = W.make(name)
    d = wl.to(DEV)
    if wl.layout == "paged":
        out, S = paged_flash_decode(d.q, d.k, d.v, d.block_table, d.seq_lens, 16, s_aux=d.s_aux,
                                    sink_mode="exp", return_block_scores=True)
        want = O.block_scores_paged(wl.q.double().numpy(), wl.k.numpy(), wl.block_table.numpy(), wl.lens,
                                    None if wl.s_aux is None else wl.s_aux.double().numpy(), "exp",
                                    n_blocks=S.shape[2])
        ref = O.decode_paged(wl.q.double().numpy(), wl.k.numpy(), wl.v.numpy(), wl.block_table.numpy(), wl.lens,
                             None if wl.s_aux is None else wl.s_aux.double().numpy())
    else:
        out, S = flash_decode_gqa_varlen(d.q, d.k, d.v, d.cu_seqlens, d.s_aux, sink_mode="exp",
                                         return_block_scores=True)
        want = O.block_scores_varlen(wl.q.double().numpy(), wl.k.numpy(), wl.cu_seqlens.numpy(),
                                     wl.s_aux.double().numpy(), "exp", n_blocks=S.shape[2])
        ref = O.decode_varlen(wl.q.double().numpy(), wl.k.double().numpy(), wl.v.double().numpy(),
                              wl.cu_seqlens.numpy(), wl.s_aux.double().numpy())
    torch.cuda.synchronize()
    close(S, want, f"{name} block scores")
    o = out.double().cpu().numpy()
    assert (np.abs(o - ref) <= 2e-3 + 2e-3 * np.abs(ref) + np.abs(ref) * 2.0 ** -11).all(), f"{name} output"
