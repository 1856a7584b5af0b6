"""GPU parity of the HF attention patch (fskernels.hip.hf).

Decode steps through the patch are compared with transformers' eager
attention evaluated in float32 on the same inputs and mask (bar: atol = rtol
= 2e-3 plus half an ulp of the output dtype), and with the float64 oracle for
the cache_position / sliding-window path.  The fp8 patch is compared with the
oracle over its own quantised inputs (atol 1e-2, the fp8 bar).  A tiny random
Qwen3 model runs prefill + decode end to end with the patch installed.
"""
import numpy as np
import pytest
import torch

transformers = pytest.importorskip("transformers")

from fskernels.hip import hf as H  # noqa: E402
from oracle import decode_oracle as O  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda"
NEG = torch.finfo(torch.float32).min


class _Attn(torch.nn.Module):
    def __init__(self, groups):
        super().__init__()
        self.num_key_value_groups = groups


def eager_f32(q, k, v, mask, scaling):
    """transformers' eager attention in float32 on the same tensors, as [B, Hq, D]."""
    m = _Attn(q.shape[1] // k.shape[1]).to(DEV)
    out, _ = H.native_eager_attention_forward(m, q.float(), k.float(), v.float(),
                                              None if mask is None else mask.float(), scaling)
    return out[:, 0]


def check(out, ref, atol=2e-3, rtol=2e-3, what=""):
    o = out.float()
    r = ref.float()
    half_ulp = r.abs() * (2.0 ** -8 if out.dtype == torch.bfloat16 else 0.0)  # bf16 outputs only
    err = (o - r).abs()
    tol = atol + rtol * r.abs() + half_ulp
    assert (err <= tol).all(), f"{what}: max err/tol {(err / tol).max().item():.3f}"


def case(B=3, Hq=16, Hkv=4, S=300, D=128, dtype=torch.bfloat16, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, 1, D, generator=g).to(dtype).to(DEV)
    k = torch.randn(B, Hkv, S, D, generator=g).to(dtype).to(DEV)
    v = torch.randn(B, Hkv, S, D, generator=g).to(dtype).to(DEV)
    return q, k, v


def mask_from_ranges(B, S, starts, ends):
    idx = torch.arange(S)
    ok = (idx[None] >= torch.tensor(starts)[:, None]) & (idx[None] < torch.tensor(ends)[:, None])
    return torch.where(ok, 0.0, NEG)[:, None, None, :].to(DEV)


@pytest.mark.parametrize("name,starts,ends", [
    ("dynamic cache", [0, 0, 0], [300, 300, 300]),
    ("left padding", [0, 37, 299], [300, 300, 300]),
    ("static cache tail", [0, 0, 0], [1, 150, 257]),
    ("sliding window", [44, 0, 100], [300, 200, 228]),
])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_matches_eager_for_each_mask(name, starts, ends, dtype):
    q, k, v = case(dtype=dtype, seed=len(name))
    mask = mask_from_ranges(3, 300, starts, ends)
    scaling = 128 ** -0.5
    out, w = H.custom_hf_decode_attention_forward(_Attn(4), q, k, v, mask, scaling, sliding_window=None)
    torch.cuda.synchronize()
    assert w is None and out.shape == (3, 16, 128) and out.dtype == dtype
    check(out, eager_f32(q, k, v, mask, scaling), what=name)
    # the bool form of the same mask
    out_b, _ = H.custom_hf_decode_attention_forward(_Attn(4), q, k, v, mask == 0, scaling)
    assert torch.equal(out_b, out)


def test_cache_position_path_and_sliding_window_fix():
    """With cache_position (the reference's contract) the length is
    cache_position[-1] + 1 and a window attends [len - window, len)."""
    q, k, v = case(S=512, seed=5)
    pos = torch.tensor([399], device=DEV)
    scaling = 128 ** -0.5
    qn, kn, vn = (t.float().cpu().numpy() for t in (q, k, v))
    for window in (None, 64, 1000):
        out, _ = H.custom_hf_decode_attention_forward(_Attn(4), q, k, v, None, scaling, cache_position=pos,
                                                      sliding_window=window)
        torch.cuda.synchronize()
        lo = 0 if window is None else max(0, 400 - window)
        want = O.decode_dense(qn[:, :, 0], kn, vn, [400] * 3, [lo] * 3)
        check(out, torch.from_numpy(want).to(DEV), what=f"window={window}")


def test_fp8_patch_matches_oracle_over_quantised_inputs():
    q, k, v = case(S=700, seed=9)
    mask = mask_from_ranges(3, 700, [0, 10, 0], [700, 700, 333])
    scaling = 128 ** -0.5
    out, _ = H.custom_hf_decode_attention_forward_fp8(_Attn(4), q, k, v, mask, scaling)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16
    q8, sq = O.quantize_to_fp8(q[:, :, 0].float().cpu().numpy())
    k8, sk = O.quantize_to_fp8(k.float().cpu().numpy())
    v8, sv = O.quantize_to_fp8(v.float().cpu().numpy())
    qd = O.dequantize_fp8(q8, sq).astype(np.float16).astype(np.float64)    # q in fp16, as :47-50
    want = O.decode_dense(qd, O.dequantize_fp8(k8, sk), O.dequantize_fp8(v8, sv), [700, 700, 333],
                          [0, 10, 0])
    check(out, torch.from_numpy(want).to(DEV), atol=1e-2, rtol=0.0, what="fp8")


def tiny_qwen3(dtype, sliding_window=None):
    cfg = transformers.Qwen3Config(vocab_size=256, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                                   num_attention_heads=8, num_key_value_heads=2, head_dim=128,
                                   max_position_embeddings=512, attn_implementation="eager",
                                   sliding_window=sliding_window, use_sliding_window=sliding_window is not None,
                                   max_window_layers=0)
    torch.manual_seed(0)
    return transformers.Qwen3ForCausalLM(cfg).to(DEV, dtype).eval()


def decode_logits(model, ids, am, tokens):
    """Prompt pass, then one step per column of ``tokens`` (teacher forced)."""
    out = model(ids, attention_mask=am, use_cache=True)
    past, logits = out.past_key_values, [out.logits[:, -1].float()]
    for t in range(tokens.shape[1]):
        am = torch.cat([am, torch.ones_like(am[:, :1])], 1)
        out = model(tokens[:, t:t + 1], attention_mask=am, past_key_values=past, use_cache=True)
        logits.append(out.logits[:, -1].float())
    return logits


def fp32_attention(module, q, k, v, mask, scaling, dropout=0.0, **kw):
    """transformers' eager attention computed in float32 (bf16 batched
    products over a transposed operand are kept off these GPUs)."""
    out, w = H.native_eager_attention_forward(module, q.float(), k.float(), v.float(),
                                              None if mask is None else mask.float(), scaling, dropout, **kw)
    return out.to(q.dtype), w


@pytest.mark.parametrize("fp8", [False, True])
def test_tiny_qwen3_decodes_through_the_patch(fp8):
    """Prompt + 12 decode steps (batch of 2, the first left-padded): every
    decode-step attention runs through the patch on the HIP kernels and agrees
    with eager float32 attention on the same inputs, and the logits stay close
    to those of the same model with float32 eager attention everywhere.  (The
    prompt passes use float32 eager attention in both runs.)"""
    model = tiny_qwen3(torch.bfloat16)
    calls = []
    patched = H.custom_hf_decode_attention_forward_fp8 if fp8 else H.custom_hf_decode_attention_forward

    def spy(module, q, k, v, mask, scaling, dropout=0.0, **kw):
        if q.shape[2] != 1:
            return fp32_attention(module, q, k, v, mask, scaling, dropout, **kw)
        out, w = patched(module, q, k, v, mask, scaling, dropout, **kw)
        calls.append(1)
        ref = eager_f32(q, k, v, mask, scaling)
        if fp8:  # quantisation error of Q, K, V at 3 mantissa bits
            assert (out.float() - ref).abs().max().item() < 0.1
        else:
            check(out, ref, what=f"layer {module.layer_idx}")
        return out, w

    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 256, (2, 9), generator=g).to(DEV)
    tokens = torch.randint(0, 256, (2, 12), generator=g).to(DEV)
    am = torch.ones(2, 9, dtype=torch.long, device=DEV)
    am[0, :3] = 0
    import transformers.models.qwen3.modeling_qwen3 as qm
    prev = qm.eager_attention_forward
    try:
        with torch.no_grad():
            qm.eager_attention_forward = fp32_attention
            want = decode_logits(model, ids, am, tokens)
            qm.eager_attention_forward = spy
            got = decode_logits(model, ids, am, tokens)
    finally:
        qm.eager_attention_forward = prev
    assert len(calls) == 12 * 2   # 12 decode steps, 2 layers
    assert torch.equal(got[0], want[0])   # the prompt pass is eager in both runs
    for t, (a, b) in enumerate(zip(got[1:], want[1:])):
        scale = b.abs().max().item()
        assert (a - b).abs().max().item() < (0.1 if fp8 else 0.03) * scale, t
