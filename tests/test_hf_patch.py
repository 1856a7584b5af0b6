"""HF attention patch (fskernels.hip.hf) on the CPU: prefill calls go to
transformers' eager attention unchanged, decode steps refuse host tensors, and
the patch helpers install and restore the module function."""
import pytest
import torch

transformers = pytest.importorskip("transformers")

import transformers.models.qwen3.modeling_qwen3 as qwen3_mod  # noqa: E402

from fskernels.hip import hf as H  # noqa: E402


class _Attn(torch.nn.Module):
    num_key_value_groups = 2
    num_key_value_heads = 2


def test_prefill_goes_to_native_eager():
    g = torch.Generator().manual_seed(0)
    q = torch.randn(2, 4, 5, 64, generator=g)
    k = torch.randn(2, 2, 5, 64, generator=g)
    v = torch.randn(2, 2, 5, 64, generator=g)
    mask = torch.triu(torch.full((5, 5), torch.finfo(torch.float32).min), 1)[None, None].expand(2, 1, 5, 5)
    want = H.native_eager_attention_forward(_Attn(), q, k, v, mask, 0.125)
    got = H.custom_hf_decode_attention_forward(_Attn(), q, k, v, mask, 0.125, sliding_window=None)
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
    got8 = H.custom_hf_decode_attention_forward_fp8(_Attn(), q, k, v, mask, 0.125)
    assert torch.equal(got8[0], want[0])


def test_decode_step_refuses_host_tensors():
    q = torch.zeros(1, 4, 1, 64)
    k = torch.zeros(1, 2, 3, 64)
    with pytest.raises(RuntimeError, match="GPU"):
        H.custom_hf_decode_attention_forward(_Attn(), q, k, k, None, 0.125)


def test_patch_helpers_install_and_restore():
    before = qwen3_mod.eager_attention_forward
    with H.patched_hf_attention():
        assert qwen3_mod.eager_attention_forward is H.custom_hf_decode_attention_forward
    assert qwen3_mod.eager_attention_forward is before
    with H.patched_hf_attention(fp8=True):
        assert qwen3_mod.eager_attention_forward is H.custom_hf_decode_attention_forward_fp8
    prev = H.patch_hf_attention()
    try:
        assert prev is before
    finally:
        qwen3_mod.eager_attention_forward = prev
    assert H._native_eager is not H.custom_hf_decode_attention_forward


def test_tiny_qwen3_prefill_runs_through_the_patch_on_cpu():
    """A whole model forward with the patch installed: the prompt pass uses
    the native path (identical logits); the next single-token step would need
    the GPU and refuses host tensors."""
    cfg = transformers.Qwen3Config(vocab_size=64, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                                   max_position_embeddings=64, attn_implementation="eager")
    torch.manual_seed(0)
    m = transformers.Qwen3ForCausalLM(cfg).eval()
    ids = torch.randint(0, 64, (1, 6))
    with torch.no_grad():
        want = m(ids).logits
        with H.patched_hf_attention():
            out = m(ids, use_cache=True)
            assert torch.equal(out.logits, want)
            with pytest.raises(RuntimeError, match="GPU"):
                m(ids[:, :1], past_key_values=out.past_key_values, use_cache=True)
