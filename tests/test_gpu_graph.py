"""HIP-graph capture of decode steps (fskernels.engine).

Every replay is checked against the eager call on the same inputs (the
kernels are deterministic for equal inputs, so bit-exact), with eager work
and synchronisations between replays, inputs changed in place, and lengths
and block tables that change between replays.  The captured serving step
(KV store + paged decode) is checked against a twin cache driven eagerly,
and the whole-model runner against float32-attention decoding.
"""
import numpy as np
import pytest
import torch

from fskernels.hip import flash_decode_gqa_varlen
from fskernels.paged_attn import PagedKVCache, paged_flash_decode
from fskernels.engine.hip_graph import DecodeGraph, PagedDecodeStep
from fskernels.hip import decode as dec
from oracle import decode_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_paged_decode_graph_replays_with_changing_inputs():
    g = torch.Generator().manual_seed(0)
    B, Hq, Hkv, D, P, MB = 4, 32, 8, 128, 600, 96
    kp = torch.randn(P, Hkv, 16, D, generator=g).half().to(DEV)
    vp = torch.randn(P, Hkv, 16, D, generator=g).half().to(DEV)
    q = torch.zeros(B, Hq, D, dtype=torch.float16, device=DEV)
    bt = torch.zeros(B, MB, dtype=torch.int32, device=DEV)
    lens = torch.zeros(B, dtype=torch.int32, device=DEV)
    sinks = torch.randn(Hq, generator=g).to(DEV)
    graph = DecodeGraph(paged_flash_decode, q, kp, vp, bt, lens, 16, s_aux=sinks)
    for rep, L in enumerate([[1, 17, 1536, 0], [1536, 1536, 1536, 1536], [5, 900, 33, 1200]]):
        q.copy_(torch.randn(B, Hq, D, generator=g).half())
        bt.copy_(torch.randperm(P, generator=g)[:B * MB].view(B, MB).int())
        lens.copy_(torch.tensor(L, dtype=torch.int32))
        out = graph.replay()
        torch.cuda.synchronize()
        eager = paged_flash_decode(q, kp, vp, bt, lens, 16, s_aux=sinks)
        torch.cuda.synchronize()
        assert torch.equal(torch.nan_to_num(out, 7.0), torch.nan_to_num(eager, 7.0)), rep


def test_varlen_and_dense_graphs():
    g = torch.Generator().manual_seed(1)
    B, Hq, Hkv, D, T, S = 3, 16, 4, 64, 5000, 2048
    k = torch.randn(T, Hkv, D, generator=g).bfloat16().to(DEV)
    v = torch.randn(T, Hkv, D, generator=g).bfloat16().to(DEV)
    q = torch.zeros(B, Hq, D, dtype=torch.bfloat16, device=DEV)
    cu = torch.zeros(B + 1, dtype=torch.int32, device=DEV)
    gv = DecodeGraph(flash_decode_gqa_varlen, q, k, v, cu)
    kd = torch.randn(B, Hkv, S, D, generator=g).bfloat16().to(DEV)
    vd = torch.randn(B, Hkv, S, D, generator=g).bfloat16().to(DEV)
    lens = torch.zeros(B, dtype=torch.int32, device=DEV)
    gd = DecodeGraph(dec.flash_decode_gqa_hf_dense_optimized, q, kd, vd, lens)
    for rep, (c, L) in enumerate([([0, 10, 3000, 5000], [1, 2048, 700]), ([0, 0, 0, 4999], [2048, 2048, 1])]):
        q.copy_(torch.randn(B, Hq, D, generator=g).bfloat16())
        cu.copy_(torch.tensor(c, dtype=torch.int32))
        lens.copy_(torch.tensor(L, dtype=torch.int32))
        a, b = gv.replay(), gd.replay()
        torch.cuda.synchronize()
        ea = flash_decode_gqa_varlen(q, k, v, cu)
        eb = dec.flash_decode_gqa_hf_dense_optimized(q, kd, vd, lens)
        torch.cuda.synchronize()
        assert torch.equal(torch.nan_to_num(a, 7.0), torch.nan_to_num(ea, 7.0)), rep
        assert torch.equal(eb, b), rep


@pytest.mark.parametrize("pool", ["f16", "e4m3"])
def test_paged_decode_step_matches_eager_twin(pool):
    """30 captured steps over 3 sequences (page boundaries crossed, fresh
    pages taken inside the graph) give the outputs, pools and block tables of
    a twin cache driven with append_kv_batch + paged_flash_decode."""
    g = torch.Generator().manual_seed(2)
    Hq, Hkv, D = 32, 8, 128
    dt = torch.float16 if pool == "f16" else torch.float8_e4m3fn
    scales = dict(k_scale=0.02, v_scale=0.02) if pool == "e4m3" else {}
    caches = [PagedKVCache(2, 64, 4, 32, Hkv, D, dt, DEV, **scales) for _ in range(2)]
    ids = []
    for c in caches:
        ids = [c.allocate_sequence() for _ in range(3)]
        ids = [ids[2], ids[0], ids[1]]           # any slot order
    prompt = [torch.randn(L, Hkv, D, generator=g).half() for L in (15, 40, 1)]
    for c in caches:
        for sid, rows in zip(ids, prompt):
            slots = c.reserve_slots([sid], rows.shape[0])
            c.write_kv(1, rows.to(DEV), rows.to(DEV), slots)
    qdt = torch.float16
    step = PagedDecodeStep(caches[0], 1, ids, Hq, q_dtype=qdt, src_dtype=torch.float16)
    twin = caches[1]
    for t in range(30):
        q = torch.randn(3, Hq, D, generator=g).half().to(DEV)
        kn = torch.randn(3, Hkv, D, generator=g).half().to(DEV)
        vn = torch.randn(3, Hkv, D, generator=g).half().to(DEV)
        out = step.step(q, kn, vn)
        torch.cuda.synchronize()
        twin.append_kv_batch(ids, 1, kn, vn)
        want = paged_flash_decode(q, twin.k_pool[1], twin.v_pool[1], twin.get_block_table_tensor(ids),
                                  twin.get_seq_lens_tensor(ids), 16, k_scale=twin.k_scale, v_scale=twin.v_scale)
        torch.cuda.synchronize()
        assert torch.equal(out, want), t
        assert torch.equal(caches[0].block_table, twin.block_table), t
    assert caches[0]._seq_lens == twin._seq_lens
    assert torch.equal(caches[0].k_pool.view(torch.uint8), twin.k_pool.view(torch.uint8))
    assert torch.equal(caches[0].v_pool.view(torch.uint8), twin.v_pool.view(torch.uint8))
    # and the last step against the oracle
    bt = twin.get_block_table_tensor(ids).cpu().numpy()
    lens = [twin._seq_lens[s] for s in ids]
    if pool == "f16":
        ref = O.decode_paged(q.double().cpu().numpy(), twin.k_pool[1].float().cpu().numpy(),
                             twin.v_pool[1].float().cpu().numpy(), bt, lens)
        tol = 2e-3 + 2e-3 * np.abs(ref) + np.abs(ref) * 2.0 ** -11
    else:
        ref = O.decode_paged(q.double().cpu().numpy(), twin.k_pool[1].view(torch.uint8).cpu().numpy(),
                             twin.v_pool[1].view(torch.uint8).cpu().numpy(), bt, lens,
                             k_scale=np.float32(0.02), v_scale=np.float32(0.02))
        tol = 1e-2 + np.abs(ref) * 2.0 ** -11
    assert (np.abs(out.double().cpu().numpy() - ref) <= tol).all()


def test_hip_graph_runner_matches_fp32_attention_decoding():
    transformers = pytest.importorskip("transformers")
    import transformers.models.qwen3.modeling_qwen3 as qm

    from fskernels.engine import HIPGraphRunner
    from fskernels.hip import hf as H

    cfg = transformers.Qwen3Config(vocab_size=256, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                                   num_attention_heads=8, num_key_value_heads=2, head_dim=128,
                                   max_position_embeddings=512, attn_implementation="eager")
    torch.manual_seed(0)
    model = transformers.Qwen3ForCausalLM(cfg).to(DEV, torch.bfloat16).eval()

    def fp32_attention(module, q, k, v, mask, scaling, dropout=0.0, **kw):
        out, w = H.native_eager_attention_forward(module, q.float(), k.float(), v.float(),
                                                  None if mask is None else mask.float(), scaling, dropout, **kw)
        return out.to(q.dtype), w

    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, 256, (2, 11), generator=g).to(DEV)
    tokens = torch.randint(0, 256, (2, 10), generator=g).to(DEV)
    prev = qm.eager_attention_forward
    try:
        qm.eager_attention_forward = fp32_attention
        with torch.no_grad():
            out = model(ids, use_cache=True)
            past, want = out.past_key_values, []
            for t in range(tokens.shape[1]):
                o = model(tokens[:, t:t + 1], past_key_values=past, use_cache=True)
                want.append(o.logits[:, -1].float())
            runner = HIPGraphRunner(model, batch_size=2, max_seq_len=64)
            first = runner.prefill(ids)
        assert torch.equal(first, out.logits[:, -1])
        runner.build(warmup_steps=3)
        assert qm.eager_attention_forward is fp32_attention       # the capture's patch was removed
        for t in range(tokens.shape[1]):
            got = runner.step(tokens[:, t]).float()
            torch.cuda.synchronize()
            scale = want[t].abs().max().item()
            assert (got - want[t]).abs().max().item() < 0.03 * scale, t
    finally:
        qm.eager_attention_forward = prev
