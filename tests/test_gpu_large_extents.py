"""GPU parity where the K/V bytes a call touches lie beyond 4 GiB of the
tensor's base address.

The kernels form K/V addresses from page ids, token rows and batch indices in
64-bit arithmetic, and their buffer descriptors are built per 16-row half
tile from those addresses, so a pool or cache can span the device's memory.
Each case puts the pages or rows that a decode or a KV write touches past
2^32 bytes (and past 2^31 elements) of its tensor, and leaves the rest of the
tensor unwritten: the oracle sees only the touched pages or rows, gathered
into a compact twin.  Bars as in test_gpu_decode.py (fp16/bf16 outputs
atol = rtol = 2e-3 plus half an ulp, e4m3 KV atol = 1e-2; KV writes
bit-exact).
"""
import numpy as np
import pytest
import torch

from fskernels.hip import decode as dec
from fskernels.hip import paged_kv_write
from oracle import decode_oracle as O

from tests.test_gpu_decode import assert_close, f64
from tests.test_gpu_kv_write import SENTINEL, compare, source_values

pytestmark = pytest.mark.gpu

DEV = "cuda"
GIB = 1 << 30


def _free():
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _pages_beyond(P_big, n_high, n_low, gen):
    """n_high distinct page ids whose byte offset is past 4 GiB and n_low
    from the first pages, shuffled together."""
    hi_lo = P_big - 4 * n_high
    high = hi_lo + torch.randperm(P_big - hi_lo, generator=gen)[:n_high]
    low = torch.randperm(64, generator=gen)[:n_low]
    ids = torch.cat([high, low])
    return ids[torch.randperm(ids.numel(), generator=gen)].to(torch.int64)


@pytest.mark.parametrize("kv", ["f16", "e4m3"])
def test_paged_pool_beyond_4gib(kv):
    gen = torch.Generator().manual_seed(41)
    B, Hq, Hkv, D, PS = 4, 32, 8, 128, 16
    lens = [5000, 1, 777, 16 * 17]
    fp8 = kv == "e4m3"
    elem = 1 if fp8 else 2
    page_bytes = Hkv * PS * D * elem
    P_big = (4 * GIB + 512 * 1024 * 1024) // page_bytes + 4096
    assert (P_big - 4096) * page_bytes > 4 * GIB
    need = [-(-n // PS) for n in lens]
    n_pages = sum(need)
    ids = _pages_beyond(P_big, n_pages - 12, 12, gen)
    assert int((ids * page_bytes > 4 * GIB).sum()) == n_pages - 12
    # compact twin: sequence b's logical pages are compact pages off[b] ...
    max_blocks = max(need) + 3
    bt_c = np.zeros((B, max_blocks), np.int32)
    off = 0
    for b, n in enumerate(need):
        bt_c[b, :n] = np.arange(off, off + n)
        off += n
    bt_big = torch.zeros((B, max_blocks), dtype=torch.int32)
    for b, n in enumerate(need):
        bt_big[b, :n] = ids[torch.from_numpy(bt_c[b, :n]).long()].to(torch.int32)
    q = torch.randn(B, Hq, D, generator=gen)
    if fp8:
        q = q.to(torch.bfloat16)
        kc = (torch.randn(n_pages, Hkv, PS, D, generator=gen) * 60).to(torch.float8_e4m3fn)
        vc = (torch.randn(n_pages, Hkv, PS, D, generator=gen) * 60).to(torch.float8_e4m3fn)
        ks, vs = 0.021, 0.0137
        ref = O.decode_paged(f64(q), kc.view(torch.uint8).numpy(), vc.view(torch.uint8).numpy(), bt_c,
                             lens, None, "exp", ks, vs)
        scales = dict(k_scale=torch.tensor(ks, device=DEV), v_scale=torch.tensor(vs, device=DEV))
        atol, rtol = 1e-2, 0.0
    else:
        q = q.to(torch.float16)
        kc = torch.randn(n_pages, Hkv, PS, D, generator=gen).to(torch.float16)
        vc = torch.randn(n_pages, Hkv, PS, D, generator=gen).to(torch.float16)
        ref = O.decode_paged(f64(q), kc.numpy(), vc.numpy(), bt_c, lens)
        scales = {}
        atol, rtol = 2e-3, 2e-3
    print(f"paged {kv}: pool {P_big} pages ({P_big * page_bytes / GIB:.2f} GiB each for K and V)", flush=True)
    k_big = torch.empty((P_big, Hkv, PS, D), dtype=kc.dtype, device=DEV)
    v_big = torch.empty((P_big, Hkv, PS, D), dtype=kc.dtype, device=DEV)
    idx = ids.to(DEV)
    k_big.view(torch.uint8).view(P_big, -1)[idx] = kc.view(torch.uint8).reshape(n_pages, -1).to(DEV)
    v_big.view(torch.uint8).view(P_big, -1)[idx] = vc.view(torch.uint8).reshape(n_pages, -1).to(DEV)
    for chunk in (0, 64):
        out = dec.paged_flash_decode(q.to(DEV), k_big, v_big, bt_big.to(DEV),
                                     torch.tensor(lens, dtype=torch.int32, device=DEV), PS,
                                     chunk_tokens=chunk, **scales)
        torch.cuda.synchronize()
        assert_close(out, ref, atol, rtol, f"paged {kv} pool beyond 4 GiB, chunk_tokens={chunk}")
    del k_big, v_big, out
    _free()


def test_varlen_rows_beyond_4gib():
    """Packed K/V rows 32 MiB apart (a strided view), so rows past the 128th
    start beyond 4 GiB of the base."""
    gen = torch.Generator().manual_seed(42)
    Hq, Hkv, D = 32, 8, 128
    cu = [0, 60, 61, 160]
    T = cu[-1]
    ST = 1 << 24   # token stride in elements: 32 MiB of f16
    q = torch.randn(len(cu) - 1, Hq, D, generator=gen).to(torch.float16)
    kc = torch.randn(T, Hkv, D, generator=gen).to(torch.float16)
    vc = torch.randn(T, Hkv, D, generator=gen).to(torch.float16)
    s_aux = torch.randn(Hq, generator=gen)
    ref = O.decode_varlen(f64(q), f64(kc), f64(vc), np.array(cu), f64(s_aux), "exp")
    n_el = (T - 1) * ST + 2 * Hkv * D
    print(f"varlen: {n_el * 2 / GIB:.2f} GiB buffer, last row at {(T - 1) * ST * 2 / GIB:.2f} GiB", flush=True)
    buf = torch.empty(n_el, dtype=torch.float16, device=DEV)
    k = buf.as_strided((T, Hkv, D), (ST, D, 1))
    v = buf.as_strided((T, Hkv, D), (ST, D, 1), Hkv * D)
    k.copy_(kc.to(DEV))
    v.copy_(vc.to(DEV))
    for chunk in (0, 32):
        out = dec.flash_decode_gqa_varlen(q.to(DEV), k, v, torch.tensor(cu, dtype=torch.int32, device=DEV),
                                          s_aux.to(DEV), sink_mode="exp", chunk_tokens=chunk)
        torch.cuda.synchronize()
        assert_close(out, ref, 2e-3, 2e-3, f"varlen rows beyond 4 GiB, chunk_tokens={chunk}")
    del buf, k, v, out
    _free()


def test_dense_batches_beyond_4gib():
    """HF-layout caches whose batch stride puts batch 2 past 4 GiB."""
    gen = torch.Generator().manual_seed(43)
    B, Hq, Hkv, S, D = 3, 32, 8, 300, 128
    lens, starts = [300, 17, 250], [0, 3, 100]
    BS = (1 << 30) + (1 << 26)   # batch stride in elements: batch 2 starts 4.25 GiB in
    q = torch.randn(B, Hq, D, generator=gen).to(torch.bfloat16)
    kc = torch.randn(B, Hkv, S, D, generator=gen).to(torch.bfloat16)
    vc = torch.randn(B, Hkv, S, D, generator=gen).to(torch.bfloat16)
    ref = O.decode_dense(f64(q), f64(kc), f64(vc), np.array(lens), np.array(starts))
    n_el = (B - 1) * BS + 2 * Hkv * S * D
    print(f"dense: {n_el * 2 / GIB:.2f} GiB buffer, batch 2 at {2 * BS * 2 / GIB:.2f} GiB", flush=True)
    buf = torch.empty(n_el, dtype=torch.bfloat16, device=DEV)
    k = buf.as_strided((B, Hkv, S, D), (BS, S * D, D, 1))
    v = buf.as_strided((B, Hkv, S, D), (BS, S * D, D, 1), Hkv * S * D)
    k.copy_(kc.to(DEV))
    v.copy_(vc.to(DEV))
    for splits in (1, 8):
        out = dec.flash_decode_gqa_hf_dense_optimized(q.to(DEV), k, v,
                                                      torch.tensor(lens, dtype=torch.int32, device=DEV),
                                                      torch.tensor(starts, dtype=torch.int32, device=DEV),
                                                      splits)
        torch.cuda.synchronize()
        assert_close(out, ref, 2e-3, 2e-3, f"dense batches beyond 4 GiB, num_splits={splits}")
    del buf, k, v, out
    _free()


@pytest.mark.parametrize("src,pool,scaled", [("f16", "f16", False), ("bf16", "e4m3", True)])
def test_kv_write_pages_beyond_4gib(src, pool, scaled):
    gen = torch.Generator().manual_seed(44)
    Hkv, PS, D, n = 8, 16, 128, 300
    dt = {"f16": torch.float16, "e4m3": torch.float8_e4m3fn}[pool]
    elem = 1 if pool == "e4m3" else 2
    page_bytes = Hkv * PS * D * elem
    P_big = (4 * GIB + 512 * 1024 * 1024) // page_bytes + 4096
    ids = _pages_beyond(P_big, 40, 4, gen)   # the pages the writes land on
    n_pages = ids.numel()
    kx = source_values(n, Hkv, D, src, gen)
    vx = source_values(n, Hkv, D, src, gen, spread=3.0)
    compact = torch.randperm(n_pages * PS, generator=gen)[:n].to(torch.int64)
    compact[7] = -1   # a skipped token
    page_c, row = compact // PS, compact % PS
    slots = torch.where(compact < 0, compact, ids[page_c.clamp(min=0)] * PS + row)
    print(f"kv write {src}->{pool}: pool {P_big} pages ({P_big * page_bytes / GIB:.2f} GiB), "
          f"largest slot {int(slots.max())}", flush=True)
    sent = SENTINEL[pool]
    store = torch.uint8 if pool == "e4m3" else torch.int16
    k_big = torch.empty((P_big, Hkv, PS, D), dtype=dt, device=DEV)
    v_big = torch.empty((P_big, Hkv, PS, D), dtype=dt, device=DEV)
    idx = ids.to(DEV)
    for t in (k_big, v_big):
        t.view(store)[idx] = torch.full((n_pages, Hkv, PS, D), sent, dtype=store, device=DEV)
    kso, vso = (np.float32(0.05), np.float32(0.004)) if scaled else (None, None)
    ks = None if kso is None else torch.tensor(kso, device=DEV)
    vs = None if vso is None else torch.tensor(vso, device=DEV)
    paged_kv_write(kx.to(DEV), vx.to(DEV), k_big, v_big, slots.to(DEV), k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    for x, big, sc, name in ((kx, k_big, kso, "K"), (vx, v_big, vso, "V")):
        if pool == "e4m3":
            o = np.full((n_pages, Hkv, PS, D), sent, dtype=np.uint8)
            O.paged_write(o, compact.numpy(), x.float().numpy(), pool, sc)
        else:
            o = np.full((n_pages, Hkv, PS, D), sent, dtype=np.uint16).view(np.float16)
            O.paged_store_rows(o.view(np.uint16), compact.numpy(), x.view(torch.int16).numpy().view(np.uint16))
        compare(big[idx], o, pool, src, f"{name} {src}->{pool} pages beyond 4 GiB")
    del k_big, v_big
    _free()
