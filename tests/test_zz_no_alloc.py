"""The allocation-free paged decode (fsk_decode_paged_noalloc) against the
workspace entry point (fsk_decode_paged), both called through the C ABI.

The two run the same kernels with the same split plan, so their outputs must
be bit-identical, eagerly and when the allocation-free call is replayed from a
captured graph.  Two calls in a row, the second on a smaller batch with
different data, check that nothing of the first call's scratch contents leaks
into the second; a shape whose workspace exceeds the scratch is refused
before any launch.
"""

import pytest
import torch

from fasterkernels_amd import native as nat
from fasterkernels_amd import workloads as W

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
SCRATCH_BYTES = 32 << 20   # FSK_NOALLOC_SCRATCH_BYTES in include/fsk_decode.h


def paged_args(wl, out):
    """fsk_decode_paged's arguments up to sm_scale (the same order for the
    allocation-free entry point)."""
    q, k, v, bt = wl.q, wl.k, wl.v, wl.block_table
    P, Hkv, PS, D = k.shape
    return (q.data_ptr(), q.stride(0), q.stride(1),
            k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
            v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
            bt.data_ptr(), bt.stride(0), bt.shape[1], wl.seq_lens.data_ptr(), P, PS,
            nat.ptr(wl.s_aux), nat.FSK_SINK_EXP, nat.ptr(wl.k_scale), nat.ptr(wl.v_scale),
            out.data_ptr(), out.stride(0), out.stride(1),
            wl.B, wl.Hq, Hkv, D, nat.DTYPE_CODES[q.dtype], nat.DTYPE_CODES[k.dtype],
            nat.DTYPE_CODES[out.dtype], 1.0 / D ** 0.5)


def both(wl):
    """(workspace entry point's output, allocation-free entry point's output)."""
    lib = nat.load()
    stream = nat.stream_handle(DEV)
    ref = torch.full((wl.B, wl.Hq, wl.D), float("nan"), dtype=wl.out_dtype, device=DEV)
    got = torch.full_like(ref, float("nan"))
    P, Hkv, PS, D = wl.k.shape
    nbytes = nat.workspace_bytes(nat.FSK_LAYOUT_PAGED, wl.B, wl.Hq, Hkv, D, wl.block_table.shape[1], PS, 0)
    assert nbytes <= SCRATCH_BYTES
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    nat.check(lib.fsk_decode_paged(*paged_args(wl, ref), ws.data_ptr(), nbytes, 0, stream))
    nat.check(lib.fsk_decode_paged_noalloc(*paged_args(wl, got), 0, stream))
    torch.cuda.synchronize()
    return ref, got


def workspace_call(wl, out):
    """The workspace entry point (fsk_decode_paged) into ``out``, eagerly."""
    lib = nat.load()
    P, Hkv, PS, D = wl.k.shape
    nbytes = nat.workspace_bytes(nat.FSK_LAYOUT_PAGED, wl.B, wl.Hq, Hkv, D, wl.block_table.shape[1], PS, 0)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    nat.check(lib.fsk_decode_paged(*paged_args(wl, out), ws.data_ptr(), nbytes, 0, nat.stream_handle(DEV)))
    torch.cuda.synchronize()


def test_noalloc_captured_in_a_graph_with_its_first_call_inside():
    """The allocation-free call captured into a HIP graph (torch.cuda.graph,
    global capture mode), with the process's first call of that entry point
    inside the capture: the scratch address lookup and the launches are
    legal there.  Each replay, after eager work and a synchronisation that
    give q and the sinks new values in place, is bit-identical to the
    workspace entry point on the same inputs.  (This test comes first in the
    file so that the captured call is the process's first.)"""
    wl = W.make("C3", overrides=dict(B=5, lens=("list", [1, 40, 700, 3000, 9000]), sinks=True), seed=44).to(DEV)
    lib = nat.load()
    out = torch.full((wl.B, wl.Hq, wl.D), float("nan"), dtype=wl.out_dtype, device=DEV)
    ref = torch.full_like(out, float("nan"))
    workspace_call(wl, ref)  # (also loads the kernels before the capture)
    print("noalloc: capturing the first allocation-free call of the process", flush=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st = lib.fsk_decode_paged_noalloc(*paged_args(wl, out), 0, nat.stream_handle(DEV))
    assert st == nat.FSK_OK, lib.fsk_last_error()
    torch.cuda.synchronize()
    g = torch.Generator().manual_seed(45)
    for r in range(4):
        if r:
            wl.q.copy_(torch.randn(wl.q.shape, generator=g).to(wl.q.dtype).to(DEV))
            wl.s_aux.copy_(torch.randn(wl.s_aux.shape, generator=g).to(DEV))
        workspace_call(wl, ref)
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        print(f"noalloc: replay {r}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(ref).all()
        assert torch.equal(out, ref), f"replay {r}"
    del graph


def test_noalloc_matches_workspace_entry_on_consecutive_calls():
    big = W.make("M0", overrides=dict(B=6, lens=("list", [32768, 5, 20000, 1, 3000, 17]), sinks=True),
                 seed=41).to(DEV)
    print("noalloc call 1: paged f16 B=6 up to 32768 tokens, sinks", flush=True)
    ref1, got1 = both(big)
    assert torch.isfinite(ref1).all()
    assert torch.equal(got1, ref1)
    small = W.make("C5", overrides=dict(B=3, lens=("list", [700, 2, 64])), seed=42).to(DEV)
    print("noalloc call 2: paged e4m3 bf16 B=3, sinks", flush=True)
    ref2, got2 = both(small)
    assert torch.isfinite(ref2).all()
    assert torch.equal(got2, ref2)


def test_noalloc_refuses_shapes_beyond_the_scratch():
    """A batch whose workspace exceeds the scratch is refused with
    FSK_ERR_UNSUPPORTED and a message naming the limit; nothing is launched,
    so the output keeps its contents."""
    B, Hq, Hkv, D, max_blocks = 256, 32, 8, 128, 2048
    need = nat.workspace_bytes(nat.FSK_LAYOUT_PAGED, B, Hq, Hkv, D, max_blocks, 16, 0)
    assert need > SCRATCH_BYTES
    wl = W.make("M0", overrides=dict(B=B, lens=("fixed", 1), max_blocks=max_blocks), seed=43).to(DEV)
    out = torch.full((B, Hq, D), 7.0, dtype=torch.float16, device=DEV)
    lib = nat.load()
    st = lib.fsk_decode_paged_noalloc(*paged_args(wl, out), 0, nat.stream_handle(DEV))
    assert st == nat.FSK_ERR_UNSUPPORTED
    assert b"scratch" in lib.fsk_last_error()
    torch.cuda.synchronize()
    assert (out == 7.0).all()
    with pytest.raises(NotImplementedError, match="scratch"):
        nat.check(st)
