"""The allocation-free paged decode (fsk_decode_paged_noalloc) against the
workspace entry point (fsk_decode_paged), both called through the C ABI.

The two run the same kernels with the same split plan, so their outputs must
be bit-identical.  Two calls in a row, the second on a smaller batch with
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
