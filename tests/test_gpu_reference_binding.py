"""GPU parity of the ctypes-only binding a reference maintainer would add
(fasterkernels_amd/reference_binding.py, the drop-in for
fskernels/cuda/cuda_fd_gqa.py:14-15): the benchmark configurations C1 and C2
at full size and short sequences with sinks, against the float64 oracle's
linear sink fold (the CUDA kernel's, flash_decode_cuda.cu:151-153), and bit
for bit against the package's own entry point, whose default fold is the
same.  Bar: atol = rtol = 2e-3 (fp16 outputs)."""
import numpy as np
import pytest
import torch

from fasterkernels_amd import reference_binding as rb
from fasterkernels_amd import workloads as W
from fskernels.hip import flash_decode_gqa_varlen
from oracle import decode_oracle as O
from tests.test_gpu_decode import DEV, assert_close, f64

pytestmark = pytest.mark.gpu


def decode_both(wl):
    """The binding's output and the package entry point's (default fold)."""
    g = wl.to(DEV)
    print(f"reference binding: {wl.name} B={wl.B} tokens={wl.total_tokens} sinks={wl.s_aux is not None}", flush=True)
    out = rb.flash_decode_gqa_varlen(g.q, g.k, g.v, g.cu_seqlens, g.s_aux)
    pkg = flash_decode_gqa_varlen(g.q, g.k, g.v, g.cu_seqlens, g.s_aux)
    torch.cuda.synchronize()
    return out, pkg


def linear_oracle(wl):
    return O.decode_varlen(f64(wl.q), f64(wl.k), f64(wl.v), wl.cu_seqlens.numpy(),
                           None if wl.s_aux is None else f64(wl.s_aux), "linear")


@pytest.mark.parametrize("name", ["C1", "C2"])
def test_reference_binding_full_size(name):
    wl = W.make(name)
    out, pkg = decode_both(wl)
    assert out.dtype == torch.float16 and out.shape == (wl.B, wl.Hq, wl.D)
    assert_close(out, linear_oracle(wl), 2e-3, 2e-3, f"reference binding {name}", report=True)
    assert torch.equal(out, pkg)


def test_reference_binding_folds_sinks_linearly():
    """Short sequences, where the two folds differ by far more than the bar
    (sinks |N(0,1)| + 0.5, so the linear denominator stays above 1.5): the
    binding matches the linear oracle and not the exp one."""
    wl = W.make("C1", overrides=dict(B=5, lens=("list", [1, 7, 17, 64, 300]), sinks=True), seed=91)
    wl.s_aux = wl.s_aux.abs() + 0.5
    out, pkg = decode_both(wl)
    assert_close(out, linear_oracle(wl), 2e-3, 2e-3, "reference binding, short sequences, linear")
    exp_ref = O.decode_varlen(f64(wl.q), f64(wl.k), f64(wl.v), wl.cu_seqlens.numpy(), f64(wl.s_aux), "exp")
    assert np.abs(f64(out) - exp_ref).max() > 0.05
    assert torch.equal(out, pkg)


def test_reference_binding_bf16_and_int64_offsets():
    """bf16 q/k/v and int64 cu_seqlens (converted by the binding)."""
    wl = W.make("C1", overrides=dict(B=3, lens=("list", [5, 900, 33]), q="bf16", kv="bf16", out="bf16",
                                     sinks=True), seed=92)
    wl.s_aux = wl.s_aux.abs() + 0.5
    g = wl.to(DEV)
    out = rb.flash_decode_gqa_varlen(g.q, g.k, g.v, g.cu_seqlens.to(torch.int64), g.s_aux)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16
    assert_close(out, linear_oracle(wl), 2e-3, 2e-3, "reference binding bf16")


def test_reference_binding_errors():
    wl = W.make("C1", overrides=dict(B=2, lens=("list", [3, 4])), seed=93).to(DEV)
    with pytest.raises(ValueError):  # fp16 q with bf16 KV
        rb.flash_decode_gqa_varlen(wl.q, wl.k.bfloat16(), wl.v.bfloat16(), wl.cu_seqlens)
    q96 = torch.zeros(2, 32, 96, dtype=torch.float16, device=DEV)
    k96 = torch.zeros(7, 8, 96, dtype=torch.float16, device=DEV)
    with pytest.raises(NotImplementedError):  # head_dim 96: raised, not uninitialised memory
        rb.flash_decode_gqa_varlen(q96, k96, k96, wl.cu_seqlens)
    # extents the library cannot see are checked before the call
    sink = torch.zeros(wl.Hq, device=DEV)
    with pytest.raises(ValueError, match="sink must have one entry per query head"):
        rb.flash_decode_gqa_varlen(wl.q, wl.k, wl.v, wl.cu_seqlens, sink[:-1])
    with pytest.raises(ValueError, match="cu_seqlens_k must have B"):
        rb.flash_decode_gqa_varlen(wl.q, wl.k, wl.v, wl.cu_seqlens[:-1])
    with pytest.raises(ValueError, match="must be"):  # K rows narrower than q's head_dim
        rb.flash_decode_gqa_varlen(wl.q, wl.k[..., :64], wl.v[..., :64], wl.cu_seqlens)
