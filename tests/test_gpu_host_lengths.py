"""Decode with the sequence lengths in host memory against the same call with
device lengths.

With host lengths the binding calls fsk_decode_varlen_host /
fsk_decode_paged_host, which build the work plan on the host (the same
clamps, split rule and prefix sums as the device's plan) and pass it in the
kernel arguments; the kernels are otherwise the same code, so the outputs
must be identical bit for bit, including NaN rows of empty sequences.  Calls
the host path does not take (block scores, more than 64 sequences) copy the
lengths to the device and must give the device-length result too.  The
device-length path itself is held to the oracle in test_gpu_decode.py.
"""

import pytest
import torch

from fasterkernels_amd import workloads as W
from fskernels.hip import decode as dec

pytestmark = pytest.mark.gpu

DEV = "cuda"


def bits(t):
    return t.detach().contiguous().view(torch.uint8).cpu()


def both(wl, **kw):
    d = W.run(wl, **kw)
    h = W.run(wl, host_lengths=True, **kw)
    torch.cuda.synchronize()
    return d, h


def assert_same(d, h, what):
    if isinstance(d, tuple):
        for x, y in zip(d, h):
            assert_same(x, y, what)
        return
    assert d.shape == h.shape and d.dtype == h.dtype, what
    assert torch.equal(bits(d), bits(h)), f"{what}: host-length output differs from the device-length one"


CASES = [
    # name, overrides, sink mode, chunk_tokens
    ("C3", dict(B=3, lens=("list", [33, 700, 2049])), "exp", 0),
    ("C3", dict(B=3, lens=("list", [33, 700, 2049])), "exp", 32),
    ("C3", dict(B=3, lens=("list", [33, 700, 2049])), "exp", -256),
    ("C3", dict(B=4, lens=("list", [0, 5, 0, 40])), "exp", 0),
    ("C3", dict(B=5, lens=("list", [1, 15, 16, 17, 4096])), "exp", 512),
    ("C1", dict(B=8, lens=("list", [1, 2047, 0, 300, 129, 2048, 5, 1500])), "exp", 0),
    ("C1", dict(B=2, lens=("list", [0, 0])), "exp", 0),
    ("C2", dict(B=3, lens=("list", [9000, 17, 3000])), "linear", 0),
    ("C4", dict(B=3, lens=("list", [8192, 100, 5000])), "exp", 0),
    ("C5", dict(B=7, lens=("list", [4096, 8200, 5000, 33, 4097, 16, 700])), "exp", 0),
    ("C5", dict(B=7, lens=("list", [4096, 8200, 5000, 33, 4097, 16, 700])), "linear", 0),
    ("C5", dict(B=6, lens=("list", [0, 900, 900, 900, 0, 900])), "exp", 0),
    ("G1", dict(B=4, lens=("list", [3000, 1, 65, 2048])), "exp", 0),
    ("G2", dict(B=2, lens=("list", [5000, 300])), "exp", 0),
    ("M0b", dict(B=2, lens=("list", [4000, 12000])), "exp", 0),
]


@pytest.mark.parametrize("name,ov,mode,chunk", CASES)
def test_host_lengths_bit_identical(name, ov, mode, chunk):
    wl = W.make(name, overrides=ov, seed=21).to(DEV)
    d, h = both(wl, sink_mode=mode, chunk_tokens=chunk)
    assert_same(d, h, f"{name} {ov} {mode} chunk {chunk}")


@pytest.mark.parametrize("seed", range(60))
def test_host_lengths_random_configurations(seed):
    """The decode suite's random configurations (layout, dtypes, head
    grouping and dim, batch, lengths with zeros and page-boundary values,
    sinks, split size; test_gpu_decode.py::_random_case), both sink modes."""
    from tests.test_gpu_decode import _random_case
    name, ov, chunk = _random_case(5000 + seed)
    wl = W.make(name, overrides=ov, seed=seed).to(DEV)
    d, h = both(wl, chunk_tokens=chunk, sink_mode=("exp", "linear")[seed % 2])
    assert_same(d, h, f"seed {seed}: {name} {ov} chunk={chunk}")


@pytest.mark.parametrize("seed", range(6))
def test_host_lengths_random_large_batches(seed):
    """The suite's random large batches (9-300 sequences): up to 64 on the
    host path, the rest through the device copy."""
    from tests.test_gpu_decode import _random_large_case
    name, ov, chunk = _random_large_case(7000 + seed)
    wl = W.make(name, overrides=ov, seed=seed, gen_device=DEV, device=DEV)
    d, h = both(wl, chunk_tokens=chunk)
    assert_same(d, h, f"large seed {seed}: {name} B={ov['B']} chunk={chunk}")


@pytest.mark.parametrize("name", ["M0", "C1", "C2", "C4"])
def test_host_lengths_benchmark_sizes(name):
    """The benchmark configurations at their stated sizes (B = 4)."""
    wl = W.make(name, gen_device=DEV, device=DEV)
    d, h = both(wl)
    assert_same(d, h, name)


def test_host_lengths_64_sequences():
    """The largest host-planned batch: C5's 64 lognormal sequences."""
    wl = W.make("C5", gen_device=DEV, device=DEV)
    assert wl.B == 64
    for mode in ("exp", "linear"):
        d, h = both(wl, sink_mode=mode)
        assert_same(d, h, f"C5 {mode}")


def test_host_lengths_beyond_64_sequences_use_device_copy():
    """More than 64 sequences: the binding copies the host lengths to the
    device and takes the device-plan path, with the same result."""
    wl = W.make("C3", overrides=dict(B=80, lens=("uniform", 1, 600)), seed=5).to(DEV)
    d, h = both(wl)
    assert_same(d, h, "B=80")


@pytest.mark.parametrize("layout", ["paged", "varlen"])
def test_host_lengths_with_block_scores_use_device_copy(layout):
    wl = W.make("C3" if layout == "paged" else "C1", overrides=dict(B=3, lens=("list", [700, 5, 2000])),
                seed=9).to(DEV)
    d, h = both(wl, block_scores=True)
    assert_same(d, h, f"{layout} with block scores")


def test_host_lengths_clamped_like_device_ones():
    """Out-of-range lengths are clamped the same way on both paths: paged
    lengths to [0, max_blocks * page_size], varlen offsets to [0, T] and
    each end to at least its start."""
    wl = W.make("C3", overrides=dict(B=4, lens=("list", [100, 40, 300, 7])), seed=13).to(DEV)
    cap = wl.block_table.shape[1] * W.PAGE
    bad = torch.tensor([-5, cap + 1000, 300, 0], dtype=torch.int32)
    d = dec.paged_flash_decode(wl.q, wl.k, wl.v, wl.block_table, bad.to(DEV), W.PAGE)
    h = dec.paged_flash_decode(wl.q, wl.k, wl.v, wl.block_table, bad, W.PAGE)
    torch.cuda.synchronize()
    assert_same(d, h, "paged clamps")

    wv = W.make("C1", overrides=dict(B=4, lens=("list", [100, 40, 300, 7])), seed=13).to(DEV)
    T = wv.k.shape[0]
    cu = torch.tensor([0, 120, 60, T + 50, T + 80], dtype=torch.int32)
    d = dec.flash_decode_gqa_varlen(wv.q, wv.k, wv.v, cu.to(DEV))
    h = dec.flash_decode_gqa_varlen(wv.q, wv.k, wv.v, cu)
    torch.cuda.synchronize()
    assert_same(d, h, "varlen clamps")


def test_host_lengths_short_tensor_raises():
    wl = W.make("C3", overrides=dict(B=3, lens=("list", [10, 20, 30])), seed=1).to(DEV)
    with pytest.raises(ValueError):
        dec.paged_flash_decode(wl.q, wl.k, wl.v, wl.block_table, torch.tensor([10, 20], dtype=torch.int32),
                               W.PAGE)
    wv = W.make("C1", overrides=dict(B=3, lens=("list", [10, 20, 30])), seed=1).to(DEV)
    with pytest.raises(ValueError):
        dec.flash_decode_gqa_varlen(wv.q, wv.k, wv.v, torch.tensor([0, 10, 30], dtype=torch.int32))
