"""Seeded synthetic decode workloads (the benchmark configurations).

Draw order with one torch.Generator: lengths -> block-table permutation -> Q ->
K -> V -> s_aux.  Paged pools hold the pages the sequences need plus 10 %
free pages; a seeded permutation of the pool assigns physical pages, so pages
of one sequence are scattered.  Every slot of the pool (including free pages
and the tail of a partial last page) holds random data, so a kernel that
reads past a sequence end produces wrong results.

fp8 pools are generated as N(0,1) fp32 and quantised per tensor with
scale = max|x| / 448 (fskernels/triton/triton_gqa_decode_hf_fp8.py:13-16).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

PAGE = 16

# name -> configuration (shapes from the benchmark definition)
CONFIGS = {
    # headline: paged fp16, B=4, 32K context
    "M0": dict(layout="paged", q="f16", kv="f16", out="f16", B=4, Hq=32, Hkv=8, D=128,
               lens=("fixed", 32768), sinks=False, seed=100),
    # varlen fp16, lengths U[1, 2048], no sinks
    "C1": dict(layout="varlen", q="f16", kv="f16", out="f16", B=4, Hq=32, Hkv=8, D=128,
               lens=("uniform", 1, 2048), sinks=False, seed=101),
    # varlen fp16, 32K, N(0,1) sinks
    "C2": dict(layout="varlen", q="f16", kv="f16", out="f16", B=4, Hq=32, Hkv=8, D=128,
               lens=("fixed", 32768), sinks=True, seed=102),
    # paged fp16, B=32, lengths U[1024, 16384]
    "C3": dict(layout="paged", q="f16", kv="f16", out="f16", B=32, Hq=32, Hkv=8, D=128,
               lens=("uniform", 1024, 16384), sinks=False, seed=103),
    # paged e4m3 KV, bf16 Q and output, 8K
    "C4": dict(layout="paged", q="bf16", kv="e4m3", out="bf16", B=4, Hq=32, Hkv=8, D=128,
               lens=("fixed", 8192), sinks=False, seed=104),
    # paged e4m3 KV + sinks, B=64, lognormal lengths
    "C5": dict(layout="paged", q="bf16", kv="e4m3", out="bf16", B=64, Hq=32, Hkv=8, D=128,
               lens=("lognormal", math.log(4096.0), 1.0, 16, 32768), sinks=True, seed=105),
    # M0 in bf16 (the dtype PagedKVCache.from_config gives its pools,
    # fskernels/paged_attn/paged_kv_cache.py:80)
    "M0b": dict(layout="paged", q="bf16", kv="bf16", out="bf16", B=4, Hq=32, Hkv=8, D=128,
                lens=("fixed", 32768), sinks=False, seed=100),
    # head_dim 64 with sinks (GPT-OSS-style attention shapes): varlen fp16,
    # B=4, Hq=64, Hkv=8, 65536 tokens each (the same 537 MB of K/V as M0)
    "G1": dict(layout="varlen", q="f16", kv="f16", out="f16", B=4, Hq=64, Hkv=8, D=64,
               lens=("fixed", 65536), sinks=True, seed=106),
    # head_dim 256 (Gemma-style attention shapes): paged fp16, B=4, Hq=32,
    # Hkv=8, 16384 tokens each (the same 537 MB of K/V as M0)
    "G2": dict(layout="paged", q="f16", kv="f16", out="f16", B=4, Hq=32, Hkv=8, D=256,
               lens=("fixed", 16384), sinks=False, seed=107),
}

DTYPES = {"f16": torch.float16, "bf16": torch.bfloat16, "e4m3": torch.float8_e4m3fn,
          "f32": torch.float32}


@dataclass
class Workload:
    name: str
    layout: str
    B: int
    Hq: int
    Hkv: int
    D: int
    lens: list
    q: torch.Tensor
    k: torch.Tensor              # varlen [T,Hkv,D] / paged pool [P,Hkv,16,D]
    v: torch.Tensor
    cu_seqlens: torch.Tensor | None = None
    block_table: torch.Tensor | None = None
    seq_lens: torch.Tensor | None = None
    s_aux: torch.Tensor | None = None
    k_scale: torch.Tensor | None = None
    v_scale: torch.Tensor | None = None
    out_dtype: torch.dtype = torch.float16
    meta: dict = field(default_factory=dict)

    @property
    def total_tokens(self) -> int:
        return int(sum(self.lens))

    def host_lengths(self) -> torch.Tensor:
        """The lengths in host memory, as the host-plan entry points take them
        (paged: seq_lens [B]; varlen: cu_seqlens [B+1]); made once."""
        if "_host_lengths" not in self.meta:
            lens = torch.tensor(self.lens, dtype=torch.int64)
            if self.layout == "paged":
                t = lens.to(torch.int32)
            else:
                t = torch.zeros(self.B + 1, dtype=torch.int32)
                t[1:] = torch.cumsum(lens, 0).to(torch.int32)
            self.meta["_host_lengths"] = t
        return self.meta["_host_lengths"]

    def to(self, device) -> "Workload":
        def mv(t):
            return None if t is None else t.to(device)
        return Workload(self.name, self.layout, self.B, self.Hq, self.Hkv, self.D, list(self.lens),
                        mv(self.q), mv(self.k), mv(self.v), mv(self.cu_seqlens),
                        mv(self.block_table), mv(self.seq_lens), mv(self.s_aux), mv(self.k_scale),
                        mv(self.v_scale), self.out_dtype, dict(self.meta))

    def algorithmic_bytes(self) -> int:
        """Bytes a decode step must move: valid-token K+V, Q, output, the block
        table entries used, lengths, sinks and scales."""
        kv_elem = self.k.element_size()
        n = self.total_tokens * self.Hkv * self.D * 2 * kv_elem
        n += self.B * self.Hq * self.D * (self.q.element_size() + DTYPES_SIZE[self.out_dtype])
        if self.layout == "paged":
            n += 4 * sum((L + PAGE - 1) // PAGE for L in self.lens) + 4 * self.B
        else:
            n += 4 * (self.B + 1)
        if self.s_aux is not None:
            n += 4 * self.Hq
        if self.k_scale is not None:
            n += 8
        return n

    def flops(self) -> int:
        return 4 * self.D * self.Hq * self.total_tokens


DTYPES_SIZE = {torch.float16: 2, torch.bfloat16: 2, torch.float32: 4}


def _lengths(spec, B, g):
    kind = spec[0]
    if kind == "fixed":
        return [int(spec[1])] * B
    if kind == "uniform":
        return torch.randint(int(spec[1]), int(spec[2]) + 1, (B,), generator=g).tolist()
    if kind == "lognormal":
        mu, sigma, lo, hi = spec[1:]
        z = torch.randn(B, generator=g, dtype=torch.float64)
        return [int(min(max(round(math.exp(mu + sigma * float(x))), lo), hi)) for x in z]
    if kind == "list":
        return [int(x) for x in spec[1]]
    raise ValueError(kind)


def _randn(shape, g, device):
    if device is None or torch.device(device).type == "cpu":
        return torch.randn(*shape, generator=g)
    return torch.randn(*shape, generator=g, device=device)


def _quantize(x):
    amax = x.abs().max().clamp(min=1e-12)
    scale = (amax / 448.0).to(torch.float32)
    return (x / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn), scale


def make(name: str = "M0", *, device=None, seed: int | None = None, overrides: dict | None = None,
         gen_device=None, data_seed: int | None = None) -> Workload:
    """Builds a workload.  ``overrides`` replaces config keys (e.g. smaller
    ``B`` or ``lens`` for tests).  Random draws use a CPU generator unless
    ``gen_device`` names a GPU (faster for large benchmark inputs, different
    values).  ``data_seed`` redraws only Q/K/V/sinks: workloads made with the
    same ``seed`` share lengths and page tables (rotating benchmark inputs)."""
    cfg = dict(CONFIGS[name])
    if overrides:
        cfg.update(overrides)
    seed = cfg["seed"] if seed is None else seed
    gdev = torch.device(gen_device) if gen_device is not None else torch.device("cpu")
    g = torch.Generator().manual_seed(seed)          # lengths, permutation (and data on CPU)
    if data_seed is not None:
        gd = torch.Generator(device=gdev).manual_seed(data_seed)
    else:
        gd = g if gdev.type == "cpu" else torch.Generator(device=gdev).manual_seed(seed)
    B, Hq, Hkv, D = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["D"]
    lens = _lengths(cfg["lens"], B, g)
    layout = cfg["layout"]
    qdt, kvdt, odt = DTYPES[cfg["q"]], DTYPES[cfg["kv"]], DTYPES[cfg["out"]]
    rd = None if gdev.type == "cpu" else gdev
    wl_meta = {"config": name, "seed": seed}
    cu = bt = sl = None
    if layout == "paged":
        npages = [(L + PAGE - 1) // PAGE for L in lens]
        total = sum(npages)
        P = max(total + int(math.ceil(0.1 * total)), 1)
        perm = torch.randperm(P, generator=g).tolist()
        max_blocks = int(cfg.get("max_blocks") or max(max(npages), 1))
        bt = torch.full((B, max_blocks), -1, dtype=torch.int32)
        off = 0
        for b, n in enumerate(npages):
            bt[b, :n] = torch.tensor(perm[off:off + n], dtype=torch.int32)
            off += n
        sl = torch.tensor(lens, dtype=torch.int32)
        kv_shape = (P, Hkv, PAGE, D)
        wl_meta.update(num_pages=P, max_blocks=max_blocks)
    else:
        T = sum(lens)
        cu = torch.zeros(B + 1, dtype=torch.int32)
        cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int64), 0).to(torch.int32)
        kv_shape = (T, Hkv, D)
    q = _randn((B, Hq, D), gd, rd).to(qdt)
    kf = _randn(kv_shape, gd, rd)
    vf = _randn(kv_shape, gd, rd)
    ks = vs = None
    if kvdt == torch.float8_e4m3fn:
        k, ks = _quantize(kf)
        v, vs = _quantize(vf)
    else:
        k, v = kf.to(kvdt), vf.to(kvdt)
    del kf, vf
    s_aux = _randn((Hq,), gd, rd).to(torch.float32) if cfg["sinks"] else None
    if s_aux is not None and cfg.get("sink_scale", 1.0) != 1.0:
        s_aux = s_aux * float(cfg["sink_scale"])
    wl = Workload(name, layout, B, Hq, Hkv, D, lens, q, k, v, cu, bt, sl, s_aux, ks, vs, odt, wl_meta)
    return wl.to(device) if device is not None else wl


def reference_sweep_workload(B: int, S: int, *, device=None, gen_device=None, data_seed: int | None = None) -> Workload:
    """The reference benchmark's decode input at batch B and maximum length S
    (benchmarks/benchmark.py:20-33): varlen fp16, Hq=32, Hkv=8, D=128,
    lengths uniform in [max(64, S // 4), S] (seed 42, drawn here from a CPU
    generator), Q/K/V N(0,1), sinks 0.1 N(0,1), which the reference kernels
    fold linearly."""
    return make("C1", device=device, gen_device=gen_device, data_seed=data_seed, seed=42,
                overrides=dict(B=B, lens=("uniform", max(64, S // 4), S), sinks=True, sink_scale=0.1))


def run(wl: Workload, *, sink_mode: str = "exp", chunk_tokens: int = 0, block_scores: bool = False,
        host_lengths: bool = False):
    """One decode step of ``wl`` through the HIP entry points (with
    ``block_scores``: also the pooled block scores, returned as (out, S); with
    ``host_lengths``: the lengths passed in host memory, so the work plan is
    built on the host)."""
    from fskernels.hip import decode as dec
    if wl.layout == "paged":
        lens = wl.host_lengths() if host_lengths else wl.seq_lens
        return dec.paged_flash_decode(wl.q, wl.k, wl.v, wl.block_table, lens, PAGE,
                                      s_aux=wl.s_aux, k_scale=wl.k_scale, v_scale=wl.v_scale,
                                      out_dtype=wl.out_dtype, sink_mode=sink_mode,
                                      chunk_tokens=chunk_tokens, return_block_scores=block_scores)
    cu = wl.host_lengths() if host_lengths else wl.cu_seqlens
    return dec.flash_decode_gqa_varlen(wl.q, wl.k, wl.v, cu, wl.s_aux,
                                       sink_mode=sink_mode, k_scale=wl.k_scale, v_scale=wl.v_scale,
                                       out_dtype=wl.out_dtype, chunk_tokens=chunk_tokens,
                                       return_block_scores=block_scores)


# ---------------------------------------------------------------------------
# KV write workloads: new rows stored into paged pools at scattered slots
# ---------------------------------------------------------------------------
WRITE_CONFIGS = {
    # the whole M0 cache (4 x 32768 tokens) stored in one launch, f16 -> f16 pools
    "W0": dict(src="f16", pool="f16", B=4, L=32768, Hkv=8, D=128, scaled=False, seed=110),
    # the same rows from bf16 projections quantised into e4m3 pools (C4/C5 pools)
    "W1": dict(src="bf16", pool="e4m3", B=4, L=32768, Hkv=8, D=128, scaled=True, seed=111),
    # one decode step's append: one token for each of C5's 64 sequences
    "W2": dict(src="bf16", pool="e4m3", B=64, L=1, Hkv=8, D=128, scaled=True, seed=112),
    # W0 and W1 on the pages a fresh PagedKVCache hands out: its LIFO free
    # list pops page ids downwards, so a prefill of sequence after sequence
    # gets consecutive pages (descending) instead of W0/W1's shuffled ones
    "W3": dict(src="f16", pool="f16", B=4, L=32768, Hkv=8, D=128, scaled=False, seed=113, pages="fresh"),
    "W4": dict(src="bf16", pool="e4m3", B=4, L=32768, Hkv=8, D=128, scaled=True, seed=114, pages="fresh"),
}


@dataclass
class WriteWorkload:
    name: str
    k: torch.Tensor              # [n, Hkv, D] new rows
    v: torch.Tensor
    slots: torch.Tensor          # int64 [n]
    k_pool: torch.Tensor         # [P, Hkv, 16, D]
    v_pool: torch.Tensor
    k_scale: torch.Tensor | None
    v_scale: torch.Tensor | None
    meta: dict = field(default_factory=dict)

    @property
    def tokens(self) -> int:
        return self.k.shape[0]

    def algorithmic_bytes(self) -> int:
        """Rows read + rows written + slots (+ scales)."""
        n, hkv, d = self.k.shape
        b = n * hkv * d * 2 * (self.k.element_size() + self.k_pool.element_size()) + 8 * n
        return b + (8 if self.k_scale is not None else 0)


def make_write(name: str, *, device, data_seed: int | None = None) -> WriteWorkload:
    """Rows for sequences of L tokens laid out on a pool with 10 % spare pages
    (shuffled, or in a fresh cache's order); token t of sequence b goes to its
    page t // 16, row t % 16."""
    cfg = WRITE_CONFIGS[name]
    B, L, hkv, d = cfg["B"], cfg["L"], cfg["Hkv"], cfg["D"]
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(cfg["seed"] if data_seed is None else data_seed)
    pages_per_seq = (L + PAGE - 1) // PAGE
    P = B * pages_per_seq + max(1, B * pages_per_seq // 10)
    if cfg.get("pages", "shuffled") == "fresh":
        perm = (P - 1 - torch.arange(B * pages_per_seq, device=dev)).view(B, pages_per_seq)
    else:
        gp = torch.Generator(device=dev).manual_seed(cfg["seed"])
        perm = torch.randperm(P, device=dev, generator=gp)[:B * pages_per_seq].view(B, pages_per_seq)
    # a decode-step append writes the next row of partly filled pages
    t = torch.arange(L, device=dev) + (7 if L == 1 else 0)
    slots = (perm[:, t // PAGE] * PAGE + t % PAGE).reshape(-1).to(torch.int64)
    src = DTYPES[cfg["src"]]
    k = torch.randn(B * L, hkv, d, device=dev, generator=g).to(src)
    v = torch.randn(B * L, hkv, d, device=dev, generator=g).to(src)
    pool = DTYPES[cfg["pool"]]
    kp = torch.zeros(P, hkv, PAGE, d, dtype=pool, device=dev)
    vp = torch.zeros_like(kp)
    ks = vs = None
    if cfg["scaled"]:
        ks = torch.tensor(4.0 / 448.0, dtype=torch.float32, device=dev)
        vs = torch.tensor(4.0 / 448.0, dtype=torch.float32, device=dev)
    return WriteWorkload(name, k, v, slots, kp, vp, ks, vs, dict(cfg, num_pages=P))


def run_write(wl: WriteWorkload) -> None:
    """One store of ``wl``'s rows through the HIP write entry point."""
    from fskernels.hip.kv_write import paged_kv_write
    paged_kv_write(wl.k, wl.v, wl.k_pool, wl.v_pool, wl.slots, k_scale=wl.k_scale, v_scale=wl.v_scale)


def step_write(wl: Workload, *, seed: int = 0) -> WriteWorkload:
    """One decode step's KV append for ``wl``: a new token for each of its
    sequences (rows of q's dtype), stored into ``wl``'s own K/V (the pools
    of a paged workload, at row 0 of free pages past the ones in use; the
    last B rows of a varlen one, seen as a pool of one-row pages)."""
    dev = wl.k.device
    g = torch.Generator(device=dev).manual_seed(seed)
    rows = wl.q.dtype if wl.q.dtype != torch.float8_e4m3fn else torch.bfloat16
    k = torch.randn(wl.B, wl.Hkv, wl.D, device=dev, generator=g).to(rows)
    v = torch.randn(wl.B, wl.Hkv, wl.D, device=dev, generator=g).to(rows)
    if wl.layout == "paged":
        used = torch.zeros(wl.k.shape[0], dtype=torch.bool, device=dev)
        bt = wl.block_table.to(dev)
        used[bt[bt >= 0].long()] = True
        free = (~used).nonzero().flatten()
        if free.numel() < wl.B:
            raise ValueError("the pool has fewer free pages than sequences")
        slots = free[:wl.B] * PAGE
        kp, vp = wl.k, wl.v
    else:
        T = wl.k.shape[0]
        slots = T - wl.B + torch.arange(wl.B, device=dev)
        kp, vp = wl.k.unsqueeze(2), wl.v.unsqueeze(2)
    return WriteWorkload(f"{wl.name}-append", k, v, slots.to(torch.int64), kp, vp, wl.k_scale, wl.v_scale,
                         dict(src=str(rows).replace("torch.", ""), pool=str(wl.k.dtype).replace("torch.", ""),
                              scaled=wl.k_scale is not None))
