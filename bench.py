#!/usr/bin/env python3
"""Decode-step benchmark of the MI355X GQA flash-decode path.

A step is one decode call over one batch (default: the headline workload M0,
paged fp16 KV, B=4, Hq=32, Hkv=8, D=128, 32768 tokens per sequence, 16-token
pages scattered by a seeded permutation).  Inputs are generated on the GPU and
are resident in HBM before timing; at least 4 independent input sets are
rotated, with a footprint above 1.1 GB, beyond the 256 MB Infinity Cache.

Prints one JSON line.  ``value`` is the achieved algorithmic HBM bandwidth of a
whole step (valid K+V bytes + Q + output + block-table entries + lengths) in
GB/s; ``us_per_step`` and ``pct_of_peak`` (of 8 TB/s) are reported beside it.
``ms_per_step`` is the mean over the K timed steps (one wall-clock interval
between synchronisations); ``us_per_step_median`` is the median over groups of
10 steps of a following pass, from HIP events between the groups;
``host_us_per_step`` is the host time spent issuing the timed steps (a step
whose GPU work is shorter than this is host-bound).  ``--layers N`` makes a
step N decode calls over N independent caches (``--with-write``: each after a
one-token KV append), eager or, with ``--graph``, one captured graph.
``roofline`` is the split-KV partial kernel alone, timed with HIP events that
its own dispatches stamp (hipExtLaunchKernel) on every call of a further
pass of the same steps: the timing costs host time per call, so the step
timing runs without it.  ``cpu_baseline`` times the reference's PyTorch
decode path restated on the host (oracle/torch_ref.py) in the inputs' own
dtypes over the same workload, median of >= 3 runs, with the thread count.  The default
warm-up (300 steps) covers the ~20 ms the shader clock takes to settle under
load.

The default run (M0 with no other workload options) then times the other
decode configurations, C1..C5, the same way and adds them under ``configs``:
each with its own warm-up and step count set from elapsed time (about 0.3 s
of each, stated in the entry), its partial kernel's roofline (with the
counter traffic of profiles/partial_kernel_<config>_traffic.md) and a CPU
baseline of about 3 s; then C1 and C4 again with their lengths passed in host
memory (``C1:host``, ``C4:host``: the opt-in host-plan path, step times; the
dispatch-stamped kernel timing does not resolve those launches).
``--configs C2,C4`` picks others, ``--configs ''`` none.  ``--sweep`` runs only the reference benchmark's own sweep
(benchmarks/benchmark.py:20-33, 150-158: varlen fp16, lengths uniform in
[max(64, S/4), S], sinks 0.1 N(0,1) folded linearly; S = 512..32768 at B=4
and B = 1..32 at S=16384), one JSON line per point.

Other workloads: ``--config C1..C5`` (decode configurations), ``--config M0b``
(M0 with bf16 Q, KV and output), ``--config G1`` (varlen with sinks at head_dim
64, Hq=64, Hkv=8), ``--config G2`` (paged at head_dim 256, 16384 tokens per
sequence), ``--config W0..W4`` (the KV write path: a
step is one store of a batch of new rows into scattered pages; ``roofline`` is
the write kernel).  ``--graph`` replays each decode step from a captured HIP
graph; ``--block-scores`` also computes the pooled 128-token block scores.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

PEAK_HBM_GBS = 8000.0
METRIC = "µs/step + achieved HBM GB/s (% peak), paged GQA decode B=4 Hq32/Hkv8 D128 32K"


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=300,
                    help="untimed steps first (the shader clock takes ~20 ms of load to settle)")
    ap.add_argument("--config", default="M0", help="workload name (decode: M0, M0b, G1, G2, C1..C5; KV write: W0..W4)")
    ap.add_argument("--sets", type=int, default=0, help="input sets to rotate (0: >= 4 and enough for > 1.1 GB)")
    ap.add_argument("--chunk", type=int, default=0, help="split size in tokens (0: library default)")
    ap.add_argument("--block-scores", action="store_true",
                    help="also compute the pooled 128-token block scores in each step")
    ap.add_argument("--qk-engine", choices=["mfma", "valu"], default="mfma",
                    help="QK/PV on the matrix cores (default) or the VALU tile (A/B measurement; f16, D=128)")
    ap.add_argument("--option", action="append", default=[], metavar="NAME=VALUE",
                    help="library option (fsk_set_option) set before the run, e.g. head_pairs=0; repeatable")
    ap.add_argument("--graph", action="store_true",
                    help="replay each decode step from a captured HIP graph (no per-step host work)")
    ap.add_argument("--layers", type=int, default=1,
                    help="decode calls per step, over that many independent caches (one decode step of an "
                         "N-layer model); with --graph the whole step is one graph")
    ap.add_argument("--host-lengths", action="store_true",
                    help="pass the sequence lengths in host memory (the work plan is built on the host)")
    ap.add_argument("--with-write", action="store_true",
                    help="with --layers: each layer first stores one new token per sequence (KV write kernel)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline budget")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--traffic", default="",
                    help="rocprof summary holding 'bytes_per_launch: N' for the measured kernel "
                         "(default: profiles/partial_kernel_<config>_traffic.md, or "
                         "kv_write_kernel_<config>_traffic.md for W0..W4, if committed)")
    ap.add_argument("--wave-stamps", action="store_true",
                    help="load the wave-stamp build and print the partial kernel's per-wave timeline "
                         "(start-up, streaming, tail, dispatch) instead of the benchmark line")
    ap.add_argument("--configs", default=None, metavar="C1,C2,...",
                    help="decode configurations timed after the headline, each with a time-based warm-up and "
                         "step count (default with a plain M0 run: C1..C5; '' for none)")
    ap.add_argument("--sweep", action="store_true",
                    help="only the reference benchmark's sweep (varlen fp16, lengths U[max(64,S/4), S], "
                         "sinks 0.1 N(0,1), linear fold): S = 512..32768 at B=4, B = 1..32 at S=16384")
    ap.add_argument("--graph-host", action="store_true",
                    help="only the host-cost breakdown of graph replays of --config's decode call (torch "
                         "replay, direct hipGraphLaunch, 10-call graphs, capture modes, first replay)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run a plain device copy of BYTES (counter calibration under rocprof)")
    return ap.parse_args()


def rotation_sets(bytes_per_set: int) -> int:
    """Independent input sets rotated through the timed steps: at least 4, and
    enough that their footprint exceeds 1.1 GB (4x the 256 MB Infinity Cache),
    so no step reads another step's data out of cache."""
    return max(4, min(128, -(-1_100_000_000 // max(1, bytes_per_set))))


def copy_calibration(nbytes: int) -> None:
    """A plain copy of known size: under rocprofv3 --pmc its FETCH_SIZE /
    WRITE_SIZE per dispatch give the counters' scale factor."""
    import torch
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes}), flush=True)


def read_traffic(path: str):
    """bytes_per_launch from a committed rocprof summary, or None."""
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.strip().startswith("bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


# The kernel-timing pass stamps every call.  A stamped dispatch starts after a
# ~5-10 µs idle gap; a stamp on one call in several, right behind unstamped
# ones, makes that kernel run ~2 µs longer (M0, rocprofv3), so a sparse
# sample reads high.  Stamping every call reads within 0.5 % of the
# back-to-back kernel durations rocprofv3 reports.
KT_EVERY = 1


def median_step_us(step, first: int, steps: int, group: int = 10) -> float:
    """Median step time in µs: HIP events on the current stream between groups
    of ``group`` consecutive steps, over a pass of ``steps`` steps (at least 3
    groups) that follows the timed ones (each record costs host time, so the
    timed steps run without them).  Returns the median over groups of each
    group's time per step."""
    import torch

    n_groups = max(3, steps // group)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n_groups + 1)]
    i = first
    evs[0].record()
    for g in range(n_groups):
        for _ in range(group):
            step(i)
            i += 1
        evs[g + 1].record()
    torch.cuda.synchronize()
    return statistics.median(evs[g].elapsed_time(evs[g + 1]) * 1e3 / group for g in range(n_groups))


def kernel_timing_steps(steps: int) -> int:
    """Length of the kernel-timing pass that follows the timed steps (>= 50 samples)."""
    return KT_EVERY * max(steps // KT_EVERY, 50)


def host_threads():
    """Threads for the CPU baseline: the process's affinity mask, capped at
    OMP_NUM_THREADS when that is set (a GPU box sets it to the CPU share it
    gives one GPU).  Returns (threads, cpus in the affinity mask)."""
    n_aff = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS", "")
    n = min(n_aff, int(cap)) if cap.isdigit() and int(cap) > 0 else n_aff
    return n, n_aff


def _median_runs(fn, budget_s: float, min_runs: int = 3, max_runs: int = 50):
    """Median of >= min_runs timed calls of fn after one warm-up call, within
    about budget_s seconds.  Returns (median seconds, runs)."""
    fn()  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_runs or (time.perf_counter() < t_end and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baseline(wl, budget_s: float):
    """The reference's PyTorch decode path on the host (oracle/torch_ref.py:
    per-sequence gather, fp8 dequantisation, repeat_kv, matmul, softmax,
    matmul), timed over the whole step in the inputs' own dtypes, with an
    fp32-upcast variant beside it.  Median of >= 3 runs after a warm-up."""
    import torch

    from oracle import torch_ref as R

    threads, n_aff = host_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    cpu = lambda t: None if t is None else t.detach().cpu()  # noqa: E731
    q, k, v = cpu(wl.q), cpu(wl.k), cpu(wl.v)
    kw = dict(block_table=cpu(wl.block_table), cu_seqlens=cpu(wl.cu_seqlens), s_aux=cpu(wl.s_aux),
              k_scale=cpu(wl.k_scale), v_scale=cpu(wl.v_scale))
    alg = wl.algorithmic_bytes()
    compute = q.dtype  # f16 / bf16: the query's dtype, fp8 KV widened to it
    try:
        # the whole step when a run fits a quarter of the budget, else the
        # first sequences that do (timed, then scaled by their share of tokens)
        t0 = time.perf_counter()
        R.decode(q, k, v, wl.lens, seqs=[0], **kw)
        per_token = (time.perf_counter() - t0) / max(wl.lens[0], 1)
        seqs, tok = [], 0
        for b, L in enumerate(wl.lens):
            if seqs and (tok + L) * per_token > budget_s / 4:
                break
            seqs.append(b)
            tok += L
        share = tok / max(wl.total_tokens, 1)
        med, runs = _median_runs(lambda: R.decode(q, k, v, wl.lens, seqs=seqs, **kw), budget_s * 2 / 3)
        med32, runs32 = _median_runs(
            lambda: R.decode(q, k, v, wl.lens, seqs=seqs, compute_dtype=torch.float32, **kw), budget_s / 3)
    finally:
        torch.set_num_threads(prev)
    us_step = med / share * 1e6
    us_step32 = med32 / share * 1e6
    dt = str(compute).replace("torch.", "")
    sample = (f"the whole step ({wl.B} sequences, {wl.total_tokens} tokens)" if len(seqs) == wl.B else
              f"sequences 0..{len(seqs) - 1} of {wl.B} ({tok} of {wl.total_tokens} tokens), scaled to the step")
    return {
        "value": round(alg / (us_step * 1e-6) / 1e9, 3),
        "unit": "GB/s",
        "us_per_step": round(us_step, 1),
        "cores": threads,
        "affinity_cpus": n_aff,
        "kind": "port",
        "dtype": dt,
        "sample": f"host torch restatement of the reference's PyTorch decode path (per-sequence gather, "
                  f"repeat_kv, matmul, softmax, matmul in {dt}{', fp8 dequantised to ' + dt if wl.k_scale is not None else ''}) "
                  f"over {sample}, median of {runs} runs after a warm-up",
        "fp32_upcast": {"value": round(alg / (us_step32 * 1e-6) / 1e9, 3), "unit": "GB/s",
                        "us_per_step": round(us_step32, 1), "runs": runs32},
    }


def cpu_baseline_write(wl, budget_s: float):
    """The reference's row store on the host: the indexed assignment of
    fskernels/paged_attn/paged_kv_cache.py:128-130 (pool[page, :, row, :] =
    rows) for every token of the step at once, with the fixed-scale e4m3
    quantiser for scaled pools.  Median of >= 3 runs after a warm-up."""
    import torch

    threads, n_aff = host_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    k, v, slots = wl.k.cpu(), wl.v.cpu(), wl.slots.cpu()
    kp, vp = wl.k_pool.cpu(), wl.v_pool.cpu()
    pages, rows = slots // 16, slots % 16
    ks = None if wl.k_scale is None else wl.k_scale.cpu()
    vs = None if wl.v_scale is None else wl.v_scale.cpu()

    def store(pool, x, scale):
        if scale is not None:
            x = (x.float() / scale).clamp(-448.0, 448.0)
        pool[pages, :, rows, :] = x.to(pool.dtype)

    def step():
        store(kp, k, ks)
        store(vp, v, vs)
    try:
        med, runs = _median_runs(step, budget_s)
    finally:
        torch.set_num_threads(prev)
    return {
        "value": round(wl.algorithmic_bytes() / med / 1e9, 3),
        "unit": "GB/s",
        "us_per_step": round(med * 1e6, 1),
        "cores": threads,
        "affinity_cpus": n_aff,
        "kind": "port",
        "sample": f"host torch indexed store of all {wl.tokens} tokens of {wl.name} "
                  f"(the reference's append_kv assignment, batched), median of {runs} runs after a warm-up",
    }


def bench_write(args):
    """The KV write path: one store of a batch of rows into scattered pages."""
    import torch

    from fasterkernels_amd import native as nat
    from fasterkernels_amd import workloads as W

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    base = W.make_write(args.config, device=dev)
    alg_bytes = base.algorithmic_bytes()
    n_sets = args.sets or rotation_sets(alg_bytes)
    sets = [base] + [W.make_write(args.config, device=dev, data_seed=base.meta["seed"] + 1000 * i)
                     for i in range(1, n_sets)]
    for i in range(args.warmup):
        W.run_write(sets[i % n_sets])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        W.run_write(sets[i % n_sets])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    med_us = median_step_us(lambda i: W.run_write(sets[i % n_sets]), args.steps, args.steps)
    # kernel duration: a second timed pass of the same steps, the write kernels
    # stamped by their own dispatches (the hook costs host time, so it stays
    # out of the step timing above)
    nat.enable_kernel_timing(KT_EVERY)
    for i in range(kernel_timing_steps(args.steps)):
        W.run_write(sets[(args.steps + i) % n_sets])
    kern_ms_sum, _, calls = nat.kernel_timing()
    nat.enable_kernel_timing(0)
    kern_ms = kern_ms_sum / max(calls, 1)
    ms_step = elapsed * 1e3 / args.steps
    gbs = alg_bytes / (ms_step / 1e3) / 1e9
    kern_gbs = alg_bytes / (kern_ms / 1e3) / 1e9
    cfg = base.meta
    out = {
        "metric": f"KV write achieved HBM GB/s (rows read + written), {args.config}",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "us_per_step": round(ms_step * 1e3, 2),
        "us_per_step_median": round(med_us, 2),
        "pct_of_peak": round(100 * gbs / PEAK_HBM_GBS, 2),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"{cfg['src']}->{cfg['pool']}",
        "data": f"synthetic N(0,1), generated on device, {n_sets} rotating input sets",
        "config": {
            "workload": f"{args.config}: paged KV write of {base.tokens} tokens x Hkv={base.k.shape[1]} "
                        f"x D={base.k.shape[2]}, {cfg['src']} rows -> {cfg['pool']} pools"
                        + (" (fixed-scale quantisation)" if cfg["scaled"] else ""),
            "tokens": base.tokens, "algorithmic_bytes": alg_bytes,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(kern_gbs, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(kern_gbs / PEAK_HBM_GBS, 4),
            "traffic": read_traffic(args.traffic or os.path.join(
                os.path.dirname(os.path.abspath(__file__)), "profiles", f"kv_write_kernel_{args.config}_traffic.md")),
            "kernel": "kv_write_kernel",
            "kernel_avg_us": round(kern_ms * 1e3, 3),
        },
        "cpu_baseline": None if args.no_cpu else cpu_baseline_write(base, args.cpu_seconds),
    }
    print(json.dumps(out), flush=True)


def wave_timeline(args):
    """The partial kernel's per-wave timeline over several calls (after the
    warm-up), each the last of 20 back-to-back calls: medians over calls of
    each stage, in µs from the first wave's start (the s_memrealtime clock,
    100 MHz), and how far the XCDs' median ends lie apart within a call.  The
    kernel's own duration is the mean of its dispatch-stamped events over a
    separate back-to-back pass."""
    import numpy as np
    import torch

    from fasterkernels_amd import native as nat
    lib = nat.use_stamped_library()
    from fasterkernels_amd import workloads as W
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    for opt in args.option:
        name, _, value = opt.partition("=")
        nat.set_option(name, int(value))
    base = W.make(args.config, gen_device=dev, device=dev)
    n_sets = args.sets or rotation_sets(base.k.numel() * base.k.element_size() * 2)
    sets = [base] + [W.make(args.config, gen_device=dev, device=dev, data_seed=base.meta["seed"] + 1000 * i)
                     for i in range(1, n_sets)]
    hl = bool(args.host_lengths)
    for i in range(args.warmup):
        W.run(sets[i % n_sets], chunk_tokens=args.chunk, host_lengths=hl)
    n_rec = max(5, min(args.steps, 50))
    # The kernel's own duration: dispatch-stamped events on every call of a
    # separate back-to-back pass (its mean), as in the roofline pass.
    nat.enable_kernel_timing(1)
    for i in range(n_rec):
        W.run(sets[i % n_sets], chunk_tokens=args.chunk, host_lengths=hl)
    part_ms, _, n_timed = nat.kernel_timing()
    nat.enable_kernel_timing(0)
    kernel_us = part_ms * 1e3 / max(n_timed, 1)
    nat.check(lib.fsk_debug_clear_wave_stamps())
    calls = []
    for r in range(n_rec):
        # The recorded call is the last of 20 back-to-back calls, as in the
        # timed steps: every wave of a call rewrites its own stamp slots, so
        # the buffer read after the synchronisation holds that call's
        # timeline.  (A call launched right after a synchronisation is not
        # representative: its waves start together, but their first tiles
        # arrive XCD by XCD, up to ~8 µs apart.)
        for i in range(20):
            W.run(sets[(r + i) % n_sets], chunk_tokens=args.chunk, host_lengths=hl)
        torch.cuda.synchronize()
        buf = np.zeros(4096 * 16, dtype=np.uint64)
        nat.check(lib.fsk_debug_wave_stamps(buf.ctypes.data, 4096))
        st = buf.reshape(4096, 16).astype(np.int64)
        wg = np.arange(4096)[st[:, 0] > 0]   # workgroup ids of the waves that ran
        st = st[st[:, 0] > 0]
        t0 = st[:, 0].min()
        us = lambda col: (st[:, col] - t0) * 0.01  # noqa: E731
        work = st[:, 5] > 0
        xcc = st[:, 6] & 0xF
        # the first round of the grid (one workgroup per SIMD, dispatched first)
        first_round = wg < 4 * torch.cuda.get_device_properties(dev).multi_processor_count

        def med(x):
            return float(np.median(x)) if len(x) else None
        seg = st[:, 5]
        ends = us(3)[work]
        last = np.argsort(ends)[-16:]  # the 16 waves that end last
        by_seg = {}
        for k, sel in (("1", seg == 1), ("2", seg == 2), ("3", seg == 3), ("4plus", seg >= 4)):
            by_seg[f"items_{k}_segments"] = int((work & sel).sum())
            by_seg[f"end_median_us_{k}_segments"] = med(us(3)[work & sel])
        xmed = [float(np.median(us(3)[work & (xcc == x)])) if (work & (xcc == x)).any() else None
                for x in range(8)]
        xvals = [v for v in xmed if v is not None]
        calls.append({
            "first_round_first_tile_us": med(us(2)[work & first_round]),
            "second_round_first_tile_us": med(us(2)[work & ~first_round]),
            "first_round_end_median_us": med(us(3)[work & first_round]),
            "second_round_end_median_us": med(us(3)[work & ~first_round]),
            "one_segment_end_median_us": med(us(3)[work & (st[:, 5] == 1)]),
            "two_segment_end_median_us": med(us(3)[work & (st[:, 5] == 2)]),
            "two_segment_items": int((work & (st[:, 5] == 2)).sum()),
            "waves": int(len(st)), "working_waves": int(work.sum()),
            "start_spread_us": float(us(0).max()),
            "plan_us_after_wave_start": float(np.median((st[:, 1] - st[:, 0]) * 0.01)),
            # the plan's stages: lengths loaded and summed, the split (with
            # the lead-in decision), the prefix tables
            "plan_lengths_us": float(np.median((st[:, 10] - st[:, 0]) * 0.01)),
            "plan_split_us": float(np.median((st[:, 11] - st[:, 10]) * 0.01)),
            "plan_prefix_us": float(np.median((st[:, 1] - st[:, 11]) * 0.01)),
            # paged: first item's set-up after the plan, its page window + Q round trip, then its first tiles
            "item_setup_us": med(((st[:, 8] - st[:, 1]) * 0.01)[work & (st[:, 8] > 0)]),
            "window_round_trip_us": med(((st[:, 9] - st[:, 8]) * 0.01)[work & (st[:, 9] > 0)]),
            "first_tile_after_window_us": med(((st[:, 2] - st[:, 9]) * 0.01)[work & (st[:, 9] > 0) & (st[:, 2] > 0)]),
            "first_tile_us": float(np.median(us(2)[work])),
            "first_tile_p90_us": float(np.percentile(us(2)[work], 90)),
            "end_p10_us": float(np.percentile(us(3)[work], 10)),
            "end_median_us": float(np.median(us(3)[work])),
            "end_max_us": float(us(3)[work].max()),
            "exit_max_us": float(us(4).max()),
            "last16_mean_segments": float(seg[work][last].mean()),
            "last16_first_tile_us": float(np.median(us(2)[work][last])),
            **by_seg,
            "xcd_end_median_us": xmed,
            # per call: latest minus earliest XCD median end, and the last exit after their mean
            "xcd_spread_us": float(max(xvals) - min(xvals)) if xvals else None,
            "exit_after_xcd_mean_us": float(us(4).max() - np.mean(xvals)) if xvals else None,
        })
    med = {"kernel_us": round(kernel_us, 2)}
    # which XCD ends late changes from call to call: the spread of each XCD's
    # deviation from its call's mean (std over calls)
    X = np.array([[v if v is not None else np.nan for v in c["xcd_end_median_us"]] for c in calls])
    dev_ = X - np.nanmean(X, axis=1, keepdims=True)
    med["xcd_deviation_std_us"] = [round(float(v), 2) for v in np.nanstd(dev_, axis=0)]
    for k in calls[0]:
        vals = [c[k] for c in calls if k != "xcd_end_median_us" and c[k] is not None]
        if k != "xcd_end_median_us":
            med[k] = round(float(np.median(vals)), 2) if vals else None
    med["xcd_end_median_us"] = [round(float(np.median([c["xcd_end_median_us"][x] for c in calls
                                                        if c["xcd_end_median_us"][x] is not None])), 2)
                                for x in range(8)]
    med["decomposition_us"] = {
        "start_up": med["first_tile_us"],                                   # first wave start -> first tile (median)
        "streaming": round(med["end_p10_us"] - med["first_tile_us"], 2),    # until the first 10 % of items end
        "tail": round(med["exit_max_us"] - med["end_p10_us"], 2),           # until the last wave exits
        "outside_waves": round(med["kernel_us"] - med["exit_max_us"], 2),   # dispatch before and after the waves
    }
    print(json.dumps({"wave_timeline": args.config, "calls": len(calls), "chunk_tokens": args.chunk or "auto",
                      "options": args.option, "algorithmic_bytes": base.algorithmic_bytes(), **med}), flush=True)


def graph_host(args) -> None:
    """Where a replayed decode graph's host time goes, for one configuration
    (--config, default M0; use C1 or C4 for small steps): per decode call,
    host µs to issue and GPU-bound µs per step, for eager calls, torch's
    CUDAGraph.replay(), hipGraphLaunch called directly on the same
    executable graph (ctypes, no torch wrapper), a graph of 10 decode calls,
    graphs captured in the thread-local and relaxed capture modes, and the
    first replay after instantiation.  One input set (the host costs are the
    subject; steps are cache-resident)."""
    import ctypes

    import torch

    from fasterkernels_amd import workloads as W
    from fskernels.engine.hip_graph import DecodeGraph
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipGraphLaunch.restype = ctypes.c_int
    hip.hipGraphLaunch.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    wl = W.make(args.config, gen_device=dev, device=dev)
    n = max(args.steps, 500)

    def per_call(fn, calls=1):
        for _ in range(50):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        return {"host_us": round((t1 - t0) / n / calls * 1e6, 2), "gpu_bound_us": round((t2 - t0) / n / calls * 1e6, 2)}

    out = {"graph_host": args.config, "calls": n}
    out["eager"] = per_call(lambda: W.run(wl))
    g = DecodeGraph(W.run, wl)
    out["torch_replay"] = per_call(g.graph.replay)
    ex, stream = g.graph.raw_cuda_graph_exec(), torch.cuda.current_stream().cuda_stream
    st = hip.hipGraphLaunch(ex, stream)
    if st != 0:
        raise RuntimeError(f"hipGraphLaunch returned {st}")
    out["hipGraphLaunch_direct"] = per_call(lambda: hip.hipGraphLaunch(ex, stream))

    def ten():
        r = None
        for _ in range(10):
            r = W.run(wl)
        return r
    g10 = DecodeGraph(ten)
    out["torch_replay_10_calls_per_call"] = per_call(g10.graph.replay, 10)
    for mode in ("thread_local", "relaxed"):
        gm = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gm, capture_error_mode=mode):
            W.run(wl)
        out[f"torch_replay_capture_{mode}"] = per_call(gm.replay)
    gf = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gf):
        W.run(wl)
    torch.cuda.synchronize()
    firsts = []
    for _ in range(2):
        t0 = time.perf_counter()
        gf.replay()
        firsts.append(round((time.perf_counter() - t0) * 1e6, 1))
        torch.cuda.synchronize()
    out["first_and_second_replay_host_us"] = firsts
    print(json.dumps(out), flush=True)


# Decode configurations timed beside the headline in the default run (the
# other decode configurations of the benchmark definition).  Each gets its own
# warm-up and step count, set from elapsed time (the headline keeps the counts
# the command line gives), and a bounded CPU-baseline budget.
SUB_CONFIGS = ("C1", "C2", "C3", "C4", "C5", "C1:host", "C4:host")
# "<config>:host": the same workload with its lengths passed in host memory
# (the host-plan entry points; an opt-in of this build, the drop-in path keeps
# device lengths).
SUB_WARMUP_S = 0.3    # warm-up: at least this long (and at least 50 steps in all)
SUB_TIMED_S = 0.3     # timed steps: about this long (100 to 5000 steps)
SUB_CPU_S = 3.0       # CPU-baseline budget per configuration (seconds)


def decode_sets(config: str, dev, layers: int = 1, sets: int = 0):
    """The rotating input sets of a decode workload: the same lengths and page
    tables with independent Q/K/V data, at least 4 sets and a footprint above
    1.1 GB, in whole groups of ``layers``."""
    from fasterkernels_amd import workloads as W
    base = W.make(config, gen_device=dev, device=dev)
    kv_bytes = base.k.numel() * base.k.element_size() * 2
    n_sets = sets or rotation_sets(kv_bytes)
    n_sets = -(-max(n_sets, layers) // layers) * layers
    out = [base] + [W.make(config, gen_device=dev, device=dev, data_seed=base.meta["seed"] + 1000 * i)
                    for i in range(1, n_sets)]
    assert all(s.lens == base.lens for s in out)
    return out


def timed_pass(step, steps: int, warmup: int):
    """``warmup`` untimed steps, then ``steps`` timed ones between two
    synchronisations, then the median pass.  Returns (elapsed s, host issue
    s, median µs per step)."""
    import torch
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    issued = time.perf_counter() - t0   # host time to issue the steps (the host-bound limit)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    return elapsed, issued, median_step_us(step, steps, steps)


def time_based_counts(step, warm_s: float, timed_s: float):
    """(warm-up steps, timed steps) for a configuration: a step time estimated
    from 10 steps after 10 others (those 20 count towards the warm-up), then
    a warm-up of at least ``warm_s`` and a timed region of about ``timed_s``."""
    import torch
    for i in range(10):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(10, 20):
        step(i)
    torch.cuda.synchronize()
    est = max((time.perf_counter() - t0) / 10, 1e-6)
    warmup = max(30, int(math.ceil(warm_s / est)))
    steps = min(5000, max(100, int(math.ceil(timed_s / est))))
    return 20 + warmup, steps, est


def decode_kernel_pass(sets, n_steps: int, chunk: int, block_scores: bool, layers: int):
    """A further pass of ``n_steps`` steps with every decode call's partial
    and reduce kernels stamped by their own dispatches.  Returns (partial ms,
    partial-start-to-reduce-end ms, calls) summed."""
    from fasterkernels_amd import native as nat
    from fasterkernels_amd import workloads as W
    n_sets = len(sets)
    nat.enable_kernel_timing(KT_EVERY)
    for i in range(n_steps):
        for j in range(layers):
            W.run(sets[(i * layers + j) % n_sets], chunk_tokens=chunk, block_scores=block_scores)
    part_ms, tot_ms, calls = nat.kernel_timing()
    nat.enable_kernel_timing(0)
    return part_ms, tot_ms, calls


def traffic_path(config: str, kernel: str = "partial_kernel") -> str:
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"{kernel}_{config}_traffic.md")


def dtype_name(t) -> str:
    import torch
    return {torch.float16: "f16", torch.bfloat16: "bf16", torch.float8_e4m3fn: "e4m3"}[t]


def workload_name(config: str, wl) -> str:
    return (f"{config}: {wl.layout} GQA decode B={wl.B} Hq={wl.Hq} Hkv={wl.Hkv} D={wl.D} "
            f"tokens={wl.total_tokens} kv={str(wl.k.dtype).replace('torch.', '')}")


def measure_decode(sets, *, sink_mode: str = "exp", warm_s: float = SUB_WARMUP_S,
                   timed_s: float = SUB_TIMED_S, host_lengths: bool = False) -> dict:
    """Step and kernel timing of eager decode calls over rotating input sets,
    with a time-based warm-up and step count (see time_based_counts)."""
    from fasterkernels_amd import native as nat
    from fasterkernels_amd import workloads as W
    n_sets = len(sets)

    def step(i):
        return W.run(sets[i % n_sets], sink_mode=sink_mode, host_lengths=host_lengths)

    warmup, steps, est = time_based_counts(step, warm_s, timed_s)
    elapsed, issued, med_us = timed_pass(step, steps, warmup - 20)
    nat.enable_kernel_timing(KT_EVERY)
    for i in range(kernel_timing_steps(steps)):
        step(steps + i)
    part_ms, tot_ms, calls = nat.kernel_timing()
    nat.enable_kernel_timing(0)
    base = sets[0]
    alg = base.algorithmic_bytes()
    us_step = elapsed * 1e6 / steps
    part_us = part_ms * 1e3 / max(calls, 1)
    kern_gbs = alg / (part_us * 1e-6) / 1e9 if part_us > 0 else None
    gbs = alg / (us_step * 1e-6) / 1e9
    return {
        "value": round(gbs, 2),
        "unit": "GB/s",
        "us_per_step": round(us_step, 2),
        "us_per_step_median": round(med_us, 2),
        "host_us_per_step": round(issued * 1e6 / steps, 2),
        "ms_per_step": round(us_step / 1e3, 5),
        "pct_of_peak": round(100 * gbs / PEAK_HBM_GBS, 2),
        "steps": steps,
        "warmup": warmup,
        "warmup_rule": f"{warm_s} s of steps (>= 30) after a 20-step estimate; timed steps ~{timed_s} s "
                       f"(100..5000); estimate {est * 1e6:.1f} us/step",
        "dtype": dtype_name(base.k.dtype),
        "data": f"synthetic N(0,1), generated on device, {n_sets} rotating input sets",
        "batch": base.B, "total_tokens": base.total_tokens, "algorithmic_bytes": alg,
        "roofline": {
            "bound": "hbm",
            "achieved": None if kern_gbs is None else round(kern_gbs, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": None if kern_gbs is None else round(kern_gbs / PEAK_HBM_GBS, 4),
            "kernel": "partial_kernel (split-KV partials)",
            "kernel_avg_us": round(part_us, 3),
            "partial_plus_reduce_avg_us": round(tot_ms * 1e3 / max(calls, 1), 3),
            "kernel_calls_timed": calls,
        },
    }


def release(sets) -> None:
    import torch
    sets.clear()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def sub_config(config: str, dev, cpu_seconds: float, no_cpu: bool) -> dict:
    """One decode configuration measured the way the headline is (rotating
    HBM-resident inputs, eager decode calls, the partial kernel timed by its
    own dispatches), with a time-based warm-up and step count."""
    t_start = time.perf_counter()
    base_name, _, mode = config.partition(":")
    host = mode == "host"
    sets = decode_sets(base_name, dev)
    m = measure_decode(sets, host_lengths=host)
    entry = {"workload": workload_name(base_name, sets[0]) + (", lengths in host memory" if host else ""),
             "sinks": None if sets[0].s_aux is None else "N(0,1), exp fold (sink logit)", **m}
    if host:
        entry["roofline"]["traffic"] = None
        entry["roofline"]["note"] = ("dispatch-stamped events do not resolve host-plan launches: use the step time "
                                     "or a rocprofv3 kernel trace for the partial kernel")
        entry["cpu_baseline"] = None
        entry["cpu_baseline_note"] = f"the same workload as {base_name}'s entry"
    else:
        entry["roofline"]["traffic"] = read_traffic(traffic_path(base_name))
        entry["cpu_baseline"] = None if no_cpu else cpu_baseline(sets[0], cpu_seconds)
    release(sets)
    entry["wall_s"] = round(time.perf_counter() - t_start, 2)
    return entry


# The reference's own benchmark sweep (benchmarks/benchmark.py:150-158):
# maximum length at B=4, then batch at a maximum length of 16384.
SWEEP_SEQ_LENS = (512, 1024, 2048, 4096, 8192, 16384, 32768)
SWEEP_BATCHES = (1, 2, 4, 8, 16, 32)


def reference_sweep(args) -> None:
    """The reference benchmark's workload on this GPU: varlen fp16 decode,
    Hq=32, Hkv=8, D=128, lengths uniform in [max(64, S/4), S], sinks
    0.1 N(0,1) folded linearly (as the reference kernels do); one JSON line
    per point, then a summary line."""
    import torch

    from fasterkernels_amd import workloads as W
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    points = [("seq_len", 4, S) for S in SWEEP_SEQ_LENS] + [("batch", B, 16384) for B in SWEEP_BATCHES]
    rows = []
    for kind, B, S in points:
        base = W.reference_sweep_workload(B, S, gen_device=dev, device=dev)
        n_sets = rotation_sets(base.k.numel() * base.k.element_size() * 2)
        sets = [base] + [W.reference_sweep_workload(B, S, gen_device=dev, device=dev, data_seed=4200 + i)
                         for i in range(1, n_sets)]
        m = measure_decode(sets, sink_mode="linear", host_lengths=args.host_lengths)
        row = {"sweep": kind, "B": B, "max_S": S, "lens": list(base.lens), "host_lengths": bool(args.host_lengths),
               **m}
        release(sets)
        rows.append(row)
        print(json.dumps(row), flush=True)
    print(json.dumps({"reference_sweep": [{k: r[k] for k in ("sweep", "B", "max_S", "total_tokens",
                                                          "us_per_step", "us_per_step_median", "value")}
                                           | {"kernel_us": r["roofline"]["kernel_avg_us"],
                                              "frac": r["roofline"]["frac"]} for r in rows]}), flush=True)


def main():
    args = parse()
    if args.wave_stamps:
        wave_timeline(args)
        return
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU (sharding the path across GPUs is a design "
                                   "only), so --gpus must be 1", "n_gpus": args.gpus}))
        sys.exit(2)
    import torch

    from fasterkernels_amd import native as nat
    from fasterkernels_amd import workloads as W

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no HIP GPU visible"}))
        sys.exit(2)
    if args.config in W.WRITE_CONFIGS:
        bench_write(args)
        return
    if args.sweep:
        reference_sweep(args)
        return
    if args.graph_host:
        graph_host(args)
        return
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    nat.set_option("qk_engine", 1 if args.qk_engine == "valu" else 0)
    for opt in args.option:
        name, _, value = opt.partition("=")
        nat.set_option(name, int(value))
    L = max(1, args.layers)
    sets = decode_sets(args.config, dev, L, args.sets)
    base = sets[0]
    n_sets = len(sets)
    alg_bytes = base.algorithmic_bytes() * L
    writes = [W.step_write(s, seed=5000 + i) for i, s in enumerate(sets)] if args.with_write else None
    if args.with_write:
        alg_bytes += sum(w.algorithmic_bytes() for w in writes[:L])

    def layer_calls(g):
        """The decode calls (and KV writes) of step group g, layer by layer."""
        out = None
        for j in range(g * L, g * L + L):
            if writes is not None:
                W.run_write(writes[j])
            out = W.run(sets[j], chunk_tokens=args.chunk, block_scores=args.block_scores,
                        host_lengths=args.host_lengths)
        return out

    n_groups = n_sets // L
    if args.graph:
        from fskernels.engine.hip_graph import DecodeGraph
        graphs = [DecodeGraph(layer_calls, g) for g in range(n_groups)]

        def step(i):
            return graphs[i % n_groups].replay()
    else:
        def step(i):
            return layer_calls(i % n_groups)

    elapsed, issued, med_us = timed_pass(step, args.steps, args.warmup)
    # Kernel durations: a second timed pass of the same steps, with timing on
    # the calls KT_EVERY selects (the timing costs host time, so it stays out
    # of the step timing above).
    n_kt = kernel_timing_steps(args.steps)
    if args.graph:
        # the library's hook does not run inside a replay: HIP events around the replay
        evs = []
        for i in range(n_kt):
            if i % KT_EVERY:
                step(args.steps + i)
                continue
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            step(args.steps + i)
            b.record()
            evs.append((a, b))
        torch.cuda.synchronize()
        tot_ms = sum(a.elapsed_time(b) for a, b in evs)
        part_ms, calls = 0.0, len(evs)
        tot_ms /= L  # per decode call of the replayed step
    else:
        # the partial and reduce kernels stamped by their own dispatches
        # (decode calls only: the write kernels' stamps would join the triples)
        part_ms, tot_ms, calls = decode_kernel_pass(sets, n_kt, args.chunk, args.block_scores, L)

    ms_step = elapsed * 1e3 / args.steps
    gbs = alg_bytes / (ms_step / 1e3) / 1e9
    part_avg_ms = part_ms / max(calls, 1)
    if args.graph:   # the replay (partial + reduce) is the timed unit
        part_avg_ms = tot_ms / max(calls, 1)
    call_bytes = base.algorithmic_bytes()
    kern_gbs = call_bytes / (part_avg_ms / 1e3) / 1e9 if part_avg_ms > 0 else None
    plain = not (args.chunk or args.graph or args.block_scores or args.qk_engine != "mfma" or args.option or L > 1)
    traffic = read_traffic(args.traffic or traffic_path(args.config)) if plain else None

    out = {
        "metric": METRIC if (args.config == "M0" and L == 1) else (
            f"µs/step + achieved HBM GB/s (% peak), {base.layout} GQA decode {args.config}"
            + (f" x {L} layers" + (" with KV writes" if args.with_write else "") if L > 1 else "")),
        "value": round(gbs, 2),
        "unit": "GB/s",
        "us_per_step": round(ms_step * 1e3, 2),
        "us_per_step_median": round(med_us, 2),
        "host_us_per_step": round(issued * 1e6 / args.steps, 2),
        "pct_of_peak": round(100 * gbs / PEAK_HBM_GBS, 2),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype_name(base.k.dtype),
        "data": f"synthetic N(0,1), generated on device, {n_sets} rotating input sets",
        "config": {
            "workload": workload_name(args.config, base),
            "batch": base.B, "total_tokens": base.total_tokens, "algorithmic_bytes": alg_bytes,
            "chunk_tokens": args.chunk or "auto",
            "launch": "hip graph replay" if args.graph else "eager",
            "qk_engine": args.qk_engine,
            "options": args.option,
            "block_scores": bool(args.block_scores),
            "layers": L,
            "with_write": bool(args.with_write),
            "host_lengths": bool(args.host_lengths),
            "us_per_call": round(ms_step * 1e3 / L, 2),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": None if kern_gbs is None else round(kern_gbs, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": None if kern_gbs is None else round(kern_gbs / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "kernel": ("partial_kernel + reduce_kernel (graph replay time per decode call)" if args.graph
                       else "partial_kernel (split-KV partials)"),
            "kernel_avg_us": round(part_avg_ms * 1e3, 3),
            "partial_plus_reduce_avg_us": round(tot_ms / max(calls, 1) * 1e3, 3),
        },
        "cpu_baseline": None,
    }
    if args.host_lengths:
        # Measured: the dispatch-stamped events read host-plan launches as long
        # as (or longer than) device-length ones, while the steps, the kernel
        # traces of rocprofv3 and the wave stamps all show them ~1 µs shorter.
        out["roofline"]["note"] = ("dispatch-stamped events do not resolve host-plan launches: use the step time "
                                   "or a rocprofv3 kernel trace for the partial kernel")
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(sets[0], args.cpu_seconds)
    del sets, base, writes
    if args.graph:
        del graphs
    subs = [c.strip() for c in args.configs.split(",") if c.strip()] if args.configs else []
    if args.configs is None and args.config == "M0" and plain:
        subs = list(SUB_CONFIGS)
    if subs:
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        out["configs"] = {}
        for name in subs:
            base_name, _, mode = name.partition(":")
            if base_name not in W.CONFIGS or mode not in ("", "host"):
                raise SystemExit(f"--configs: unknown decode configuration {name!r}")
            print(f"# timing {name}", file=sys.stderr, flush=True)
            if mode:
                # an opt-in variant of a workload already reported: its failure is
                # recorded in its entry and does not take the line down
                try:
                    out["configs"][name] = sub_config(name, dev, SUB_CPU_S, args.no_cpu)
                except Exception as e:  # noqa: BLE001
                    out["configs"][name] = {"error": f"{type(e).__name__}: {e}"}
            else:
                out["configs"][name] = sub_config(name, dev, SUB_CPU_S, args.no_cpu)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
