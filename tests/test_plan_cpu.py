"""Invariants of the decode kernels' device-side work plan, checked on the host.

fsk_debug_split runs the same split_geometry / chunk_lo / chunk_of / item_of
code that every workgroup of the partial kernel runs, compiled for the host.
The split policy arguments are the ones a decode call passes (automatic
splits: chunk bounds 128..4096 tokens, down to 64 for short streams, 4 items
per CU, the workspace capacity the host sizes; fixed splits: one chunk size,
no XCD skew).  Checked: chunk
sizes and alignment, contiguous coverage of the token stream, the token ->
chunk map, room for every partial in the workspace, and that work items map
one-to-one onto (chunk, head slot) pairs with the long chunks on even XCDs.
No GPU needed.
"""
import ctypes

import numpy as np
import pytest

from fasterkernels_amd import native as nat

CHUNK_MIN, CHUNK_MAX, SKEW_MIN, SHORT_CHUNK, CHUNK_PREF = 128, 4096, 512, 64, 2432


def cdiv(a, b):
    return -(-a // b)


def doubled_target(target, total, cpref, cmax):
    """The chunk count bound of a split: doubled once past cpref, then while
    chunks would exceed cmax."""
    t = target * 2 if target < cdiv(total, cpref) else target
    while t < cdiv(total, cmax) and t < (1 << 24):
        t *= 2
    return t


def host_policy(total, B, NH, cus, fixed=0, skew=3, most=0, kv_bytes=2):
    """(chunk_min, chunk_max, chunk_pref, target_units, u_max, xcd_skew) as the host sets
    them for a stream of `total` padded tokens (stream bound total + 128 B);
    `most` > 0: an automatic split of chunks of at most `most` tokens (a
    negative chunk_tokens); kv_bytes: bytes per KV element."""
    bound = total + 128 * B

    def unit_bound(c):
        return cdiv(bound, c) + B + 1

    if fixed:
        return fixed, fixed, fixed, 1, unit_bound(fixed), 0
    cmax = min(most, CHUNK_MAX) if most else CHUNK_MAX
    cmin = CHUNK_MIN if cmax >= CHUNK_MIN else min(SHORT_CHUNK, cmax)
    cpref = max(cmin, min(cmax, CHUNK_PREF * 2 // kv_bytes // 128 * 128))
    target = max(1, cus * 4 // NH)
    cap = max(4 * target, 256)
    u_plan = unit_bound(cmin)
    if bound < target * CHUNK_MIN:
        u_plan = max(u_plan, min(unit_bound(SHORT_CHUNK), 33 * B + 1))
    t = doubled_target(target, bound, cpref, cmax)  # chunk_bound, less one
    return cmin, cmax, cpref, target, max(t + 1 + B + 1, min(u_plan, cap)), skew


def split(total, cmin, cmax, cpref, target, u_max, B, skew, NH, align):
    lib = nat.load()
    geo = (ctypes.c_int32 * 4)()
    nat.check(lib.fsk_debug_split(total, cmin, cmax, cpref, target, u_max, B, skew, NH, align, geo, None, None, None, None))
    ce, co, n, paired = list(geo)
    starts = np.zeros(max(n, 1), np.int32)
    ic = np.zeros(max(n * NH, 1), np.int32)
    isl = np.zeros(max(n * NH, 1), np.int32)
    tok = np.zeros(max(total, 1), np.int32)
    nat.check(lib.fsk_debug_split(total, cmin, cmax, cpref, target, u_max, B, skew, NH, align, geo,
                                  starts.ctypes.data, ic.ctypes.data, isl.ctypes.data, tok.ctypes.data))
    return ce, co, n, bool(paired), starts[:n], ic[:n * NH], isl[:n * NH], tok[:total]


def check_case(total, B, NH, cus, fixed, skew, align):
    cmin, cmax, cpref, target, u_max, skew = host_policy(total, B, NH, cus, fixed, skew)
    ce, co, n, paired, starts, ic, isl, tok = split(total, cmin, cmax, cpref, target, u_max, B, skew, NH, align)
    what = f"total={total} B={B} NH={NH} cus={cus} fixed={fixed} skew={skew} align={align}: ce={ce} co={co} n={n}"
    # chunk sizes
    assert ce % align == 0 and co % align == 0 and co >= align and ce <= cmax, what
    if paired:
        assert skew > 0 and co < ce and (ce + co) % 2 == 0 and (ce + co) // 2 >= SKEW_MIN, what
        assert n % 2 == 0 and (n * NH) % 8 == 0, what
    else:
        # automatic splits of short streams go down to SHORT_CHUNK (rounded to align)
        lo = cmin if cmin == cmax else min(cmin, cdiv(SHORT_CHUNK, align) * align)
        assert ce == co and lo <= ce <= cmax, what
    # contiguous coverage of [0, total): chunk j starts where chunk j-1 ends
    lens = np.where(np.arange(n) % 2 == 0, ce, co)
    assert n == len(starts)
    if n:
        assert starts[0] == 0, what
        assert np.array_equal(starts[1:], np.cumsum(lens)[:-1]), what
    if total == 0:
        assert n == 0, what
    else:
        assert starts[-1] + lens[-1] >= total, what
        # at most the one trailing chunk an even count adds lies past the stream
        assert starts[-1] < total or (paired and starts[-2] < total), what
    # token -> chunk map
    x = np.arange(total)
    assert np.array_equal(tok, np.searchsorted(starts, x, side="right") - 1), what
    # every partial fits: at most n + B of them, and the workspace holds u_max
    assert n + B + 1 <= u_max, what
    # at most the target count of chunks (doubled once past chunk_pref, then
    # while chunks would exceed chunk_max) plus one: the host sizes the
    # persistent grid on this bound
    assert n <= doubled_target(target, total, cpref, cmax) + 1, what
    # work items: a bijection onto (chunk, head slot), long chunks on even XCDs
    assert ((ic >= 0) & (ic < n) & (isl >= 0) & (isl < NH)).all(), what
    assert len(np.unique(ic.astype(np.int64) * NH + isl)) == n * NH, what
    if paired:
        assert np.array_equal(ic % 2, np.arange(n * NH) % 2), what
    return paired


def test_split_rejects_bad_arguments():
    lib = nat.load()
    geo = (ctypes.c_int32 * 4)()
    bad = [
        (-1, 128, 2048, 2048, 1, 100, 1, 0, 8, 32),
        (100, 16, 2048, 2048, 1, 100, 1, 0, 8, 32),      # chunk_min below 32
        (100, 128, 64, 64, 1, 100, 1, 0, 8, 32),         # chunk_max below chunk_min
        (100, 96, 2048, 2048, 1, 100, 1, 0, 8, 128),     # not a multiple of align
        (100, 128, 2048, 64, 1, 100, 1, 0, 8, 32),       # chunk_pref below chunk_min
        (100, 128, 2048, 4096, 1, 100, 1, 0, 8, 32),     # chunk_pref above chunk_max
        (100, 128, 2048, 2048, 0, 100, 1, 0, 8, 32),     # no target
        (100, 128, 2048, 2048, 1, 100, 1, 0, 0, 32),     # no head slots
        (100, 128, 2048, 2048, 1, 100, 1, 0, 8, 48),     # align
        (100, 128, 2048, 2048, 1, 100, 1, 51, 8, 32),    # skew
    ]
    for args in bad:
        assert lib.fsk_debug_split(*args, geo, None, None, None, None) == nat.FSK_ERR_INVALID, args


@pytest.mark.parametrize("total", [0, 32, 128, 4096, 131072, 131072 + 32, 1_000_000])
@pytest.mark.parametrize("NH", [8, 4, 16, 3])
def test_split_headline_and_edge_streams(total, NH):
    for align in (32, 128):
        total_a = cdiv(total, align) * align
        check_case(total_a, 4, NH, 256, 0, 3, align)


def test_split_m0_geometry():
    """M0: 131072 tokens, 8 KV heads, 256 CUs -> 1056/992-token chunk pairs,
    128 chunks, the long ones on the even XCDs."""
    ce, co, n, paired, *_ = split(131072, *host_policy(131072, 4, 8, 256)[:5], 4, 3, 8, 32)
    assert (ce, co, n, paired) == (1056, 992, 128, True)


@pytest.mark.parametrize("total,B,kv_bytes,want", [
    (524288, 128, 2, (2112, 1984, 256)), (507904, 124, 2, (2048, 1920, 256)), (393216, 96, 2, (1600, 1472, 256)),
    (327680, 80, 2, (1344, 1216, 256)), (262144, 64, 2, (2112, 1984, 128)), (278528, 32, 2, (2272, 2080, 128)),
    (300896, 32, 2, (2464, 2272, 128)), (655360, 160, 2, (2656, 2464, 256)), (819200, 200, 2, (3296, 3104, 256)), (393216, 96, 1, (3168, 2976, 128))])
def test_split_long_streams(total, B, kv_bytes, want):
    """Streams longer than 128 chunks of 2432 16-bit tokens (8 KV heads, 256
    CUs) take twice as many chunks, once: B=128 x 4096 tokens gets 256 chunk
    pairs of 2112/1984 tokens, not 128 of 4096; B=160 x 4096 keeps 256
    chunks of 2560 rather than 512; e4m3 KV (1 byte) splits at twice the
    tokens."""
    ce, co, n, paired, *_ = split(total, *host_policy(total, B, 8, 256, kv_bytes=kv_bytes)[:5], B, 3, 8, 32)
    assert (ce, co, n) == want and paired


@pytest.mark.parametrize("total,B,want", [(5120, 4, 96), (4096, 4, 64), (2048, 4, 64), (8192, 4, 128),
                                          (16384, 4, 128), (4096, 1, 128), (2048, 1, 64), (4096, 2, 64)])
def test_split_short_streams(total, B, want):
    """Streams too short for 128 chunks of 128 tokens (8 KV heads, 256 CUs)
    take half as many chunks, of 64 to 128 tokens, while that averages at
    most 32 chunks per sequence; from 8192 tokens up the split is the plain
    128-token one.  Block scores (align 128) keep 128."""
    ce, co, n, paired, *_ = split(total, *host_policy(total, B, 8, 256)[:5], B, 3, 8, 32)
    assert (ce, co, paired) == (want, want, False) and n == cdiv(total, want)
    ce, *_ = split(total, *host_policy(total, B, 8, 256)[:5], B, 3, 8, 128)
    assert ce == 128


@pytest.mark.parametrize("most", [32, 64, 96, 512, 1024, 4096])
@pytest.mark.parametrize("total,B", [(4096, 4), (131072, 4), (131072, 1), (297_167, 32), (2_000_000, 16)])
def test_split_chunk_size_caps(most, total, B):
    """Automatic splits with a chunk-size cap (negative chunk_tokens, the
    dense split-count hint): chunks never exceed the cap, the usual
    invariants hold, and a capped split has at least as many chunks as
    cdiv(total, cap) and as the uncapped one."""
    for align in (32, 128):
        if most % align:
            continue
        total_a = cdiv(total, align) * align
        pol = host_policy(total_a, B, 8, 256, most=most)
        ce, co, n, *_ = split(total_a, *pol[:5], B, pol[5], 8, align)
        assert max(ce, co) <= most and n >= cdiv(total_a, most)
        n_auto = split(total_a, *host_policy(total_a, B, 8, 256)[:5], B, 3, 8, align)[2]
        assert n >= n_auto or max(ce, co) < most
        check_case_policy(total_a, B, 8, pol, align)


def check_case_policy(total, B, NH, pol, align):
    cmin, cmax, cpref, target, u_max, skew = pol
    ce, co, n, paired, starts, ic, isl, tok = split(total, cmin, cmax, cpref, target, u_max, B, skew, NH, align)
    assert ce % align == 0 and co % align == 0 and co >= align and ce <= cmax
    lens = np.where(np.arange(n) % 2 == 0, ce, co)
    if n:
        assert starts[0] == 0 and np.array_equal(starts[1:], np.cumsum(lens)[:-1])
        assert starts[-1] + lens[-1] >= total
    assert np.array_equal(tok, np.searchsorted(starts, np.arange(total), side="right") - 1)
    assert n + B + 1 <= u_max
    assert len(np.unique(ic.astype(np.int64) * NH + isl)) == n * NH


def test_split_random_policies():
    r = np.random.default_rng(0)
    seen_paired = seen_plain = 0
    for _ in range(1500):
        align = int(r.choice([32, 128]))
        B = int(r.integers(1, 300))
        total = int(r.choice([r.integers(0, 5000), r.integers(0, 300_000), r.integers(0, 3_000_000)]))
        total = cdiv(total, align) * align
        NH = int(r.choice([1, 2, 3, 4, 5, 8, 12, 16, 32, 64]))
        cus = int(r.choice([1, 32, 80, 256, 304]))
        fixed = int(r.choice([0, 0, 0, align, 2 * align, 1024, 4096])) if align == 32 else int(
            r.choice([0, 0, 0, 128, 256, 2048]))
        skew = int(r.choice([0, 3, 6, 20, 50]))
        if check_case(total, B, NH, cus, fixed, skew, align):
            seen_paired += 1
        else:
            seen_plain += 1
    assert seen_paired > 100 and seen_plain > 100


def split_model(total, cmin, cmax, cpref, target_units, u_max, B, skew, NH, align):
    """The split policy in plain integer arithmetic (Python's unbounded ints,
    real divisions): the chunk count target (doubled once past chunk_pref,
    then while chunks would exceed chunk_max, up to 2^24), the short-stream
    halving, the workspace cap and the XCD-skewed long/short pairs.  The
    device computes the same choice with multiply-shift divisors and a
    chunk reciprocal; this states it without them."""
    up = lambda x: cdiv(x, align) * align  # noqa: E731
    target = target_units
    if target < cdiv(total, cpref):
        target *= 2
    while target < cdiv(total, cmax) and target < (1 << 24):
        target *= 2
    want, lo, hi = cdiv(total, target), cmin, cmax
    if want < lo and cmin < cmax:
        w2 = cdiv(total, max(target // 2, 1))
        lo2 = up(SHORT_CHUNK)
        hi2 = max(cmin, lo2)
        if cdiv(total, min(max(up(w2), lo2), hi2)) <= 32 * B:
            want, lo, hi = w2, lo2, hi2
    chunk = min(max(up(want), lo), hi)
    cap = u_max - B - 1 if u_max > B + 1 else 0
    chunk = min(max(chunk, up(cdiv(total, cap))), cmax) if cap > 0 else cmax
    geo = (chunk, chunk, cdiv(total, chunk), 0)
    if skew > 0 and chunk >= SKEW_MIN and total > 0:
        ce = min(up(chunk * (100 + skew) // 100), cmax)
        co = 2 * chunk - ce
        q, r = divmod(total, 2 * chunk)
        n = 2 * q + (r > 0) + (r > ce)
        n += n & 1
        if align <= co < ce and n <= cap and (n * NH) % 8 == 0:
            geo = (ce, co, n, 1)
    return geo


def test_split_matches_the_policy_model():
    """The device's division-free split gives exactly split_model's choice:
    every policy the host sets (as in test_split_random_policies) and
    arbitrary argument sets within the entry point's bounds, including
    streams near 2^31 tokens, odd target counts and workspace caps that
    bind."""
    lib = nat.load()
    geo = (ctypes.c_int32 * 4)()
    r = np.random.default_rng(11)
    cases = []
    for _ in range(3000):
        align = int(r.choice([32, 128]))
        B = int(r.choice([1, 4, 32, 64, 65, int(r.integers(1, 5000))]))
        total = int(r.choice([r.integers(0, 5000), r.integers(0, 1 << 20), r.integers(0, (1 << 31) - 4097)]))
        total = cdiv(total, align) * align if r.random() < 0.8 else total
        NH = int(r.choice([1, 3, 4, 8, 16, int(r.integers(1, 1 << 16))]))
        cus = int(r.choice([1, 32, 80, 256, 304]))
        fixed = int(r.choice([0, 0, 0, align, 2 * align, 1024 // align * align, 4096]))
        skew = int(r.choice([0, 3, 6, 20, 50]))
        pol = list(host_policy(total, B, NH, cus, fixed, skew, most=int(r.choice([0, 0, 64, 512])) // align * align))
        if pol[0] % align or pol[1] % align or pol[2] % align:
            continue
        cases.append((total, *pol[:5], B, pol[5], NH, align))
    for _ in range(3000):
        align = int(r.choice([32, 128]))
        cmin = align * int(r.integers(1, 9))
        cmax = max(cmin, int(r.choice([cmin, cmin * int(r.integers(1, 40)), 4096 // align * align,
                                       (1 << int(r.integers(7, 25))) // align * align])))
        cpref = align * int(r.integers(cmin // align, cmax // align + 1))
        tu = int(r.choice([1, 2, 3, 5, 7, 64, 85, 128, 341, int(r.integers(1, (1 << 20) + 1))]))
        B = int(r.choice([0, 1, 4, 64, 200, int(r.integers(0, 5000))]))
        u_max = int(r.choice([0, B + 1, B + 2, int(r.integers(0, 100_000)), (1 << 31) - 1]))
        total = int(r.choice([r.integers(0, 4096), r.integers(0, 1 << 20), r.integers(0, (1 << 31) - 4097),
                              tu * cpref, tu * cpref + 1, tu * cmax, (1 << 31) - 4097]))
        total = min(total, (1 << 31) - 4097)
        cases.append((total, cmin, cmax, cpref, tu, u_max, B, int(r.choice([0, 3, 10, 50])),
                      int(r.choice([1, 4, 8, int(r.integers(1, 1 << 16))])), align))
    for args in cases:
        nat.check(lib.fsk_debug_split(*args, geo, None, None, None, None))
        assert tuple(geo) == split_model(*args), args
