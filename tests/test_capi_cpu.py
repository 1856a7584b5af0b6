"""CPU checks of the C ABI: the library loads, exports exactly what
include/fsk_decode.h declares, and rejects bad arguments on the host before
any HIP call (so these run without a GPU)."""
import ctypes
import os
import re
import subprocess

import pytest
import torch

from fasterkernels_amd import native as nat

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "fsk_decode.h")
FAKE = 0x10000  # 64 KiB-aligned dummy address; never dereferenced on the host


def header_functions(instrumented=False):
    """Functions the header declares (those of the instrumented build, inside
    #ifdef FSK_WAVE_STAMPS, only when ``instrumented``)."""
    text = open(HEADER).read()
    if not instrumented:
        text = re.sub(r"#ifdef FSK_WAVE_STAMPS.*?#endif", "", text, flags=re.S)
    return sorted(set(re.findall(r"FSK_API\s+[\w\s\*]+?\b(fsk_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(nat.LIB_PATH):
        from fasterkernels_amd import build
        build.build()
    return nat.load()


def test_exports_match_header(lib):
    declared = header_functions()
    assert len(declared) >= 10
    out = subprocess.run(["nm", "-D", "--defined-only", nat.LIB_PATH], capture_output=True, text=True).stdout
    exported = sorted(set(re.findall(r"\bT (fsk_\w+)", out)))
    assert exported == declared
    assert sorted(nat.SIGNATURES) == declared
    for name in declared:
        assert getattr(lib, name) is not None


def test_instrumented_library_exports():
    """The wave-stamp build exports the same C ABI plus its two debug entry
    points, under the same soname (so the torch binding binds to whichever
    of the two libraries the process loaded first)."""
    from fasterkernels_amd import build
    if not os.path.exists(build.STAMPS_PATH):
        pytest.skip("libfsk_decode_stamps.so not built")
    out = subprocess.run(["nm", "-D", "--defined-only", build.STAMPS_PATH], capture_output=True, text=True).stdout
    exported = sorted(set(re.findall(r"\bT (fsk_\w+)", out)))
    assert exported == header_functions(instrumented=True)
    assert set(exported) - set(header_functions()) == set(nat.STAMP_SIGNATURES)
    dyn = subprocess.run(["readelf", "-d", build.STAMPS_PATH], capture_output=True, text=True).stdout
    assert "SONAME" in dyn and "[libfsk_decode.so]" in dyn


def test_version_and_options(lib):
    assert lib.fsk_version() == 1
    assert lib.fsk_set_option(b"no_such_option", 1) == nat.FSK_ERR_INVALID
    assert b"unknown option" in lib.fsk_last_error()
    assert lib.fsk_set_option(b"chunk_tokens", 33) == nat.FSK_ERR_INVALID
    assert lib.fsk_set_option(b"chunk_tokens", 0) == nat.FSK_OK
    assert lib.fsk_set_option(b"waves_per_cu", 0) == nat.FSK_ERR_INVALID
    assert lib.fsk_set_option(b"waves_per_cu", 8) == nat.FSK_OK
    for name in (b"qk_engine", b"head_pairs"):
        assert lib.fsk_set_option(name, 2) == nat.FSK_ERR_INVALID
        assert lib.fsk_set_option(name, -1) == nat.FSK_ERR_INVALID
    assert lib.fsk_set_option(b"qk_engine", 0) == nat.FSK_OK
    assert lib.fsk_set_option(b"head_pairs", 1) == nat.FSK_OK
    for bad in (-1, 33, 288):  # a multiple of 32 in [0, 256]
        assert lib.fsk_set_option(b"seg_tokens", bad) == nat.FSK_ERR_INVALID
    for ok in (0, 256, 96):
        assert lib.fsk_set_option(b"seg_tokens", ok) == nat.FSK_OK


def test_workspace_bytes(lib):
    f = lib.fsk_workspace_bytes
    a = f(nat.FSK_LAYOUT_PAGED, 4, 32, 8, 128, 2048, 16, 512)
    b = f(nat.FSK_LAYOUT_PAGED, 4, 32, 8, 128, 2048, 16, 256)
    assert 0 < a < b  # smaller splits -> more partials
    # partial storage: units * Hkv * G * (D + 2) floats, plus the unit table
    units = 4 * (2048 * 16 // 512)
    assert a >= units * 8 * 4 * 130 * 4
    assert f(nat.FSK_LAYOUT_VARLEN, 4, 32, 8, 128, 10000, 0, 0) > 0
    assert f(nat.FSK_LAYOUT_DENSE, 4, 32, 8, 64, 4096, 0, 0) > 0
    assert f(7, 4, 32, 8, 128, 2048, 16, 0) == nat.FSK_ERR_INVALID
    assert f(nat.FSK_LAYOUT_PAGED, 4, 30, 8, 128, 2048, 16, 0) == nat.FSK_ERR_INVALID
    assert f(nat.FSK_LAYOUT_PAGED, 4, 32, 8, 96, 2048, 16, 0) == nat.FSK_ERR_UNSUPPORTED
    assert f(nat.FSK_LAYOUT_PAGED, 4, 32, 8, 128, 2048, 24, 0) == nat.FSK_ERR_UNSUPPORTED
    assert f(nat.FSK_LAYOUT_PAGED, 4, 32, 8, 128, 2048, 16, 48) == nat.FSK_ERR_INVALID


def test_workspace_sizes_reject_overflowing_shapes(lib):
    assert lib.fsk_score_workspace_bytes(1 << 30, 1 << 16, 1 << 24) == nat.FSK_ERR_UNSUPPORTED
    assert lib.fsk_score_workspace_bytes(4, 1 << 20, 256) == nat.FSK_ERR_UNSUPPORTED
    assert lib.fsk_score_workspace_bytes(16384, 1 << 16, 1 << 24) > 0
    assert lib.fsk_workspace_bytes(nat.FSK_LAYOUT_PAGED, 4, 1 << 20, 8, 128, 2048, 16, 0) == nat.FSK_ERR_UNSUPPORTED
    assert lib.fsk_workspace_bytes(nat.FSK_LAYOUT_PAGED, 1 << 20, 32, 8, 128, 2048, 16, 0) == nat.FSK_ERR_UNSUPPORTED


def test_workspace_size_cache_is_bounded(lib, monkeypatch):
    """A varlen serving loop asks for a new total length every step: the
    cached sizes must not grow without bound."""
    monkeypatch.setattr(nat, "launch", lambda device_index, fn, *args: fn(*args))
    nat._WS_CACHE.clear()
    try:
        sizes = {nat.workspace_bytes(nat.FSK_LAYOUT_VARLEN, 4, 32, 8, 128, 1000 + t, 16, 0, 0)
                 for t in range(nat._WS_CACHE_MAX + 10)}
        assert min(sizes) > 0
        assert 0 < len(nat._WS_CACHE) <= nat._WS_CACHE_MAX
    finally:
        nat._WS_CACHE.clear()


def paged_args(**kw):
    """A valid argument set for fsk_decode_paged (fake pointers), overridable."""
    a = dict(q=FAKE, q_sb=32 * 128, q_sh=128, k=FAKE, k_sp=8 * 16 * 128, k_sh=16 * 128, k_st=128,
             v=FAKE, v_sp=8 * 16 * 128, v_sh=16 * 128, v_st=128, bt=FAKE, bt_sb=64, mb=64, lens=FAKE,
             P=100, ps=16, sink=None, mode=0, ks=None, vs=None, out=FAKE, o_sb=32 * 128, o_sh=128,
             B=4, Hq=32, Hkv=8, D=128, qdt=nat.FSK_F16, kvdt=nat.FSK_F16, odt=nat.FSK_F16,
             scale=0.088, ws=FAKE, wsb=1 << 30, chunk=0, stream=None)
    a.update(kw)
    return list(a.values())


@pytest.mark.parametrize("override,code", [
    (dict(q=None), nat.FSK_ERR_INVALID),
    (dict(lens=None), nat.FSK_ERR_INVALID),
    (dict(bt=None), nat.FSK_ERR_INVALID),
    (dict(Hq=30), nat.FSK_ERR_INVALID),
    (dict(D=96), nat.FSK_ERR_UNSUPPORTED),
    (dict(ps=24), nat.FSK_ERR_UNSUPPORTED),
    (dict(mode=5), nat.FSK_ERR_INVALID),
    (dict(odt=nat.FSK_E4M3), nat.FSK_ERR_UNSUPPORTED),
    (dict(kvdt=nat.FSK_BF16), nat.FSK_ERR_UNSUPPORTED),        # q f16 with bf16 KV
    (dict(kvdt=nat.FSK_E4M3), nat.FSK_ERR_INVALID),            # fp8 KV without scales
    (dict(qdt=nat.FSK_E4M3, kvdt=nat.FSK_E4M3, ks=FAKE, vs=FAKE), nat.FSK_ERR_UNSUPPORTED),
    (dict(k_st=100), nat.FSK_ERR_INVALID),                     # rows not 16-byte aligned
    (dict(k_st=64), nat.FSK_ERR_INVALID),                      # overlapping rows
    (dict(q=FAKE + 2), nat.FSK_ERR_INVALID),
    (dict(bt_sb=10), nat.FSK_ERR_INVALID),                     # row stride < width
    (dict(P=0), nat.FSK_ERR_INVALID),
    (dict(ws=None), nat.FSK_ERR_WORKSPACE),
    (dict(wsb=1024), nat.FSK_ERR_WORKSPACE),
    (dict(chunk=48), nat.FSK_ERR_INVALID),
    (dict(chunk=4096 + 32), nat.FSK_ERR_UNSUPPORTED),         # above the 256-page window
    (dict(scale=float("nan")), nat.FSK_ERR_INVALID),
    # size arithmetic stays inside int64: strides, heads and batch are bounded
    (dict(q_sb=(1 << 62) + 8), nat.FSK_ERR_UNSUPPORTED),
    (dict(k_sp=1 << 40), nat.FSK_ERR_UNSUPPORTED),
    (dict(bt_sb=(1 << 63) - 1), nat.FSK_ERR_UNSUPPORTED),
    (dict(o_sh=-128), nat.FSK_ERR_INVALID),
    (dict(k_st=-128), nat.FSK_ERR_INVALID),
    (dict(Hq=1 << 17, Hkv=8), nat.FSK_ERR_UNSUPPORTED),
    (dict(B=16385), nat.FSK_ERR_UNSUPPORTED),
])
def test_paged_validation(lib, override, code):
    assert lib.fsk_decode_paged(*paged_args(**override)) == code
    assert lib.fsk_last_error()  # a message explains the status


def test_host_length_entries(lib):
    """The host-length entry points validate like the device-length ones,
    read the lengths from host memory, refuse more than 64 sequences, and
    otherwise reach the launch (which fails here, without a GPU, with the
    device-length entry's status)."""
    lens = (ctypes.c_int32 * 65)(*([100] * 65))
    host = ctypes.cast(lens, ctypes.c_void_p).value
    assert lib.fsk_decode_paged_host(*paged_args(lens=None)) == nat.FSK_ERR_INVALID
    assert lib.fsk_decode_paged_host(*paged_args(lens=host, D=96)) == nat.FSK_ERR_UNSUPPORTED
    assert lib.fsk_decode_paged_host(*paged_args(lens=host, B=65)) == nat.FSK_ERR_UNSUPPORTED
    assert b"64" in lib.fsk_last_error()
    want = lib.fsk_decode_paged(*paged_args())
    assert want != nat.FSK_OK
    assert lib.fsk_decode_paged_host(*paged_args(lens=host)) == want
    assert lib.fsk_decode_paged_host(*paged_args(lens=host, B=64)) == want
    cu = (ctypes.c_int32 * 65)(*range(0, 650, 10))
    ok = [FAKE, 32 * 128, 128, FAKE, 8 * 128, 128, FAKE, 8 * 128, 128, ctypes.cast(cu, ctypes.c_void_p).value,
          1000, None, 0, None, None, FAKE, 32 * 128, 128, 4, 32, 8, 128, nat.FSK_F16, nat.FSK_F16, nat.FSK_F16,
          0.088, FAKE, 1 << 30, 0, None]
    dev = list(ok)
    dev[9] = FAKE
    assert lib.fsk_decode_varlen_host(*ok) == lib.fsk_decode_varlen(*dev) != nat.FSK_OK
    bad = list(ok)
    bad[18] = 65
    assert lib.fsk_decode_varlen_host(*bad) == nat.FSK_ERR_UNSUPPORTED


def test_varlen_and_dense_validation(lib):
    ok = [FAKE, 32 * 128, 128, FAKE, 8 * 128, 128, FAKE, 8 * 128, 128, FAKE, 1000, None, 0, None, None,
          FAKE, 32 * 128, 128, 4, 32, 8, 128, nat.FSK_F16, nat.FSK_F16, nat.FSK_F16, 0.088, FAKE, 1 << 30, 0,
          None]
    bad = list(ok)
    bad[21] = 80  # head_dim
    assert lib.fsk_decode_varlen(*bad) == nat.FSK_ERR_UNSUPPORTED
    bad = list(ok)
    bad[9] = None  # cu_seqlens
    assert lib.fsk_decode_varlen(*bad) == nat.FSK_ERR_INVALID
    bad = list(ok)
    bad[3] = None  # k, with 1000 rows
    assert lib.fsk_decode_varlen(*bad) == nat.FSK_ERR_INVALID
    assert b"null" in lib.fsk_last_error()
    dense = [FAKE, 32 * 128, 128, FAKE, 8 * 512 * 128, 512 * 128, 128, FAKE, 8 * 512 * 128, 512 * 128, 128,
             512, FAKE, None, None, 0, None, None, None, FAKE, 32 * 128, 128, 4, 32, 8, 128,
             nat.FSK_E4M3, nat.FSK_E4M3, nat.FSK_F16, 0.088, FAKE, 1 << 30, 0, None]
    assert lib.fsk_decode_dense(*dense) == nat.FSK_ERR_INVALID  # e4m3 KV without scales
    assert b"scale" in lib.fsk_last_error()


def test_debug_entry_validation(lib):
    assert lib.fsk_fp8_decode_table(None, None) == nat.FSK_ERR_INVALID
    assert lib.fsk_paged_gather(None, 0, 0, 0, FAKE, 4, 4, FAKE, 8, 16, 2, 8, 128, 0, FAKE, None) == nat.FSK_ERR_INVALID
    assert lib.fsk_paged_gather(FAKE, 1, 1, 128, FAKE, 4, 4, FAKE, 8, 16, 2, 8, 128, 0, FAKE, None) == nat.FSK_ERR_INVALID
    assert lib.fsk_paged_gather(FAKE, 8 * 16 * 128, 16 * 128, 128, FAKE, 4, 4, FAKE, 8, 16, 2, 8, 128,
                                nat.FSK_F32, FAKE, None) == nat.FSK_ERR_UNSUPPORTED


def write_args(**kw):
    """A valid argument set for fsk_paged_write (fake pointers), overridable."""
    a = dict(k=FAKE, k_st=8 * 128, k_sh=128, v=FAKE, v_st=8 * 128, v_sh=128, slots=FAKE, n=4,
             kp=FAKE, kp_sp=8 * 16 * 128, kp_sh=16 * 128, kp_st=128, vp=FAKE, vp_sp=8 * 16 * 128,
             vp_sh=16 * 128, vp_st=128, P=100, ps=16, Hkv=8, D=128, sdt=nat.FSK_F16, pdt=nat.FSK_F16,
             ks=None, vs=None, bt=None, bt_numel=0, upd=None, n_upd=0, stream=None)
    a.update(kw)
    return list(a.values())


@pytest.mark.parametrize("override,code", [
    (dict(k=None), nat.FSK_ERR_INVALID),
    (dict(slots=None), nat.FSK_ERR_INVALID),
    (dict(n=-1), nat.FSK_ERR_INVALID),
    (dict(Hkv=0), nat.FSK_ERR_INVALID),
    (dict(D=100), nat.FSK_ERR_UNSUPPORTED),                    # not a multiple of 8
    (dict(D=4096), nat.FSK_ERR_UNSUPPORTED),
    (dict(ps=0), nat.FSK_ERR_INVALID),
    (dict(P=0), nat.FSK_ERR_INVALID),
    (dict(sdt=nat.FSK_E4M3), nat.FSK_ERR_UNSUPPORTED),         # source must be f16/bf16/f32
    (dict(pdt=nat.FSK_F32), nat.FSK_ERR_UNSUPPORTED),
    (dict(ks=FAKE), nat.FSK_ERR_INVALID),                      # one scale only
    (dict(ks=FAKE, vs=FAKE), nat.FSK_ERR_INVALID),             # scales on an f16 pool
    (dict(k=FAKE + 8), nat.FSK_ERR_INVALID),                   # unaligned source rows
    (dict(k_st=100), nat.FSK_ERR_INVALID),
    (dict(kp_st=100), nat.FSK_ERR_INVALID),
    (dict(kp_st=64), nat.FSK_ERR_INVALID),                     # overlapping pool rows
    (dict(kp_sh=-16), nat.FSK_ERR_INVALID),
    (dict(n_upd=2, upd=FAKE), nat.FSK_ERR_INVALID),            # updates without a block table
    (dict(P=1 << 28, ps=16), nat.FSK_ERR_UNSUPPORTED),         # 2^32 slots
    (dict(n=1 << 40), nat.FSK_ERR_UNSUPPORTED),                # size products stay inside int64
    (dict(k_st=(1 << 62) + 8), nat.FSK_ERR_UNSUPPORTED),
    (dict(kp_sp=1 << 40), nat.FSK_ERR_UNSUPPORTED),
    (dict(Hkv=1 << 20), nat.FSK_ERR_UNSUPPORTED),
])
def test_paged_write_validation(lib, override, code):
    assert lib.fsk_paged_write(*write_args(**override)) == code
    assert lib.fsk_last_error()


def test_paged_write_noop_without_gpu(lib):
    # nothing to store and nothing to update: returns before any HIP call
    assert lib.fsk_paged_write(*write_args(n=0, k=None, v=None, kp=None, vp=None, slots=None)) == nat.FSK_OK


def test_no_bit_cast_of_vector_elements():
    """This hipcc lowers __builtin_bit_cast(T, vec[i]) to a load of the
    vector's first element; the sources must go through a scalar instead."""
    from fasterkernels_amd import build
    src = open(build.SRC).read()
    bad = re.findall(r"__builtin_bit_cast\(\s*\w+\s*,\s*\w+\s*\[[^]]*\]\s*\)", src)
    assert not bad, bad


def test_write_kernels_load_whole_source_groups():
    """Every column group of the KV write kernels loads 16 bytes of an f16 /
    bf16 source (32 of f32) and widens all eight elements.  A thread's first
    row is loaded ahead of the loop (before the scale), the others in it, so
    each kernel has two load sites and one store site."""
    from fasterkernels_amd import build
    res = subprocess.run([build.hipcc(), *[f for f in build.compile_flags() if f not in ("-shared", "-fPIC")],
                          "--cuda-device-only", "-S", build.SRC, "-o", "-"],
                         capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stderr[-2000:]
    rows = 2  # load sites of a row
    found = 0
    for m in re.finditer(r"\n(_ZN12_GLOBAL__N_115kv_write_kernelILi(\d)ELi(\d)ELb(\d)\w*):[^\n]*\n(.*?)s_endpgm",
                         res.stdout, re.S):
        src_dt, pool_dt, body = int(m.group(2)), int(m.group(3)), m.group(5)
        x4 = len(re.findall(r"global_load_dwordx4", body))
        assert x4 == rows * (2 if src_dt == nat.FSK_F32 else 1), (m.group(1), x4, rows)
        if src_dt == nat.FSK_F16 and pool_dt != nat.FSK_F16:
            assert len(re.findall(r"v_cvt_f32_f16", body)) == 8, m.group(1)
        found += 1
    assert found == 12


def test_timing_hook_without_gpu(lib):
    a, b, n = ctypes.c_double(), ctypes.c_double(), ctypes.c_int64()
    assert lib.fsk_enable_kernel_timing(1) == nat.FSK_OK
    assert lib.fsk_kernel_timing(ctypes.byref(a), ctypes.byref(b), ctypes.byref(n)) == nat.FSK_OK
    assert n.value == 0
    assert lib.fsk_enable_kernel_timing(0) == nat.FSK_OK
    assert lib.fsk_kernel_timing(None, None, None) == nat.FSK_ERR_INVALID


def test_python_wrappers_reject_host_tensors():
    from fskernels.hip import paged_flash_decode, flash_decode_gqa_varlen
    q = torch.zeros(2, 32, 128, dtype=torch.float16)
    k = torch.zeros(4, 8, 16, 128, dtype=torch.float16)
    bt = torch.zeros(2, 2, dtype=torch.int32)
    with pytest.raises(RuntimeError):
        paged_flash_decode(q, k, k, bt, torch.tensor([3, 4], dtype=torch.int32), 16)
    with pytest.raises(RuntimeError):
        flash_decode_gqa_varlen(q, k[0], k[0], torch.tensor([0, 1, 2], dtype=torch.int32))


def test_fp8_kernels_keep_both_convert_halves():
    """Regression guard for the compiler: every e4m3 widening in the decode
    kernels must keep its high-word form (op_sel) next to the low-word one.
    (A debug kernel that widened the converted values straight to fp32 lost
    the high-word form in this compiler; the decode kernels must not.)"""
    from fasterkernels_amd import build
    res = subprocess.run([build.hipcc(), *[f for f in build.compile_flags() if f not in ("-shared", "-fPIC")],
                          "--cuda-device-only", "-S", build.SRC, "-o", "-"],
                         capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stderr[-2000:]
    asm = res.stdout
    kernels = re.split(r"\n(?=_ZN12_GLOBAL__N_114partial_kernel)", asm)
    checked = 0
    for k in kernels[1:]:
        name = k.split(":", 1)[0]
        body = k.split("s_endpgm", 1)[0]
        for ins in ("v_cvt_scalef32_pk_f16_fp8", "v_cvt_scalef32_pk_bf16_fp8"):
            lo = len(re.findall(ins + r" v\d+, v\d+, 1\.0\s*$", body, re.M))
            hi = len(re.findall(ins + r" .*op_sel", body))
            assert lo == hi, f"{name}: {ins} low {lo} vs high {hi}"
            checked += lo
    assert checked > 0


def test_partial_kernels_keep_uniform_state_in_scalars():
    """Every decode kernel keeps its work-plan state wave-uniform: no private
    (scratch) memory and no readfirstlane loop around a buffer load, which
    this compiler emits when a buffer resource is built from a value it
    cannot prove uniform (a select lowered to a table in scratch, a value
    leaving a loop whose bound came out of a wave shuffle).  And each takes
    its lengths pointers and batch size preloaded in SGPRs (5 dwords), its
    first memory instruction past the preload prologue being a length load,
    not a kernel-argument load."""
    from fasterkernels_amd import build
    res = subprocess.run([build.hipcc(), *[f for f in build.compile_flags() if f not in ("-shared", "-fPIC")],
                          "--cuda-device-only", "-S", build.SRC, "-o", "-"],
                         capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stderr[-2000:]
    asm = res.stdout
    names = re.findall(r"^(_ZN12_GLOBAL__N_114partial_kernel\w*):", asm, re.M)
    assert len(names) >= 40
    for name in names:
        body = asm[asm.index(name + ":"):]
        body = body[:body.index(".Lfunc_end")]
        meta = asm[asm.index(".amdhsa_kernel " + name):][:4000]
        scratch = int(re.search(r"amdhsa_private_segment_fixed_size (\d+)", meta).group(1))
        waterfalls = len(re.findall(r"v_cmp_eq_u64_e32 vcc, s\[\d+:\d+\], v\[", body))
        assert scratch == 0 and waterfalls == 0, (name, scratch, waterfalls)
        preload = int(re.search(r"amdhsa_user_sgpr_kernarg_preload_length (\d+)", meta).group(1))
        entry = body.split("s_branch", 1)[1]
        first = re.search(r"^\s+((?:global|buffer|flat|s)_load\w*)", entry, re.M).group(1)
        assert preload == 5 and first.startswith("global_load"), (name, preload, first)


def test_xcd_skew_option(lib):
    assert lib.fsk_set_option(b"xcd_skew", -1) == nat.FSK_ERR_INVALID
    assert lib.fsk_set_option(b"xcd_skew", 51) == nat.FSK_ERR_INVALID
    assert lib.fsk_set_option(b"xcd_skew", 0) == nat.FSK_OK
    assert lib.fsk_set_option(b"xcd_skew", 3) == nat.FSK_OK


def test_chunk_pref_option(lib):
    for bad in (0, 64, 200, 4224, 8192):
        assert lib.fsk_set_option(b"chunk_pref", bad) == nat.FSK_ERR_INVALID, bad
    assert lib.fsk_set_option(b"chunk_pref", 4096) == nat.FSK_OK
    assert lib.fsk_set_option(b"chunk_pref", 2432) == nat.FSK_OK


def test_workspace_holds_the_doubled_split(lib):
    """A stream over 128 chunks of 2432 tokens (8 KV heads) plans 256
    chunks: the workspace holds them, whatever chunk_pref says (the query
    sizes for 16-bit KV, the smallest chunk ceiling)."""
    cus = 256  # MI355X's CU count, and the library's count where no GPU is visible
    per_unit = 8 * 4 * (128 + 2) * 4
    need = nat.workspace_bytes(nat.FSK_LAYOUT_PAGED, 128, 32, 8, 128, 256, 16, 0)
    assert need >= (2 * max(1, cus * 4 // 8) + 1 + 128 + 1) * per_unit


def test_torch_binding_loads_with_the_library():
    """The torch binding is built next to the library, links that same file
    (one copy of the library's state: options, timing, last error) and
    exposes the decode and write calls."""
    import os
    ext = nat.ext()
    for name in ("paged", "varlen", "dense", "kv_write"):
        assert callable(getattr(ext, name)), name
    assert os.path.dirname(os.path.abspath(ext.__file__)) == os.path.dirname(nat.LIB_PATH)
    maps = open("/proc/self/maps").read()
    assert maps.count(os.path.realpath(nat.LIB_PATH)) >= 1
    loaded = {line.split()[-1] for line in maps.splitlines() if line.endswith("libfsk_decode.so")}
    assert loaded == {os.path.realpath(nat.LIB_PATH)}
    # an option set through ctypes is seen by calls made through the binding
    nat.set_option("chunk_tokens", 33 * 32)
    try:
        assert nat.load().fsk_workspace_bytes(1, 1, 8, 8, 128, 1 << 16, 16, 0) == \
            nat.load().fsk_workspace_bytes(1, 1, 8, 8, 128, 1 << 16, 16, 33 * 32)
    finally:
        nat.set_option("chunk_tokens", 0)


def test_workspace_bytes_with_a_chunk_cap(lib):
    """A negative chunk_tokens caps the automatic split's chunk size (the
    dense split-count hint): finer splits need at least the automatic
    split's workspace; the cap must be a multiple of 32."""
    for layout, extent in ((nat.FSK_LAYOUT_PAGED, 2048), (nat.FSK_LAYOUT_DENSE, 32768), (nat.FSK_LAYOUT_VARLEN, 131072)):
        auto = lib.fsk_workspace_bytes(layout, 4, 32, 8, 128, extent, 16, 0)
        for cap in (-32, -96, -512, -4096, -8192):
            assert lib.fsk_workspace_bytes(layout, 4, 32, 8, 128, extent, 16, cap) >= auto > 0, (layout, cap)
        assert lib.fsk_workspace_bytes(layout, 4, 32, 8, 128, extent, 16, -48) == nat.FSK_ERR_INVALID


def header_param_count(name):
    """Number of parameters of ``name``'s prototype in the header."""
    text = open(HEADER).read()
    m = re.search(r"FSK_API\s+[\w\s\*]+?\b" + name + r"\s*\((.*?)\);", text, flags=re.S)
    assert m, name
    return len([p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"])


def test_reference_side_binding_signature(lib):
    """The ctypes-only binding a reference maintainer would add
    (fasterkernels_amd/reference_binding.py) declares fsk_decode_varlen and
    fsk_workspace_bytes exactly as the package's own binding and the header
    do, and loads the library without a GPU."""
    from fasterkernels_amd import reference_binding as rb
    assert rb.VARLEN_ARGTYPES == nat.SIGNATURES["fsk_decode_varlen"][1]
    assert len(rb.VARLEN_ARGTYPES) == header_param_count("fsk_decode_varlen")
    assert rb.WORKSPACE_ARGTYPES == nat.SIGNATURES["fsk_workspace_bytes"][1]
    assert len(rb.WORKSPACE_ARGTYPES) == header_param_count("fsk_workspace_bytes")
    assert rb.FSK_SINK_LINEAR == nat.FSK_SINK_LINEAR and rb.FSK_LAYOUT_VARLEN == nat.FSK_LAYOUT_VARLEN
    rlib = rb.load(nat.LIB_PATH)
    assert rlib.fsk_decode_varlen.argtypes == rb.VARLEN_ARGTYPES
    assert rlib.fsk_workspace_bytes(0, 4, 32, 8, 128, 4096, 16, 0) == lib.fsk_workspace_bytes(0, 4, 32, 8, 128, 4096,
                                                                                            16, 0) > 0
    q = torch.zeros(2, 32, 128, dtype=torch.float16)
    k = torch.zeros(4, 8, 128, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="must be a CUDA"):
        rb.flash_decode_gqa_varlen(q, k, k, torch.tensor([0, 1, 2], dtype=torch.int32))


def test_every_signature_matches_the_header_arity():
    """Each ctypes signature has as many parameters as its prototype."""
    for name, (_, args) in nat.SIGNATURES.items():
        assert len(args) == header_param_count(name), name
