// fsk_decode.hip -- split-KV GQA flash decoding for MI355X (gfx950).
//
// Two kernels per decode call:
//   1. partial_kernel: a persistent grid of one-wave workgroups walks a device
//      work list of (sequence chunk, kv head) units (varlen at head_dim 64:
//      a pair of neighbouring kv heads read as one 128-wide row).  Each unit streams its
//      chunk of K/V in 32-token tiles with 128-bit buffer loads, computes
//      S^T = K Q^T and O^T += V^T P^T on the matrix cores
//      (v_mfma_f32_16x16x32_{f16,bf16}), keeps the online-softmax state in the
//      MFMA accumulator layout, and writes an fp32 partial (m, l, acc[D]) per
//      query head.  The work list is built by every workgroup from the
//      sequence lengths (a wave prefix scan into LDS), so the host never reads
//      lengths back and the grid size only depends on host-known bounds.
//      When the caller holds the lengths in host memory (the *_host entry
//      points), the host builds the same work list and passes it in the
//      kernel arguments instead (HostPlan).
//   2. reduce_kernel: one 256-thread workgroup per (sequence, query head) combines the
//      partials with a log-sum-exp merge, folds the attention sink and writes
//      the output in the requested dtype.
//
// The maths follows the reference kernels: scores s = q.k * sm_scale,
// online softmax, P rounded to the KV compute type before P.V
// (fskernels/triton/triton_gqa_decode.py:86-109), split partials combined as
// in fskernels/triton/triton_gqa_decode_hf.py:103-137.  bf16 P is carried as a
// hi+lo pair of bf16 values so that the P.V product keeps fp32-level accuracy.
// Scores are kept in the log2 domain (scale folded with log2 e), so every
// exponential is a single v_exp_f32.

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>
#include <math.h>
#include <algorithm>
#include <cmath>
#include <string.h>
#include <mutex>
#include <string>
#include <vector>

#include "fsk_decode.h"

// Device scratch of the allocation-free entry point fsk_decode_paged_noalloc:
// the decode workspace (plan, partial maxima/sums, partial outputs) lives in
// this file-scope array instead of caller- or library-allocated memory.  The
// array belongs to the library's code object, so every device on which the
// code object is loaded (any kernel of the library launched there) holds its
// own copy of FSK_NOALLOC_SCRATCH_BYTES until the process ends.  In host code
// the name is only a host-side stand-in: the device address comes from
// hipGetSymbolAddress, once per device (see noalloc_scratch).
static __device__ __align__(256) uint8_t scratch[FSK_NOALLOC_SCRATCH_BYTES];

// Per-wave timeline of the partial kernel, in builds with FSK_WAVE_STAMPS
// only (libfsk_decode_stamps.so; the normal library has none of this): lane
// 0 of workgroup w < kStampWaves stores s_memrealtime (100 MHz) at its start
// [0], when its plan is built [1], when the first tile of its first item is in
// registers [2], after its last item's epilogue [3] and at its exit [4], plus
// the number of segments it processed [5], its XCC_ID [6] and its HW_ID [7]
// (wave slot, SIMD, CU, shader array and engine), and for its first item
// (paged units) when the page window and Q loads are issued [8] and when
// they have arrived [9]; inside the plan, when the lengths are summed [10]
// and when the split (with its lead-in decision) is chosen [11].  Vector
// stores, read back by fsk_debug_wave_stamps.
#ifdef FSK_WAVE_STAMPS
constexpr int kStampWaves = 4096;
constexpr int kStampSlots = 16;
__device__ unsigned long long g_wave_stamps[kStampWaves * kStampSlots];
#define FSK_STAMP_AT(slot, value)                                                         \
  do {                                                                                     \
    if (threadIdx.x == 0 && blockIdx.x < kStampWaves) g_wave_stamps[blockIdx.x * kStampSlots + (slot)] = (value); \
  } while (0)
#define FSK_STAMP(slot) FSK_STAMP_AT(slot, __builtin_amdgcn_s_memrealtime())
#else
#define FSK_STAMP_AT(slot, value) do { } while (0)
#define FSK_STAMP(slot) do { } while (0)
#endif

namespace {

// ---------------------------------------------------------------------------
// Types and small helpers
// ---------------------------------------------------------------------------
typedef _Float16 f16;
typedef __bf16 bf16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
// Raw buffer resource dword 3 for gfx9-family parts (format fields unused by
// raw dword loads).
constexpr int kRsrcWord3 = 0x00020000;
constexpr float E4M3_MAX_F = 448.f;  // largest finite e4m3fn value

enum Layout { kVarlen = 0, kPaged = 1, kDense = 2 };
enum Kind { kF16 = FSK_F16, kBF16 = FSK_BF16, kF32 = FSK_F32, kE4M3 = FSK_E4M3 };

__device__ __forceinline__ uint32_t f2u(float x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ float u2f(uint32_t x) { return __builtin_bit_cast(float, x); }

// Max / sum over the four lanes {l, l^16, l^32, l^48} (the four k-groups of an
// MFMA operand) with the gfx950 permlane swaps; every lane gets the result.
__device__ __forceinline__ float group4_max(float x) {
  auto a = __builtin_amdgcn_permlane32_swap(f2u(x), f2u(x), false, false);
  x = fmaxf(u2f(a[0]), u2f(a[1]));
  auto b = __builtin_amdgcn_permlane16_swap(f2u(x), f2u(x), false, false);
  return fmaxf(u2f(b[0]), u2f(b[1]));
}
__device__ __forceinline__ float group4_sum(float x) {
  auto a = __builtin_amdgcn_permlane32_swap(f2u(x), f2u(x), false, false);
  x = u2f(a[0]) + u2f(a[1]);
  auto b = __builtin_amdgcn_permlane16_swap(f2u(x), f2u(x), false, false);
  return u2f(b[0]) + u2f(b[1]);
}

// Inclusive prefix sum over the 64 lanes with DPP: row_shr 1, 2, 4, 8 scan
// each row of 16 lanes, then row_bcast:15 adds row 0's total to row 1 and
// row 2's to row 3, and row_bcast:31 adds the total of rows 0-1 to rows 2-3
// (lanes a DPP step does not write keep `old` = 0).
__device__ __forceinline__ int wave_incl_sum(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15 -> rows 1, 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31 -> rows 2, 3
  return x;
}

// e4m3fn -> f16 / bf16, two codes per call (bytes 0,1 or 2,3 of `w`).  Both
// conversions are exact: every e4m3 value is representable in f16 and bf16.
template <bool kToBf16, bool kHi>
__device__ __forceinline__ uint32_t e4m3x2_to(uint32_t w) {
  if constexpr (kToBf16) {
    bf16x2 h = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, kHi);
    return __builtin_bit_cast(uint32_t, h);
  } else {
    f16x2 h = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, kHi);
    return __builtin_bit_cast(uint32_t, h);
  }
}
// Four e4m3 codes in one dword -> four 16-bit values in two dwords.
template <bool kToBf16>
__device__ __forceinline__ u32x2 e4m3x4_to(uint32_t w) {
  return u32x2{e4m3x2_to<kToBf16, false>(w), e4m3x2_to<kToBf16, true>(w)};
}

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  f16x2 h = {(f16)a, (f16)b};
  return __builtin_bit_cast(uint32_t, h);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2 h = {(bf16)a, (bf16)b};
  return __builtin_bit_cast(uint32_t, h);
}
__device__ __forceinline__ float bf16_lo_to_f32(uint32_t w) { return u2f(w << 16); }
__device__ __forceinline__ float bf16_hi_to_f32(uint32_t w) { return u2f(w & 0xffff0000u); }

template <bool kBf16>
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (kBf16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, kRsrcWord3);
}

// Cache policy of the K/V stream: every K/V byte is read exactly once per
// call, so the loads are marked non-temporal (the gfx950 "nt" bit).
#ifndef FSK_KV_CACHE_POLICY
#define FSK_KV_CACHE_POLICY 2
#endif
constexpr int kKvAux = FSK_KV_CACHE_POLICY;

// Load `kBytes` (4, 8, 16 or 32) from a buffer resource; bytes past the
// resource's range read as zero.
template <int kBytes>
struct Chunk {
  uint32_t w[kBytes / 4];
};
template <int kBytes, int kAux = 0>
__device__ __forceinline__ Chunk<kBytes> buf_load(__amdgpu_buffer_rsrc_t r, int off) {
  Chunk<kBytes> c;
  if constexpr (kBytes == 4) {
    c.w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kAux);
  } else if constexpr (kBytes == 8) {
    u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kAux);
    c.w[0] = x[0]; c.w[1] = x[1];
  } else {
#pragma unroll
    for (int i = 0; i < kBytes / 16; ++i) {
      u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16 * i, 0, kAux);
      c.w[4 * i + 0] = x[0]; c.w[4 * i + 1] = x[1]; c.w[4 * i + 2] = x[2]; c.w[4 * i + 3] = x[3];
    }
  }
  return c;
}

__device__ __forceinline__ int clampi(int x, int lo, int hi) { return x < lo ? lo : (x > hi ? hi : x); }
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Division by a divisor fixed per call, as a multiply and shift: m and s
// from make_fastdiv on the host, exact for dividends below 2^31.
struct FastDiv {
  uint32_t d, m, s;
};
__host__ __device__ __forceinline__ uint32_t fdiv(uint32_t x, FastDiv f) {
  return (uint32_t)(((uint64_t)x * f.m) >> f.s);
}

// The split policy's constants for one call (make_split_args on the host;
// split_geometry states the policy).  Streams are below 2^31 tokens, so the
// products with target_units saturate there.
struct SplitArgs {
  uint32_t chunk_min, chunk_max;  // split size bounds in tokens (multiples of the padding)
  uint32_t pref_total;            // min(target_units * chunk_pref, 2^31)
  uint32_t max_total;             // min(target_units * chunk_max, 2^31)
  uint32_t short_units;           // min(32 B, 2^32 - 1): most chunks of a short stream's split
  uint32_t cap;                   // u_max - B - 1 (0: no room): most chunks any split may have
  FastDiv target;                 // divisor target_units (<= 2^20): preferred number of chunks
  FastDiv target_half;            // divisor max(target_units / 2, 1)
  FastDiv cap_div;                // divisor max(cap, 1)
  uint32_t k_cap;                 // doublings that take target_units to 2^24
  uint32_t xcd_skew;              // percent (<= 50), 0: equal chunks
  uint32_t nh7;                   // head slots per chunk, mod 8
};

// ---------------------------------------------------------------------------
// Kernel parameters (passed by value)
// ---------------------------------------------------------------------------
struct Params {
  const uint8_t* q;        // query rows
  int64_t q_sb, q_sh;      // bytes
  const uint8_t* k;
  const uint8_t* v;
  int64_t k_s0, k_sh, k_st;  // bytes; s0 = page stride (paged) / batch stride (dense)
  int64_t v_s0, v_sh, v_st;
  const int32_t* lens;     // varlen: cu_seqlens[B+1]; paged: seq_lens[B]; dense: cache_lens[B]
  const int32_t* starts;   // dense: start offsets or null
  const int32_t* block_table;
  int64_t bt_sb;           // elements
  int max_blocks, num_pages, page_size;
  FastDiv page;            // divisor page_size (paged token -> page)
  int kv_extent;           // varlen: total rows; dense: S_max
  const float* q_scale;
  const float* k_scale;
  const float* v_scale;
  float score_scale;       // sm_scale * log2(e)
  int B, Hkv, G, n_hb;
  int n_items_h;           // head slots per chunk: Hkv * n_hb, or Hkv / 2 with pair
  FastDiv nh_div;          // divisor n_items_h
  FastDiv hb_div;          // divisor n_hb
  FastDiv hkv_div;         // divisor Hkv
  int pair;                // varlen, head_dim 64: a wave takes KV heads 2i and 2i+1 as one 128-wide row
  SplitArgs split;          // the split policy's constants
  int u_max;               // workspace capacity in units
  int seg_tokens;          // stream tokens laid before each non-empty sequence (a multiple of 32)
  int32_t* plan;           // [B+1] unit prefix offsets
  float* part_ml;          // [u_max, Hkv, G, 2]
  float* part_acc;         // [u_max, Hkv, G, D]
  // Block scores (kScores kernels only): raw log2-domain maximum of each
  // 128-token block [B, Hq, nblk] and the sequence lengths [B] for the reduce.
  float* blk_max;
  int32_t* lens_out;
  int nblk;
};

// A plan built on the host (the host-plan entry points, for callers that
// hold the sequence lengths in host memory): the split and each sequence's
// tables, exactly as build_plan computes them on the device, passed in the
// kernel arguments.  Entries past B hold flat[B] and pre[B].
constexpr int kHostPlanMax = FSK_HOST_PLAN_MAX_BATCH;  // most sequences of a host-planned call
struct HostPlan {
  int32_t c_e, c_o, n, paired;
  uint32_t m;
  int32_t seg_x;
  int32_t pre_end;              // pre[B]: the call's partials
  int32_t len[kHostPlanMax];    // sequence lengths (clamped as seq_range does)
  int32_t start[kHostPlanMax];  // first row of each sequence (varlen, dense)
  int32_t flat[kHostPlanMax];   // stream offset of each sequence's region
  int32_t pre[kHostPlanMax];    // first partial of each sequence
};

// Token range [start, start+len) of sequence b in its layout's row space.
template <int kLayout>
__device__ __forceinline__ void seq_range(const Params& p, int b, int& start, int& len) {
  if constexpr (kLayout == kVarlen) {
    int s = clampi(p.lens[b], 0, p.kv_extent);
    int e = clampi(p.lens[b + 1], s, p.kv_extent);
    start = s;
    len = e - s;
  } else if constexpr (kLayout == kPaged) {
    start = 0;
    len = clampi(p.lens[b], 0, p.max_blocks * p.page_size);
  } else {
    int e = clampi(p.lens[b], 0, p.kv_extent);
    int s = p.starts ? clampi(p.starts[b], 0, e) : 0;
    start = s;
    len = e - s;
  }
}

// Base addresses of rows [t, t+16) (sequence-local token t, a multiple of 16)
// of kv head `kvh`, and how many of those rows are valid.  This is the single
// page-addressing routine of the library: the decode kernels and the
// fsk_paged_gather debug entry point both go through it.
struct HalfTile {
  const uint8_t* k;
  const uint8_t* v;
  int rows;
};
template <int kLayout>
__device__ __forceinline__ HalfTile half_tile(const Params& p, int b, int start, int len, int kvh,
                                              int t) {
  HalfTile h;
  h.rows = clampi(len - t, 0, 16);
  if constexpr (kLayout == kVarlen) {
    int64_t row = (int64_t)start + t;
    if (h.rows == 0) row = 0;
    h.k = p.k + row * p.k_st + kvh * p.k_sh;
    h.v = p.v + row * p.v_st + kvh * p.v_sh;
  } else if constexpr (kLayout == kPaged) {
    int page = 0, off = 0;
    if (h.rows > 0) {
      int lp = t / p.page_size;
      off = t - lp * p.page_size;
      page = clampi(p.block_table[(int64_t)b * p.bt_sb + lp], 0, p.num_pages - 1);
    }
    h.k = p.k + (int64_t)page * p.k_s0 + kvh * p.k_sh + off * p.k_st;
    h.v = p.v + (int64_t)page * p.v_s0 + kvh * p.v_sh + off * p.v_st;
  } else {
    int64_t row = (int64_t)start + t;
    if (h.rows == 0) row = 0;
    h.k = p.k + (int64_t)b * p.k_s0 + kvh * p.k_sh + row * p.k_st;
    h.v = p.v + (int64_t)b * p.v_s0 + kvh * p.v_sh + row * p.v_st;
  }
  return h;
}

// Work plan.  The sequences' tokens are laid end to end, each sequence padded
// to a multiple of kAlign (32 tokens, 128 with block scores), and the stream
// is cut into equal chunks: work item (chunk j, head block) processes
// stream positions [j*c, (j+1)*c) of one KV head.  A chunk that crosses
// sequence boundaries is processed as one segment per sequence, and every
// segment with valid tokens produces one fp32 partial, so all work items
// carry the same number of tokens whatever the length distribution.  Each
// non-empty sequence is preceded in the stream by seg_tokens positions that
// hold no tokens: a segment start costs its wave a few memory round trips
// (partial store, page window and Q, first tiles), and an item that crosses
// a sequence boundary carries that many fewer tokens in exchange.
//
// The chunk c is the larger of
//   * stream / target (target = target_units, doubled once if the chunk
//     would exceed chunk_pref, then while it would exceed chunk_max: enough
//     equal chunks to fill the GPU evenly), and
//   * stream / (u_max - B - 1) (so every partial fits the workspace: a batch
//     has at most n_chunks + B partials),
// rounded to kAlign and clamped to [chunk_min, chunk_max]; the host sizes
// u_max for chunk_max.  In LDS: flat[b] = stream offset of sequence b's
// region (its first token sits seg_tokens later; flat[B] = stream length),
// pre[b] = first partial of sequence b (pre[B] =
// total); lane b also returns its own entries flat[b] and pre[b] (the work
// loop reads them from registers when B <= 64).  Workgroup 0 publishes pre
// for the reduce kernel.  Every workgroup computes the same plan from the
// same lengths (split_geometry has the exact rule, with a short-stream case).
// build_plan returns the split.
// Chunk geometry.  The stream is cut into pairs of a long chunk (c_e tokens)
// and a short one (c_o); c_e == c_o without an XCD skew.  Chunk j starts at
// (j / 2) * (c_e + c_o) + (j odd ? c_e : 0).
struct Split {
  int c_e, c_o, pair;  // pair = c_e + c_o = twice the split's base chunk
  int n;               // chunks in the call
  int paired;          // items map even chunks to even XCDs (see item_of)
  uint32_t m;          // ceil(2^32 / (pair / 2)): see div_m
};
// floor(x / d) for x < 2^31 from m = ceil(2^32 / d): the high word of x m
// exceeds x / d by less than x / 2^32 < 1/2, so it is floor(x / d) or one
// more, and one multiply-compare settles which.  (A long division is ~20
// dependent instructions; this is four.)
__host__ __device__ __forceinline__ uint32_t div_m(uint32_t x, uint32_t d, uint32_t m) {
  const uint32_t q = (uint32_t)(((uint64_t)x * m) >> 32);
  return q - (q * d > x ? 1u : 0u);
}
__host__ __device__ __forceinline__ int chunk_of(const Split& sp, int x) {  // x >= 0
  const uint32_t half = (uint32_t)sp.pair >> 1;
  const int q = (int)(div_m((uint32_t)x, half, sp.m) >> 1);  // floor(x / pair)
  return 2 * q + (x - q * sp.pair >= sp.c_e ? 1 : 0);
}
__host__ __device__ __forceinline__ int chunk_lo(const Split& sp, int j) { return (j >> 1) * sp.pair + (j & 1) * sp.c_e; }
// (arithmetic, not a select: the compiler turns the select into a two-entry
// table in scratch memory, whose loads are not known to be wave-uniform)
__host__ __device__ __forceinline__ int chunk_len(const Split& sp, int j) { return sp.c_e + (j & 1) * (sp.c_o - sp.c_e); }

// Work item w -> (chunk, head slot).  Workgroups are dealt to the 8 XCDs
// round-robin (XCD = w mod 8 for the items of the first round), and on this
// part the odd XCDs stream the same work 6-20 % slower than the even ones;
// with a skew the long (even) chunks go to the even XCDs: item w = 8 m + x
// takes pair index P = 4 m + x / 2 of its parity class, chunk 2 (P / NH) +
// (x & 1), head slot P mod NH.  (A bijection when n is even and n NH is a
// multiple of 8, which the plan ensures before setting `paired`.)  nh
// divides by NH; w < 2^31 (the host bounds the item count), so 32-bit
// arithmetic and the multiply-shift division are exact.
__host__ __device__ __forceinline__ void item_of(const Split& sp, uint32_t w, FastDiv nh, int& jc, int& hh) {
  if (sp.paired) {
    const uint32_t x = w & 7;
    const uint32_t P = (w >> 3) * 4 + (x >> 1);
    const uint32_t q = fdiv(P, nh);
    jc = (int)(2 * q + (x & 1));
    hh = (int)(P - q * nh.d);
  } else {
    const uint32_t q = fdiv(w, nh);
    jc = (int)q;
    hh = (int)(w - q * nh.d);
  }
}

constexpr int kSkewMinChunk = 512;  // smallest split that gets the XCD skew (tokens)
constexpr int kShortChunk = 64;     // smallest automatic split of a short stream (tokens)

// The scalar part of the plan: the chunk geometry of a stream of `total`
// padded tokens (align = the padding, 32 or 128).  Compiled for the host too,
// so that the split can be checked without a GPU (fsk_debug_split).
// ceil(x / d) for x < 2^31 (x = 0 included, without a branch).
__host__ __device__ __forceinline__ uint32_t cdiv_fast(uint32_t x, FastDiv d) {
  const uint32_t nz = x != 0 ? 1u : 0u;
  return (fdiv(x - nz, d) + 1) * nz;
}
// ceil(x / (d 2^k)) = ceil(ceil(x / 2^k) / d), for x < 2^31 and k <= 25.
__host__ __device__ __forceinline__ uint32_t cdiv_shift(uint32_t x, uint32_t k, FastDiv d) {
  return cdiv_fast((x + (1u << k) - 1) >> k, d);
}
__host__ __device__ __forceinline__ uint32_t clz32(uint32_t x) { return (uint32_t)__builtin_clz(x); }  // x > 0
__host__ __device__ __forceinline__ uint32_t umulhi32(uint32_t x, uint32_t y) {
  return (uint32_t)(((uint64_t)x * y) >> 32);
}
// Every workgroup runs this on its critical path before its first K/V load,
// where each dependent instruction costs a few cycles: it is branch-free
// scalar arithmetic (so that two calls interleave, see build_plan), the
// divisors are the host's multiply-shift pairs, the comparisons with
// ceil(x / c) are products (ceil(x / c) > t exactly when x > t c), and one
// division gives the chunk's reciprocal, which the chunk count, the skewed
// pairs and chunk_of share.
__host__ __device__ __forceinline__ Split split_geometry(uint32_t total, const SplitArgs& a, uint32_t align) {
  auto umax = [](uint32_t x, uint32_t y) { return x > y ? x : y; };
  auto umin = [](uint32_t x, uint32_t y) { return x < y ? x : y; };
  auto up = [&](uint32_t x) { return (x + align - 1) & ~(align - 1); };  // align: a power of two
  // Chunks per call: target = target_units << k, doubled once if the chunks
  // would exceed chunk_pref, then while they would exceed chunk_max, up to
  // 2^24 chunks (a batch too long for target_units chunks gets twice as many
  // rather than a count that leaves some CUs one item short).  k1: the
  // fewest doublings with target chunk_max >= total.
  const uint32_t P = a.max_total;
  const uint32_t d = P < total ? clz32(P) - clz32(total) : 0u;  // P << d has total's top bit
  const uint32_t k1 = P < total ? d + ((P << d) < total ? 1u : 0u) : 0u;
  const uint32_t k = umax(a.pref_total < total ? 1u : 0u, umin(k1, a.k_cap));
  uint32_t want = cdiv_shift(total, k, a.target);  // ceil(total / target)
  // A short stream (target chunks would be below chunk_min): half as many
  // chunks, of kShortChunk to chunk_min tokens.  Items of 2-3 tiles finished
  // sooner than both 4-tile items (fewer waves, twice the round trips each)
  // and 1-tile items (per-item costs).  Only while that keeps to 32 chunks
  // per sequence on average: the reduce merges 32 partials of a sequence per
  // memory round trip (head_dim 128).
  const uint32_t lo2 = up((uint32_t)kShortChunk), hi2 = umax(a.chunk_min, lo2);
  const uint32_t w2 = cdiv_shift(total, k > 0 ? k - 1 : 0u, k > 0 ? a.target : a.target_half);  // ceil(total / max(target / 2, 1))
  const uint32_t c2 = umin(umax(up(w2), lo2), hi2);
  const bool fits = umulhi32(a.short_units, c2) != 0 || total <= a.short_units * c2;  // ceil(total / c2) <= 32 B
  const bool take = want < a.chunk_min && a.chunk_min < a.chunk_max && fits;
  want = take ? w2 : want;
  uint32_t chunk = umin(umax(up(want), take ? lo2 : a.chunk_min), take ? hi2 : a.chunk_max);
  // at most `cap` chunks: every partial must fit the workspace
  const uint32_t c_cap = up(cdiv_fast(total, a.cap_div));  // up(ceil(total / cap))
  chunk = a.cap == 0 ? a.chunk_max : umin(umax(chunk, c_cap), a.chunk_max);
  Split sp;
  sp.m = 0xFFFFFFFFu / chunk + 1;  // ceil(2^32 / chunk): chunk >= 32
  const uint32_t whole = div_m(total, chunk, sp.m);  // floor(total / chunk)
  const uint32_t n_eq = whole + (whole * chunk != total ? 1u : 0u);
  // XCD skew: long chunks (1 + skew %) for the even XCDs, short ones for the
  // odd, in pairs of 2 chunk tokens (short splits are latency-bound: there
  // the longer chunks cost more).  The count is even (a trailing chunk past
  // the stream has no tokens) and the items map onto the XCDs (n NH a
  // multiple of 8).
  const uint32_t ce = umin(up(chunk * (100 + a.xcd_skew) / 100), a.chunk_max);
  const uint32_t co = 2 * chunk - ce;
  const uint32_t q = whole >> 1, r = total - q * 2 * chunk;
  uint32_t n_sk = 2 * q + (r > 0 ? 1u : 0u) + (r > ce ? 1u : 0u);
  n_sk += n_sk & 1;
  const bool skew = a.xcd_skew > 0 && chunk >= (uint32_t)kSkewMinChunk && total > 0 && co >= align && co < ce &&
                    n_sk <= a.cap && (((n_sk & 7) * a.nh7) & 7) == 0;
  sp.c_e = (int)(skew ? ce : chunk);
  sp.c_o = (int)(skew ? co : chunk);
  sp.n = (int)(skew ? n_sk : n_eq);
  sp.paired = skew ? 1 : 0;
  sp.pair = sp.c_e + sp.c_o;
  return sp;
}

// seq_range of sequence `lane` (0 for lanes at or past B) with its loads
// issued unconditionally (index clamped to B - 1; B >= 1), so that they go
// out before the kernel arguments they are clamped with have arrived.
template <int kLayout>
__device__ __forceinline__ void seq_range_first(const Params& p, int lane, int& start, int& len) {
  const int b = min(lane, p.B - 1);
  const int l0 = p.lens[b];
  const int l1 = kLayout == kVarlen ? p.lens[b + 1] : 0;
  const int s0 = (kLayout == kDense && p.starts) ? p.starts[b] : 0;
  if constexpr (kLayout == kVarlen) {
    start = clampi(l0, 0, p.kv_extent);
    len = clampi(l1, start, p.kv_extent) - start;
  } else if constexpr (kLayout == kPaged) {
    start = 0;
    len = clampi(l0, 0, p.max_blocks * p.page_size);
  } else {
    const int e = clampi(l0, 0, p.kv_extent);
    start = p.starts ? clampi(s0, 0, e) : 0;
    len = e - start;
  }
  if (lane >= p.B) start = len = 0;
}

// len0: length of sequence `lane` (0 past B), from seq_range_first, whose
// loads the caller issues first.
template <int kLayout, bool kScores>
__device__ __forceinline__ Split build_plan(const Params& p, int32_t* pre, int32_t* flat, const int len0,
                                            int& seg_out, int& flat0_out, int& pre0_out) {
  constexpr int kAlign = kScores ? 128 : 32;
  const int lane = threadIdx.x;
  // Lengths of sequences lane, lane + 64, ...; the first block stays in a
  // register so that the common case (B <= 64) reads them once (and the
  // work loop reads them from these registers, not from memory).
  // The lengths of sequences 64 and up go to the pre[] table first (which
  // the unit prefix overwrites below, each entry after its own lane has read
  // it), four blocks of 64 per memory round trip rather than one.
  for (int b0 = kWave; b0 < p.B; b0 += 4 * kWave) {
    int l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int s;
      seq_range_first<kLayout>(p, b0 + i * kWave + lane, s, l[i]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (b0 + i * kWave + lane < p.B) pre[b0 + i * kWave + lane] = l[i];
  }
  auto length = [&](int b0, int b) { return b0 == 0 ? len0 : b < p.B ? pre[b] : 0; };
  // Stream length (the host bounds it below 2^31 - 4096, so the split
  // arithmetic is unsigned 32-bit: the plan sits on every workgroup's
  // critical path, and 64-bit division is a long software sequence).
  uint32_t total = 0;
  int nonempty = 0;   // sequences with tokens
  int ref = -1;       // the first such sequence's length
  bool varied = false;  // non-empty lengths differ
  for (int b0 = 0; b0 < p.B; b0 += kWave) {
    const int l = length(b0, b0 + lane);
    const int padded = (l + kAlign - 1) / kAlign * kAlign;
    total += (uint32_t)__builtin_amdgcn_readlane(wave_incl_sum(padded), kWave - 1);
    const uint64_t has = __ballot(l > 0);
    nonempty += __builtin_popcountll(has);
    if (ref < 0 && has) ref = __builtin_amdgcn_readlane(l, __builtin_ctzll(has));
    varied = varied || __ballot(l > 0 && l != ref) != 0;
  }
  total = (uint32_t)uniform((int)total);
  nonempty = uniform(nonempty);
  FSK_STAMP(10);
  // Lead-ins where sequence boundaries are common and fall anywhere: lengths
  // that differ, at most 8 chunks per sequence.  Then many items hold a
  // boundary, and the lead-ins balance them.  Equal lengths (whose chunks
  // can line up with the sequences) and a few long sequences keep the plain
  // split, where lead-ins measured slower.  Short chunks (no longer than the
  // lead-in) take lead-ins too, whatever the chunk count: a lead-in of at
  // least a chunk keeps every item to one sequence's tokens, so no short
  // item pays a second segment's round trips.  The test is made on the split
  // with lead-ins, so that a call that takes them computes one split (each
  // costs ~0.4 us of a workgroup's start).
  int X = 0;
  Split sp;
  const uint32_t seg = (uint32_t)p.seg_tokens;
  if (!kScores && seg > 0 && varied) {
    sp = split_geometry(total + (uint32_t)nonempty * seg, p.split, kAlign);
    if (sp.n <= 8 * nonempty || (uint32_t)sp.c_e <= seg) X = (int)seg;
    else sp = split_geometry(total, p.split, kAlign);
  } else {
    sp = split_geometry(total, p.split, kAlign);
  }
  FSK_STAMP(11);
  seg_out = X;
  sp.c_e = uniform(sp.c_e);
  sp.c_o = uniform(sp.c_o);
  sp.pair = sp.c_e + sp.c_o;
  sp.n = uniform(sp.n);
  sp.paired = uniform(sp.paired);
  sp.m = (uint32_t)uniform((int)sp.m);

  int carry_f = 0, carry_u = 0;
  for (int b0 = 0; b0 < p.B; b0 += kWave) {
    const int b = b0 + lane;
    const int len = length(b0, b);
    const int padded = (len + kAlign - 1) / kAlign * kAlign + (len > 0 ? X : 0);
    const int incl_f = wave_incl_sum(padded);
    const int fb = carry_f + incl_f - padded;
    const int fs = fb + X;  // the sequence's first token in the stream
    const int n = len > 0 ? chunk_of(sp, fs + len - 1) - chunk_of(sp, fs) + 1 : 0;
    const int incl_u = wave_incl_sum(n);
    const int pb = min(carry_u + incl_u - n, p.u_max);  // the cap never binds with the host's u_max
    if (b < p.B) {
      flat[b] = fb;
      pre[b] = pb;
    }
    if (b0 == 0) {  // lane b's entries (lanes past B hold flat[B] and pre[B])
      flat0_out = fb;
      pre0_out = pb;
    }
    if constexpr (kScores)
      if (blockIdx.x == 0 && b < p.B) p.lens_out[b] = len;
    carry_f += __builtin_amdgcn_readlane(incl_f, kWave - 1);
    carry_u += __builtin_amdgcn_readlane(incl_u, kWave - 1);
  }
  if (lane == 0) {
    flat[p.B] = carry_f;
    pre[p.B] = min(carry_u, p.u_max);
  }
  __syncthreads();
  if (blockIdx.x == 0) {
    for (int b = lane; b <= p.B; b += kWave) p.plan[b] = pre[b];
  }
  return sp;
}

// Largest b with pre[b] <= u (u < pre[B]).
__device__ __forceinline__ int find_seq(const int32_t* pre, int B, int u) {
  int lo = 0, hi = B;
  while (hi - lo > 1) {
    int mid = (lo + hi) >> 1;
    if (pre[mid] <= u) lo = mid; else hi = mid;
  }
  return lo;
}

// ---------------------------------------------------------------------------
// Partial kernel
// ---------------------------------------------------------------------------
// Lane l = 16*g + c (g = k-group 0..3, c = column 0..15).
//
// QK (v_mfma_f32_16x16x32, A = K rows, B = Q^T columns): for the 16-token half
// h2 of a tile and k-step i, lane l holds 8 head_dim values of token row c
// (A) and of query head c (B); which 8 is fixed by qk_dim0(i, g) for both
// operands (any consistent split of head_dim over the k-slots gives the same
// dot product).  Output: lane l holds S^T[token 4g+r][head c], r = 0..3.
//
// PV (A = V^T rows, B = P^T columns): k-slot s = 0..7 of k-group g is token
// tau(g, s) = 16*(s/4) + 4g + (s%4) of the tile, which is exactly where the QK
// output left P, so P needs no data movement.  MFMA j (0..D/16-1) treats
// column c as head_dim element (D/16)*c + j; the lane therefore loads the
// D/16 consecutive elements [(D/16)c, (D/16)(c+1)) of each of its 8 token rows
// and transposes them in registers with v_perm_b32.  Output: lane l holds
// O[head c][(D/16)(4g+r) + j].
//
// Each wave software-pipelines its unit: the K/V loads of tile n+1 are in
// flight while tile n is computed.  Paged units read their page ids once, into
// a 256-entry window (four VGPRs, entry i in lane i % 64), so no block-table
// load sits in front of a K/V load.  (256 pages of 16 tokens allow 4096-token
// chunks, so that long batches such as 32 x 8K or 64 x 6K tokens get one work
// item per SIMD, not two: one wave per SIMD streams more evenly.)

// First head_dim element of k-step i for k-group g (the same for Q and K).
template <bool kKvFp8>
__device__ __forceinline__ int qk_dim0(int i, int g) {
  // 16-bit KV: k-step i reads the 16-byte chunk 4i+g of a row.
  // e4m3 KV: one 16-byte chunk (4(i/2)+g) covers k-steps i and i+1.
  return kKvFp8 ? 16 * (4 * (i >> 1) + g) + 8 * (i & 1) : 8 * (4 * i + g);
}

template <int D, int kKV>
struct TileRegs {
  static constexpr bool kFp8 = (kKV == kE4M3);
  static constexpr int kSteps = D / 32;
  static constexpr int kVBytes = (D / 16) * (kFp8 ? 1 : 2);   // V bytes per row per lane
  static constexpr int kVLoads = kVBytes > 16 ? kVBytes / 16 : 1;
  // K rows go through LDS (see issue_tile): 16 rows per half tile.
  static constexpr int kRowBytes = D * (kFp8 ? 1 : 2);
  static constexpr int kChunks = kRowBytes / 16;               // 16-byte chunks per K row
  static constexpr int kHalfBytes = 16 * kRowBytes;
  static constexpr int kDma = kHalfBytes / 1024;               // 16-byte-per-lane DMA loads per half
  static constexpr int kLoads = 2 * kDma + 8 * kVLoads;        // vector memory instructions per tile
  Chunk<kVBytes> v[8];
  int nrow[2];  // valid rows of each 16-token half (wave-uniform)
};

// LDS pointers (address space 3): the K stage is addressed through these so
// that no generic-to-LDS cast is needed.
typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef __attribute__((address_space(3))) const u32x4 lds_u32x4;

// 16-byte-per-lane DMA load into LDS: lane L's 16 bytes from byte voffset of
// the buffer go to LDS offset lds_off + 16 L.  (Kept out of the templates:
// the host pass of hipcc rejects this builtin inside a template.)
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, uint32_t lds_off, int voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_u8*)(uintptr_t)lds_off, 16, voffset, 0, 0, kKvAux);
}

// K rows are staged in LDS with the 16-byte chunks of row R stored in the
// order m ^ swz(R), so that the MFMA-operand reads (16 rows, one chunk each)
// hit 16 different 16-byte bank groups.
template <int kChunks>
__device__ __forceinline__ int k_swizzle(int row) {
  constexpr int kRowsPerCycle = kChunks >= 16 ? 1 : 16 / kChunks;
  constexpr int kMask = (kChunks >= 16 ? 16 : kChunks) - 1;
  return (row / kRowsPerCycle) & kMask;
}

// s_waitcnt immediate (gfx9 encoding) that waits until at most n vector memory
// operations are outstanding and leaves the other counters alone.
constexpr int vm_wait_imm(int n) { return (n & 0xF) | (0x7 << 4) | (0xF << 8) | (((n >> 4) & 3) << 14); }

// Waits for the K stage of a tile whose later tiles (``later`` of them, each
// kLoads instructions) may still be in flight.  The LDS DMA writes are not
// visible to the compiler's memory model, hence the explicit wait and the
// compiler barrier that keeps the LDS reads after it.
template <int kLoads, int kDepth>
__device__ __forceinline__ void wait_k_stage(int later) {
  static_assert(kLoads * (kDepth - 1) < 64, "vmcnt holds at most 63");
  if constexpr (kDepth >= 3) {
    if (later >= 2) __builtin_amdgcn_s_waitcnt(vm_wait_imm(2 * kLoads));
    else if (later == 1) __builtin_amdgcn_s_waitcnt(vm_wait_imm(kLoads));
    else __builtin_amdgcn_s_waitcnt(vm_wait_imm(0));
  } else if constexpr (kDepth == 2) {
    if (later >= 1) __builtin_amdgcn_s_waitcnt(vm_wait_imm(kLoads));
    else __builtin_amdgcn_s_waitcnt(vm_wait_imm(0));
  } else {
    __builtin_amdgcn_s_waitcnt(vm_wait_imm(0));
  }
  asm volatile("" ::: "memory");
}

struct Unit {
  int b, kvh, start, len, t_begin, t_end;
  int p_first;     // paged: first logical page of the unit
  int win0, win1, win2, win3;  // paged: physical page of logical page p_first + lane (+64, +128, +192)
};

template <int kLayout>
__device__ __forceinline__ HalfTile unit_half(const Params& p, const Unit& un, int t) {
  HalfTile h;
  h.rows = uniform(clampi(un.t_end - t, 0, 16));
  if constexpr (kLayout == kPaged) {
    int page = 0, off = 0;
    if (h.rows > 0) {
      const int lp = (int)fdiv((uint32_t)t, p.page);
      off = t - lp * p.page_size;
      const int idx = lp - un.p_first;  // 0 .. 255
      // all four reads and two selects: no branches in the tile issue
      const int w0 = __builtin_amdgcn_readlane(un.win0, idx & 63);
      const int w1 = __builtin_amdgcn_readlane(un.win1, idx & 63);
      const int w2 = __builtin_amdgcn_readlane(un.win2, idx & 63);
      const int w3 = __builtin_amdgcn_readlane(un.win3, idx & 63);
      const int lo = (idx & 64) ? w1 : w0, hi = (idx & 64) ? w3 : w2;
      page = (idx & 128) ? hi : lo;
    }
    h.k = p.k + (int64_t)page * p.k_s0 + un.kvh * p.k_sh + off * p.k_st;
    h.v = p.v + (int64_t)page * p.v_s0 + un.kvh * p.v_sh + off * p.v_st;
  } else {
    HalfTile a = half_tile<kLayout>(p, un.b, un.start, un.len, un.kvh, h.rows > 0 ? t : 0);
    h.k = a.k;
    h.v = a.v;
  }
  return h;
}

// First tile of the unit's tile order.  On the varlen and dense layouts the
// KV heads of a token row are 256-byte neighbours, and the waves of one chunk
// (one per head) would read the same rows at the same moment: KV head h
// starts at tile h * n / Hkv of its unit instead, and wraps round (C2: 84.7
// -> 84.0 µs).  Paged units keep token order (their 4 KB page slabs stream
// well in order; rotated, M0 83.0 -> 83.7 µs and C3 185 -> 188.7 µs), and so
// do block scores (the running block maximum is stored when a block ends).
template <int kLayout, bool kScores>
__device__ __forceinline__ int tile_rotation(int kvh, int n_tiles, FastDiv hkv) {
  if constexpr (kScores || kLayout == kPaged) return 0;
  return (int)fdiv((uint32_t)(kvh * n_tiles), hkv);  // kvh < Hkv, n_tiles <= 128
}

// Token position of the k-th tile of a unit of n tiles starting at t0 with
// rotation rot (0 <= rot < n, or 0); tiles past the unit map to its end (an
// empty tile).
__device__ __forceinline__ int tile_pos(int k, int n, int rot, int t0, int t_end) {
  int j = k + rot;
  j -= j >= n ? n : 0;
  return k < n ? t0 + 32 * j : t_end;
}

// Per-lane byte offsets of a tile's loads and of its K-stage reads.  They
// depend on the lane and the KV row strides only, so a workgroup computes
// them while its length loads are in flight instead of after its plan, on
// the way to its first tile loads (each instruction there costs a few
// cycles of the start-up); the empty asm statements keep the compiler from
// recomputing them later.
template <int D, int kKV>
struct LaneGeo {
  using TR = TileRegs<D, kKV>;
  static constexpr int kReads = TR::kFp8 ? (D / 32 + 1) / 2 : D / 32;  // K chunks a lane reads per half tile
  int dma[TR::kDma];     // K DMA r: row R = r kRowsPerDma + lane / kChunks, chunk (lane % kChunks) ^ swz(R)
  int vrow[4];           // V rows 4g + r, this lane's kVBytes of them
  uint32_t kread[kReads];  // K-stage offset of the chunk of k-step i (e4m3: k-steps 2i, 2i + 1) in row c
};
template <int D, int kKV>
__device__ __forceinline__ LaneGeo<D, kKV> lane_geo(const Params& p, int lane, int g, int c) {
  using TR = TileRegs<D, kKV>;
  using LG = LaneGeo<D, kKV>;
  constexpr int kRowsPerDma = 64 / TR::kChunks;
  const int kst = (int)p.k_st, vst = (int)p.v_st;
  LG lg;
#pragma unroll
  for (int r = 0; r < TR::kDma; ++r) {
    const int R = r * kRowsPerDma + lane / TR::kChunks;
    lg.dma[r] = R * kst + 16 * ((lane % TR::kChunks) ^ k_swizzle<TR::kChunks>(R));
    asm volatile("" : "+v"(lg.dma[r]));
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    lg.vrow[r] = (4 * g + r) * vst + c * TR::kVBytes;
    asm volatile("" : "+v"(lg.vrow[r]));
  }
#pragma unroll
  for (int i = 0; i < LG::kReads; ++i) {
    lg.kread[i] = 16 * (c * TR::kChunks + ((4 * i + g) ^ k_swizzle<TR::kChunks>(c)));
    asm volatile("" : "+v"(lg.kread[i]));
  }
  return lg;
}

template <int D, int kKV, int kLayout>
__device__ __forceinline__ void issue_tile(TileRegs<D, kKV>& T, uint32_t kstage_off, const Params& p,
                                           const Unit& un, int t, const LaneGeo<D, kKV>& lg) {
  using TR = TileRegs<D, kKV>;
  constexpr int kElem = TR::kFp8 ? 1 : 2;
  const int kst = (int)p.k_st, vst = (int)p.v_st;
  // The stage is about to be overwritten: keep earlier LDS reads of it before this point.
  asm volatile("" ::: "memory");
#pragma unroll
  for (int h2 = 0; h2 < 2; ++h2) {
    const HalfTile ht = unit_half<kLayout>(p, un, t + 16 * h2);
    T.nrow[h2] = ht.rows;
    const int kbytes = ht.rows > 0 ? (ht.rows - 1) * kst + D * kElem : 0;
    const int vbytes = ht.rows > 0 ? (ht.rows - 1) * vst + D * kElem : 0;
    const auto rk = make_rsrc(ht.k, kbytes);
    const auto rv = make_rsrc(ht.v, vbytes);
    // K: coalesced 16-byte DMA loads straight into LDS (lane L of load r
    // fetches row R = r * kRowsPerDma + L / kChunks, chunk (L % kChunks) ^
    // swz(R); rows past the valid ones read as zero).
#pragma unroll
    for (int r = 0; r < TR::kDma; ++r) lds_dma16(rk, kstage_off + h2 * TR::kHalfBytes + r * 1024, lg.dma[r]);
#pragma unroll
    for (int r = 0; r < 4; ++r) T.v[4 * h2 + r] = buf_load<TR::kVBytes, kKvAux>(rv, lg.vrow[r]);
  }
}

// 16-byte chunk `chunk` of K row c of half h2 from the LDS stage.
template <int D, int kKV>
__device__ __forceinline__ u32x4 k_chunk(uint32_t kstage_off, int h2, int c, int chunk) {
  using TR = TileRegs<D, kKV>;
  const uint32_t off = kstage_off + h2 * TR::kHalfBytes + 16 * (c * TR::kChunks + (chunk ^ k_swizzle<TR::kChunks>(c)));
  return *(lds_u32x4*)(uintptr_t)off;
}

template <int D, int kQ, int kKV>
struct Softmax {
  static constexpr bool kQkBf16 = (kQ == kBF16);   // QK operand type
  static constexpr bool kPvBf16 = (kKV == kBF16);  // PV operand type (e4m3 V -> f16)
  static constexpr int kSteps = D / 32;
  static constexpr int kDpc = D / 16;
  float m_run, l_run;
  f32x4 acc[kDpc];
};

// Returns the tile's maximum score of head column c (log2 domain, -inf when
// the tile has no valid row).
template <int D, int kQ, int kKV>
__device__ __forceinline__ float compute_tile(const TileRegs<D, kKV>& T, uint32_t kstage,
                                              Softmax<D, kQ, kKV>& st, const u32x4 (&qop)[D / 32], float sscale,
                                              int g, const LaneGeo<D, kKV>& lg) {
  using TR = TileRegs<D, kKV>;
  using SM = Softmax<D, kQ, kKV>;
  constexpr int kSteps = SM::kSteps;
  constexpr int kDpc = SM::kDpc;

  // ---- S^T = K Q^T
  f32x4 s[2];
#pragma unroll
  for (int h2 = 0; h2 < 2; ++h2) {
    s[h2] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kSteps; ++i) {
      u32x4 kop;
      if constexpr (TR::kFp8) {
        // e4m3: chunk 4 (i / 2) + g holds k-steps i and i + 1
        const u32x4 raw = *(lds_u32x4*)(uintptr_t)(kstage + h2 * TR::kHalfBytes + lg.kread[i >> 1]);
        const u32x2 a = e4m3x4_to<SM::kQkBf16>(raw[2 * (i & 1)]);
        const u32x2 bb = e4m3x4_to<SM::kQkBf16>(raw[2 * (i & 1) + 1]);
        kop = u32x4{a[0], a[1], bb[0], bb[1]};
      } else {
        kop = *(lds_u32x4*)(uintptr_t)(kstage + h2 * TR::kHalfBytes + lg.kread[i]);
      }
      s[h2] = mfma16x16x32<SM::kQkBf16>(kop, qop[i], s[h2]);
    }
  }

  // ---- online softmax over this tile (log2 domain)
  float sv[8];
#pragma unroll
  for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float x = s[h2][r] * sscale;
      if (4 * g + r >= T.nrow[h2]) x = -INFINITY;
      sv[4 * h2 + r] = x;
    }
  float mt = sv[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) mt = fmaxf(mt, sv[i]);
  mt = group4_max(mt);
  const float m_new = fmaxf(st.m_run, mt);
  const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
  if (__builtin_amdgcn_ballot_w64(m_new > st.m_run) != 0) {
    const float alpha = __builtin_amdgcn_exp2f(st.m_run - m_use);
    st.l_run *= alpha;
#pragma unroll
    for (int j = 0; j < kDpc; ++j) st.acc[j] *= alpha;
  }
  st.m_run = m_new;
  float pv[8];
  float psum = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    pv[i] = __builtin_amdgcn_exp2f(sv[i] - m_use);
    psum += pv[i];
  }
  st.l_run += psum;

  // ---- P^T operand(s); bf16 P is split into hi + lo parts
  u32x4 pop, plo;
  if constexpr (SM::kPvBf16) {
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      hi[i] = pack_bf16x2(pv[2 * i], pv[2 * i + 1]);
      lo[i] = pack_bf16x2(pv[2 * i] - bf16_lo_to_f32(hi[i]), pv[2 * i + 1] - bf16_hi_to_f32(hi[i]));
    }
    pop = u32x4{hi[0], hi[1], hi[2], hi[3]};
    plo = u32x4{lo[0], lo[1], lo[2], lo[3]};
  } else {
    pop = u32x4{pack_f16x2(pv[0], pv[1]), pack_f16x2(pv[2], pv[3]), pack_f16x2(pv[4], pv[5]),
                pack_f16x2(pv[6], pv[7])};
    (void)plo;
  }

  // ---- V^T operands (16-bit view of each row; e4m3 rows widened to f16)
  constexpr int kVWords = kDpc / 2;
  uint32_t vw[8][kVWords];
#pragma unroll
  for (int sidx = 0; sidx < 8; ++sidx) {
    if constexpr (TR::kFp8) {
#pragma unroll
      for (int e = 0; e < TR::kVBytes / 4; ++e) {
        const u32x2 x = e4m3x4_to<false>(T.v[sidx].w[e]);
        vw[sidx][2 * e] = x[0];
        vw[sidx][2 * e + 1] = x[1];
      }
    } else {
#pragma unroll
      for (int e = 0; e < kVWords; ++e) vw[sidx][e] = T.v[sidx].w[e];
    }
  }
  // ---- O^T += V^T P^T
#pragma unroll
  for (int j = 0; j < kDpc; ++j) {
    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
    u32x4 vop;
#pragma unroll
    for (int m = 0; m < 4; ++m) vop[m] = __builtin_amdgcn_perm(vw[2 * m + 1][j >> 1], vw[2 * m][j >> 1], sel);
    st.acc[j] = mfma16x16x32<SM::kPvBf16>(vop, pop, st.acc[j]);
    if constexpr (SM::kPvBf16) st.acc[j] = mfma16x16x32<true>(vop, plo, st.acc[j]);
  }
  return mt;
}

// Block scores: running maximum of the current 128-token block, stored when
// the block (or the unit) ends.  Units start on block boundaries (the split
// size is a multiple of 128 when scores are requested).
constexpr int kScoreBlock = 128;
struct BlockMax {
  float m = -INFINITY;
  __device__ __forceinline__ void add(const Params& p, const Unit& un, int t, float mt, int head, bool head_ok,
                                      int g) {
    m = fmaxf(m, mt);
    if (((t + 32) % kScoreBlock) == 0 || t + 32 >= un.t_end) {
      const int blk = t / kScoreBlock;
      if (head_ok && g == 0 && blk < p.nblk)
        p.blk_max[((int64_t)un.b * p.Hkv * p.G + un.kvh * p.G + head) * p.nblk + blk] = m;
      m = -INFINITY;
    }
  }
};

// ---------------------------------------------------------------------------
// VALU formulation of a tile: the counterpart of compute_tile without matrix
// cores, kept for A/B measurement (option qk_engine = 1; f16 Q and KV,
// D = 128, at most 4 query heads per KV head, no block scores).  Lane (g, c)
// owns dims [8c, 8c+8) of tokens 4g+r and 16+4g+r (r = 0..3) of the tile:
// the rows and dims its V registers already hold.  Scores: partial q.k over
// its 8 dims with v_dot2_f32_f16, summed over the 16 lanes of its DPP row;
// then the online softmax of each head (the 4 k-groups combined with the
// permlane swaps) and P.V as fp32 FMAs into the lane's 8 dims of each head,
// with P rounded to f16 first as the MFMA path does.  The k-groups' output
// sums are combined once per unit.
// ---------------------------------------------------------------------------
constexpr int kValuHeads = 4;
struct SoftmaxV {
  float m_run[kValuHeads], l_run[kValuHeads];
  float acc[kValuHeads][8];
};

// Sum over the 16 lanes of a DPP row (every lane gets it): quad_perm
// [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror.
__device__ __forceinline__ float row16_sum(float x) {
  x += u2f(__builtin_amdgcn_update_dpp(0, f2u(x), 0xB1, 0xf, 0xf, false));
  x += u2f(__builtin_amdgcn_update_dpp(0, f2u(x), 0x4E, 0xf, 0xf, false));
  x += u2f(__builtin_amdgcn_update_dpp(0, f2u(x), 0x141, 0xf, 0xf, false));
  x += u2f(__builtin_amdgcn_update_dpp(0, f2u(x), 0x140, 0xf, 0xf, false));
  return x;
}

__device__ __forceinline__ f16x2 as_f16x2(uint32_t w) { return __builtin_bit_cast(f16x2, w); }

template <int D>
__device__ __forceinline__ void compute_tile_valu(const TileRegs<D, kF16>& T, uint32_t kstage, SoftmaxV& st,
                                                  const u32x4 (&qv)[kValuHeads], float sscale, int g, int c) {
  static_assert(D == 128, "the VALU tile covers D = 128 (16 lanes x 8 dims)");
  // ---- S = q.k: 8 token slots (i = 4 h2 + r) x 4 heads per lane
  float s[8][kValuHeads];
#pragma unroll
  for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const u32x4 kk = k_chunk<D, kF16>(kstage, h2, 4 * g + r, c);
      uint32_t kw[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) kw[e] = kk[e];
#pragma unroll
      for (int h = 0; h < kValuHeads; ++h) {
        float a = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t qw = qv[h][e];
          a = __builtin_amdgcn_fdot2(as_f16x2(kw[e]), as_f16x2(qw), a, false);
        }
        s[4 * h2 + r][h] = a;
      }
    }
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int h = 0; h < kValuHeads; ++h) s[i][h] = row16_sum(s[i][h]);

  // ---- V rows of the lane's slots, widened once
  float vf[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t w = T.v[i].w[e];
      const f16x2 h = as_f16x2(w);
      vf[i][2 * e] = (float)h[0];
      vf[i][2 * e + 1] = (float)h[1];
    }

  // ---- online softmax and P.V, head by head (log2 domain)
#pragma unroll
  for (int h = 0; h < kValuHeads; ++h) {
    float mt = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float x = s[i][h] * sscale;
      if (4 * g + (i & 3) >= T.nrow[i >> 2]) x = -INFINITY;
      s[i][h] = x;
      mt = fmaxf(mt, x);
    }
    mt = group4_max(mt);
    const float m_new = fmaxf(st.m_run[h], mt);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(st.m_run[h] - m_use);
    st.m_run[h] = m_new;
    st.l_run[h] *= alpha;
#pragma unroll
    for (int d = 0; d < 8; ++d) st.acc[h][d] *= alpha;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float pv = __builtin_amdgcn_exp2f(s[i][h] - m_use);
      st.l_run[h] += pv;
      const float pr = (float)(f16)pv;  // P in the PV operand type
#pragma unroll
      for (int d = 0; d < 8; ++d) st.acc[h][d] = fmaf(pr, vf[i][d], st.acc[h][d]);
    }
  }
}

#ifndef FSK_PIPE_DEPTH
#define FSK_PIPE_DEPTH 2
#endif
// Waves per SIMD the register budget is sized for (2: <= 256 VGPRs).
constexpr int kWavesPerEu = FSK_PIPE_DEPTH > 2 ? 1 : 2;

// The host's plan, when a launch passes one (after the Params).
__device__ __forceinline__ const HostPlan* plan_ptr() { return nullptr; }
__device__ __forceinline__ const HostPlan* plan_ptr(const HostPlan& h) { return &h; }

// The partial kernel.  Plan: none (the kernel builds the plan on the device
// from the lengths) or a HostPlan (built by the host from host lengths,
// B <= kHostPlanMax; lens_arg and starts_arg are then unused).
template <int D, int kQ, int kKV, int kLayout, bool kScores, bool kValu = false, typename... Plan>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(kWavesPerEu))) void partial_kernel(
    const int32_t* lens_arg, const int32_t* starts_arg, int B_arg, Params pk, Plan... host_plan) {
  // The plan's first loads (the lengths) need only these three, which lead
  // the argument list so that the dispatch preloads them into SGPRs
  // (-amdgpu-kernarg-preload-count): the length loads issue without waiting
  // for a kernel-argument load.
  Params p = pk;
  p.lens = lens_arg;
  p.starts = starts_arg;
  p.B = B_arg;
  constexpr bool kHostPlan = sizeof...(Plan) == 1;
  const HostPlan* hp = plan_ptr(host_plan...);
  using TR = TileRegs<D, kKV>;
  using SM = Softmax<D, kQ, kKV>;
  constexpr bool kKvFp8 = TR::kFp8;
  constexpr int kSteps = SM::kSteps;
  constexpr int kDpc = SM::kDpc;
  // Tiles in flight per wave (registers: ~64 VGPRs per fp16 tile at D=128).
  constexpr int kDepth = (D <= 128) ? FSK_PIPE_DEPTH : 1;
  static_assert(kKV != kBF16 || kQ == kBF16, "bf16 KV needs bf16 Q");
  static_assert(kKV != kF16 || kQ != kBF16, "f16 KV needs f16 Q");
  static_assert(!kValu || (D == 128 && kQ == kF16 && kKV == kF16 && !kScores && kLayout != kDense),
                "the VALU tile is built for f16, D = 128, paged and varlen");
  static_assert(!kHostPlan || (!kScores && !kValu), "host plans are for the plain decode kernels");

  __shared__ __attribute__((aligned(16))) uint8_t s_kstage_mem[kDepth * 2 * TR::kHalfBytes];
  // LDS offset of the stage = low 32 bits of its generic address
  const uint32_t s_kstage = (uint32_t)(uintptr_t)s_kstage_mem;
  extern __shared__ int32_t s_plan[];
  int32_t* s_pre = s_plan;              // [B+1] first partial of each sequence
  int32_t* s_flat = s_plan + p.B + 1;   // [B+1] stream offset of each sequence
  const int lane = threadIdx.x;
  const int g = lane >> 4;
  const int c = lane & 15;

  FSK_STAMP(0);
  FSK_STAMP_AT(6, (unsigned long long)__builtin_amdgcn_s_getreg((3 << 11) | 20));  // HW_REG_XCC_ID bits 3:0
  FSK_STAMP_AT(7, (unsigned long long)__builtin_amdgcn_s_getreg((31 << 11) | 4));  // HW_REG_HW_ID, all 32 bits
  FSK_STAMP_AT(2, 0ull);
  FSK_STAMP_AT(3, 0ull);
  int lane_start, lane_len;  // start and length of sequence `lane` (B <= 64)
  int lane_flat, lane_pre;   // flat[lane] and pre[lane] of the plan (B <= 64)
  int seg_x;  // empty stream positions before each sequence (see build_plan)
  Split sp;
  if constexpr (kHostPlan) {
    // The host's plan: each lane's entries from the kernel arguments (one
    // round trip), the split from scalar loads.
    lane_len = hp->len[lane];
    lane_start = hp->start[lane];
    lane_flat = hp->flat[lane];
    lane_pre = hp->pre[lane];
    __builtin_amdgcn_sched_barrier(0);
    sp.c_e = hp->c_e;
    sp.c_o = hp->c_o;
    sp.pair = sp.c_e + sp.c_o;
    sp.n = hp->n;
    sp.paired = hp->paired;
    sp.m = hp->m;
    seg_x = hp->seg_x;
  } else {
    seq_range_first<kLayout>(p, lane, lane_start, lane_len);  // the wave's first memory requests
    __builtin_amdgcn_sched_barrier(0);                        // (ahead of any kernel-argument load)
  }
  // ... and while they are in flight, the lane's tile offsets
  const LaneGeo<D, kKV> lg = lane_geo<D, kKV>(p, lane, g, c);
  // The KV scales, read before the plan (their round trip overlaps the
  // lengths') and used after it.
  const float k_scale = kKvFp8 ? p.k_scale[0] : 1.0f;
  const float v_scale = kKvFp8 ? p.v_scale[0] : 1.0f;
  if constexpr (kHostPlan) {
    // Workgroup 0 publishes the unit prefix for the reduce kernel, as
    // build_plan does (lanes past B hold pre[B]).
    if (blockIdx.x == 0) {
      if (lane < p.B) p.plan[lane] = lane_pre;
      if (lane == 0) p.plan[p.B] = hp->pre_end;
    }
  } else {
    sp = build_plan<kLayout, kScores>(p, s_pre, s_flat, lane_len, seg_x, lane_flat, lane_pre);
  }
  FSK_STAMP(1);
  int segments_done = 0;
  const int NH = p.n_items_h;
  const int W = sp.n * NH;  // < 2^31: the host bounds the workspace's units times NH
  // Plan tables: from the lanes' registers when B <= 64 (no LDS round trips
  // on the way to a unit's first loads), else from LDS.
  const bool small_b = p.B <= kWave;
  auto flat_at = [&](int b) { return small_b ? __builtin_amdgcn_readlane(lane_flat, b) : uniform(s_flat[b]); };
  auto pre_at = [&](int b) { return small_b ? __builtin_amdgcn_readlane(lane_pre, b) : uniform(s_pre[b]); };
  // Head pairs (varlen, head_dim 64, instantiated at D = 128): the token rows
  // of KV heads 2i and 2i+1 are 128-byte neighbours in [T, Hkv, 64], read as
  // one 256-byte row.  Columns 0..G-1 are head 2i's query heads with Q zero
  // in dims 64..127, columns G..2G-1 head 2i+1's with Q zero in dims 0..63,
  // so each column's scores are its own head's; of the 128 output dims a
  // column keeps its head's half.
  const bool pair = (kLayout == kVarlen && D == 128 && !kScores && !kValu) ? (uniform(p.pair) != 0) : false;
  const float sscale = p.score_scale * k_scale;

  for (int w = blockIdx.x; w < W; w += gridDim.x) {
    int jc, hh;
    item_of(sp, (uint32_t)w, p.nh_div, jc, hh);
    const int kvh = (int)fdiv((uint32_t)hh, p.hb_div);  // (with pair: the pair index, n_hb = 1)
    const int hb = hh - kvh * p.n_hb;
    const int lo = chunk_lo(sp, jc), hi = lo + chunk_len(sp, jc);  // stream range of this chunk
    // the last sequence whose region starts at or before lo (flat is nondecreasing, flat[0] = 0)
    const int b_first = small_b ? __builtin_popcountll(__ballot(lane < p.B && lane_flat <= lo)) - 1
                                : find_seq(s_flat, p.B, lo);
    for (int b = uniform(b_first); b < p.B; ++b) {
    const int fb = flat_at(b);
    if (fb >= hi) break;
    Unit un;
    un.b = b;
    un.kvh = pair ? 2 * kvh : kvh;
    if (p.B <= kWave) {
      un.start = __builtin_amdgcn_readlane(lane_start, un.b);
      un.len = __builtin_amdgcn_readlane(lane_len, un.b);
    } else {
      seq_range<kLayout>(p, un.b, un.start, un.len);
      un.start = uniform(un.start);
      un.len = uniform(un.len);
    }
    const int fs = fb + seg_x;  // sequence b's first token in the stream
    un.t_begin = max(lo - fs, 0);
    un.t_end = min(hi - fs, un.len);
    if (un.t_end <= un.t_begin) continue;  // only padding (or the empty lead-in) of sequence b in this chunk
    const int u = pre_at(b) + (jc - chunk_of(sp, fs));  // this segment's partial
    if (u >= p.u_max) continue;                          // (the host sizes u_max so this never holds)
    un.p_first = 0;
    un.win0 = un.win1 = un.win2 = un.win3 = 0;
    int win_raw0 = 0, win_raw1 = 0, win_raw2 = 0, win_raw3 = 0;
    if (segments_done == 0) FSK_STAMP(8);
    if constexpr (kLayout == kPaged) {
      un.p_first = (int)fdiv((uint32_t)un.t_begin, p.page);
      const int npg = (int)fdiv((uint32_t)(un.t_end - 1), p.page) - un.p_first + 1;  // <= 256 (chunk <= 4096)
      const int32_t* row = p.block_table + (int64_t)un.b * p.bt_sb + un.p_first;
      // Four range-checked loads (entries past npg read as 0) without
      // branches, so they and the Q loads below share one memory round trip;
      // the page ids are clamped to the pool once Q is in flight.
      const auto rw = make_rsrc(row, 4 * npg);
      win_raw0 = (int)buf_load<4>(rw, 4 * lane).w[0];
      win_raw1 = (int)buf_load<4>(rw, 4 * (lane + 64)).w[0];
      win_raw2 = (int)buf_load<4>(rw, 4 * (lane + 128)).w[0];
      win_raw3 = (int)buf_load<4>(rw, 4 * (lane + 192)).w[0];
    }

    // ---- Q^T operand: head c of this head block, zero for padding heads.
    // With pair, column c is query head c - G*hs of KV head un.kvh + hs.
    const int hs = (pair && c >= p.G) ? 1 : 0;
    const int head = hb * 16 + c - hs * p.G;
    const bool head_ok = head < p.G;
    u32x4 qop[kSteps];
    {
      const uint8_t* qrow =
          p.q + (int64_t)un.b * p.q_sb + (int64_t)((un.kvh + hs) * p.G + (head_ok ? head : 0)) * p.q_sh;
#pragma unroll
      for (int i = 0; i < kSteps; ++i) {
        const int dk = qk_dim0<kKvFp8>(i, g);  // dim of the (paired) K row
        const int d0 = pair ? (dk & 63) : dk;  // dim of this column's query row
        const bool q_ok = head_ok && (!pair || (dk >> 6) == hs);
        // Every lane loads (padding heads read head 0's row, then zero it):
        // unconditional loads keep the compiler's wait counts exact.
        u32x4 x;
        if constexpr (kQ == kE4M3) {
          // q = f16(f32(q8) * scale_q)  (triton_gqa_decode_hf_fp8.py:47-50)
          const u32x2 raw = *(const u32x2*)(qrow + d0);
          const float sq = p.q_scale[0];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(raw[e], false);
            const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(raw[e], true);
            x[2 * e] = pack_f16x2(lo[0] * sq, lo[1] * sq);
            x[2 * e + 1] = pack_f16x2(hi[0] * sq, hi[1] * sq);
          }
        } else {
          x = *(const u32x4*)(qrow + 2 * d0);
        }
        qop[i] = q_ok ? x : u32x4{0, 0, 0, 0};
      }
    }
    // VALU tile: dims [8c, 8c+8) of each of the (up to 4) query heads
    u32x4 qv[kValuHeads];
    if constexpr (kValu) {
#pragma unroll
      for (int h = 0; h < kValuHeads; ++h) {
        const uint8_t* qr = p.q + (int64_t)un.b * p.q_sb + (int64_t)(un.kvh * p.G + min(h, p.G - 1)) * p.q_sh;
        const u32x4 x = *(const u32x4*)(qr + 16 * c);
        qv[h] = h < p.G ? x : u32x4{0, 0, 0, 0};
      }
    }
    if constexpr (kLayout == kPaged) {
      un.win0 = clampi(win_raw0, 0, p.num_pages - 1);
      un.win1 = clampi(win_raw1, 0, p.num_pages - 1);
      un.win2 = clampi(win_raw2, 0, p.num_pages - 1);
      un.win3 = clampi(win_raw3, 0, p.num_pages - 1);
#ifdef FSK_WAVE_STAMPS
      // (the first tile's issue waits for the window anyway; Q shares its round trip)
      if (segments_done == 0) {
        __builtin_amdgcn_s_waitcnt(vm_wait_imm(0));
        FSK_STAMP(9);
      }
#endif
    }

    SM st;
    st.m_run = -INFINITY;
    st.l_run = 0.f;
#pragma unroll
    for (int j = 0; j < kDpc; ++j) st.acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    SoftmaxV sv;
    if constexpr (kValu) {
#pragma unroll
      for (int h = 0; h < kValuHeads; ++h) {
        sv.m_run[h] = -INFINITY;
        sv.l_run[h] = 0.f;
#pragma unroll
        for (int d = 0; d < 8; ++d) sv.acc[h][d] = 0.f;
      }
    }
    BlockMax bm;

    if constexpr (kDepth > 1) {
      // Tile slot s holds tile n with n % kDepth == s (its K stage is slot s
      // of s_kstage); while tile n is computed, tiles n+1 .. n+kDepth-1 are
      // in flight.
      // Tiles past the unit's end are issued too: their buffer ranges are
      // empty, so the loads read zeros without memory traffic, and every
      // tile is computed with exactly kDepth - 1 later tiles in flight (a
      // conditional issue would make the compiler wait for all loads).
      TR tiles[kDepth];
      const int n_tiles = (un.t_end - un.t_begin + 31) >> 5;
      const int rot = uniform(tile_rotation<kLayout, kScores>(un.kvh, n_tiles, p.hkv_div));
      int k = 0;  // tiles computed so far
#pragma unroll
      for (int s = 0; s < kDepth - 1; ++s)
        issue_tile<D, kKV, kLayout>(tiles[s], s_kstage + s * 2 * TR::kHalfBytes, p, un,
                                    tile_pos(s, n_tiles, rot, un.t_begin, un.t_end), lg);
      bool done = false;
      while (!done) {
#pragma unroll
        for (int s = 0; s < kDepth; ++s) {
          if (!done) {
            const int tn = tile_pos(k + kDepth - 1, n_tiles, rot, un.t_begin, un.t_end);
            const int sn = (s + kDepth - 1) % kDepth;
            issue_tile<D, kKV, kLayout>(tiles[sn], s_kstage + sn * 2 * TR::kHalfBytes, p, un, tn, lg);
            wait_k_stage<TR::kLoads, kDepth>(kDepth - 1);
            if (k == 0 && segments_done == 0) FSK_STAMP(2);
            if constexpr (kValu) {
              compute_tile_valu<D>(tiles[s], s_kstage + s * 2 * TR::kHalfBytes, sv, qv, sscale, g, c);
            } else {
              const float mt = compute_tile<D, kQ, kKV>(tiles[s], s_kstage + s * 2 * TR::kHalfBytes, st, qop,
                                                        sscale, g, lg);
              if constexpr (kScores) bm.add(p, un, un.t_begin + 32 * k, mt, head, head_ok, g);
            }
            ++k;
            done = k >= n_tiles;
          }
        }
      }
    } else {
      TR ta;
      for (int t = un.t_begin; t < un.t_end; t += 32) {
        issue_tile<D, kKV, kLayout>(ta, s_kstage, p, un, t, lg);
        wait_k_stage<TR::kLoads, 1>(0);
        if (t == un.t_begin && segments_done == 0) FSK_STAMP(2);
        if constexpr (kValu) {
          compute_tile_valu<D>(ta, s_kstage, sv, qv, sscale, g, c);
        } else {
          const float mt = compute_tile<D, kQ, kKV>(ta, s_kstage, st, qop, sscale, g, lg);
          if constexpr (kScores) bm.add(p, un, t, mt, head, head_ok, g);
        }
      }
    }

    // ---- unit epilogue: fp32 partial for each real head of the block
    if constexpr (kValu) {
      // k-group g holds the sums over its tokens: combine the four, then the
      // lanes of k-group 0 store dims [8c, 8c+8) of every head.
#pragma unroll
      for (int h = 0; h < kValuHeads; ++h) {
        const float l_h = group4_sum(sv.l_run[h]);
        float o[8];
#pragma unroll
        for (int d = 0; d < 8; ++d) o[d] = group4_sum(sv.acc[h][d]);
        if (h < p.G && g == 0) {
          const int64_t idx = ((int64_t)u * p.Hkv + un.kvh) * p.G + h;
          float* dst = p.part_acc + idx * D + 8 * c;
          *(f32x4*)dst = f32x4{o[0], o[1], o[2], o[3]};
          *(f32x4*)(dst + 4) = f32x4{o[4], o[5], o[6], o[7]};
          if (c == 0) *(f32x2*)(p.part_ml + 2 * idx) = f32x2{sv.m_run[h], l_h};
        }
      }
      continue;
    }
    const float l_tot = group4_sum(st.l_run);
    if (head_ok) {
      // Lane (g, c) holds dims [kDpc*4*g, kDpc*4*(g+1)) of column c: with
      // pair (kDpc = 8), k-groups 0-1 hold dims 0..63 and 2-3 dims 64..127,
      // and a column stores its own head's half into a 64-wide partial.
      const int64_t idx = ((int64_t)u * p.Hkv + un.kvh + hs) * p.G + head;
      const int dl = pair ? 64 : D;
      float* dst = p.part_acc + idx * dl + kDpc * 4 * g - hs * 64;
      if (!pair || (g >> 1) == hs) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int j = 0; j < kDpc; j += 4) {
            const f32x4 o = {st.acc[j][r] * v_scale, st.acc[j + 1][r] * v_scale, st.acc[j + 2][r] * v_scale,
                             st.acc[j + 3][r] * v_scale};
            *(f32x4*)(dst + kDpc * r + j) = o;
          }
      }
      if (g == 0) *(f32x2*)(p.part_ml + 2 * idx) = f32x2{st.m_run, l_tot};
    }
    ++segments_done;
    FSK_STAMP(3);
    }  // segments of the chunk
  }
  FSK_STAMP_AT(5, (unsigned long long)segments_done);
  FSK_STAMP(4);
  (void)segments_done;
  (void)hp;
}

// ---------------------------------------------------------------------------
// Reduce kernel: LSE merge of a sequence's partials + sink fold.
// ---------------------------------------------------------------------------
struct ReduceParams {
  const int32_t* plan;
  const float* part_ml;
  const float* part_acc;
  const float* s_aux;
  int sink_mode;
  uint8_t* out;
  int64_t o_sb, o_sh;  // bytes
  int Hq, Hkv, G;
  // Block scores (null scores: none): S[b, h, j] = largest attention
  // probability of block j = exp2(blk_max - M) / den; 0 past the sequence.
  const float* blk_max;
  const int32_t* lens;
  uint8_t* scores;     // [B, Hq, nblk] in the output dtype, contiguous
  int nblk;
};

constexpr int kReduceThreads = 256;

template <int D, int kOut, int kRows>
__global__ __launch_bounds__(kReduceThreads) void reduce_kernel(ReduceParams p) {
  // One workgroup per kRows query heads of a sequence (kRows > 1 for large
  // batches of short sequences, whose rows have few partials each).  Thread
  // t of row r = t / (256 / kRows) owns the float4 column d4 = t % (D/4) of
  // unit group grp; group grp merges units grp, grp + kGroups, ... with an
  // online LSE update, loading kPer units per round trip, and the groups
  // combine through LDS.
  constexpr int kD4 = D / 4;
  constexpr int kRowThreads = kReduceThreads / kRows;
  constexpr int kGroups = kRowThreads / kD4;
  static_assert(kGroups >= 1, "a row needs at least one group of D/4 threads");
  constexpr int kPer = 4;
  __shared__ float s_m[kRows][kGroups];
  __shared__ float s_l[kRows][kGroups];
  __shared__ f32x4 s_acc[kRows][kGroups][kD4];
  const int tid = threadIdx.x;
  const int row = tid / kRowThreads;
  const int d4 = (tid - row * kRowThreads) % kD4;
  const int grp = (tid - row * kRowThreads) / kD4;
  const int h = blockIdx.x * kRows + row;
  const int b = blockIdx.y;
  const int kvh = h / p.G;
  const int hg = h - kvh * p.G;
  // The sink and the sequence length are loaded with the unit range, not
  // after the merge, so they cost no round trip of their own.
  const float z = p.s_aux ? p.s_aux[h] : 0.f;
  const int len_b = *(p.scores ? p.lens + b : p.plan + b);  // (no branch: one round trip with the plan)
  const int u0 = p.plan[b];
  const int n = p.plan[b + 1] - u0;
  const int64_t base = ((int64_t)u0 * p.Hkv + kvh) * p.G + hg;  // partial index of unit u0
  const int64_t ustride = (int64_t)p.Hkv * p.G;                 // between consecutive units
  // Block scores: every thread loads up to kScorePre of this row's block
  // maxima now, in the same round trip as the partials, and stores their
  // scores once the denominator is known.
  constexpr int kScorePre = 4;
  float bmax[kScorePre];
  if (kRows == 1 && p.scores) {
    const float* src = p.blk_max + ((int64_t)b * p.Hq + h) * p.nblk;
#pragma unroll
    for (int i = 0; i < kScorePre; ++i) {
      const int j = tid + i * kReduceThreads;
      bmax[i] = j < p.nblk ? src[j] : -INFINITY;
    }
  }

  float m_t = -INFINITY, l_t = 0.f;
  f32x4 a_t = {0.f, 0.f, 0.f, 0.f};
  for (int i0 = grp; i0 < n; i0 += kGroups * kPer) {
    f32x2 ml[kPer];
    f32x4 ac[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = i0 + j * kGroups;
      if (i < n) {
        const int64_t idx = base + i * ustride;
        ml[j] = *(const f32x2*)(p.part_ml + 2 * idx);
        ac[j] = *(const f32x4*)(p.part_acc + idx * D + 4 * d4);
      } else {
        ml[j] = f32x2{-INFINITY, 0.f};
        ac[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
    float mx = m_t;
#pragma unroll
    for (int j = 0; j < kPer; ++j) mx = fmaxf(mx, ml[j][0]);
    const float mu = (mx == -INFINITY) ? 0.f : mx;
    const float f = __builtin_amdgcn_exp2f(m_t - mu);
    l_t *= f;
    a_t *= f;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const float w = __builtin_amdgcn_exp2f(ml[j][0] - mu);
      l_t += ml[j][1] * w;
      a_t += ac[j] * w;
    }
    m_t = mx;
  }
  if (d4 == 0) s_m[row][grp] = m_t;
  __syncthreads();
  float M = s_m[row][0];
#pragma unroll
  for (int q = 1; q < kGroups; ++q) M = fmaxf(M, s_m[row][q]);
  const float M_use = (M == -INFINITY) ? 0.f : M;
  const float f = __builtin_amdgcn_exp2f(m_t - M_use);
  s_acc[row][grp][d4] = a_t * f;
  if (d4 == 0) s_l[row][grp] = l_t * f;
  __syncthreads();
  // The denominator (every thread when block scores need it), then the
  // numerator (group 0, which stores the output row).
  const bool scores = kRows == 1 && p.scores;
  if (grp != 0 && !scores) return;
  float den = s_l[row][0];
#pragma unroll
  for (int q = 1; q < kGroups; ++q) den += s_l[row][q];
  float fs = 1.f;     // scale of the numerator for an exp sink
  float ref = M_use;  // reference point of den
  if (p.s_aux) {
    if (p.sink_mode == FSK_SINK_EXP) {
      // Extra logit z with a zero value vector (log2 domain: z * log2 e).
      const float z2 = z * kLog2e;
      const float Mn = fmaxf(M, z2);
      const float Mn_use = (Mn == -INFINITY) ? 0.f : Mn;
      // An empty sequence (M = -inf, num = den = 0) keeps a zero numerator.
      fs = (M == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(M - Mn_use);
      den = den * fs + __builtin_amdgcn_exp2f(z2 - Mn_use);
      ref = Mn_use;
    } else {
      den += z;  // linear fold relative to the running max (flash_decode_cuda.cu:151-153)
    }
  }

  if (scores) {
    const int nvalid = (len_b + kScoreBlock - 1) / kScoreBlock;
    const float inv = 1.f / den;
    const float* src = p.blk_max + ((int64_t)b * p.Hq + h) * p.nblk;
    uint8_t* dst = p.scores + ((int64_t)b * p.Hq + h) * p.nblk * (kOut == kF32 ? 4 : 2);
    auto put = [&](int j, float mx) {
      const float sc = j < nvalid ? __builtin_amdgcn_exp2f(mx - ref) * inv : 0.f;
      if constexpr (kOut == kF32) ((float*)dst)[j] = sc;
      else if constexpr (kOut == kF16) ((f16*)dst)[j] = (f16)sc;
      else ((bf16*)dst)[j] = (bf16)sc;
    };
#pragma unroll
    for (int i = 0; i < kScorePre; ++i) {
      const int j = tid + i * kReduceThreads;
      if (j < p.nblk) put(j, bmax[i]);
    }
    for (int j = tid + kScorePre * kReduceThreads; j < p.nblk; j += kReduceThreads) put(j, src[j]);
  }
  if (grp != 0) return;
  f32x4 num = s_acc[row][0][d4];
#pragma unroll
  for (int q = 1; q < kGroups; ++q) num += s_acc[row][q][d4];
  if (p.s_aux && p.sink_mode == FSK_SINK_EXP) num *= fs;

  uint8_t* o = p.out + (int64_t)b * p.o_sb + (int64_t)h * p.o_sh;
  const f32x4 val = num / den;
  if constexpr (kOut == kF32) {
    *(f32x4*)((float*)o + 4 * d4) = val;
  } else if constexpr (kOut == kF16) {
    *(uint32_t __attribute__((ext_vector_type(2)))*)((f16*)o + 4 * d4) =
        u32x2{pack_f16x2(val[0], val[1]), pack_f16x2(val[2], val[3])};
  } else {
    *(uint32_t __attribute__((ext_vector_type(2)))*)((bf16*)o + 4 * d4) =
        u32x2{pack_bf16x2(val[0], val[1]), pack_bf16x2(val[2], val[3])};
  }
}

// ---------------------------------------------------------------------------
// Debug kernels
// ---------------------------------------------------------------------------
template <int D, int kElem>
__global__ __launch_bounds__(64) void paged_gather_kernel(Params p, uint8_t* out, int64_t o_rows) {
  // grid: (tiles of 16 rows, Hkv, B); out [B, Hkv, o_rows, D] contiguous
  constexpr int kRowBytes = D * kElem;
  constexpr int kChunks = kRowBytes / 16;
  const int t = blockIdx.x * 16;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  int start, len;
  seq_range<kPaged>(p, b, start, len);
  HalfTile ht = half_tile<kPaged>(p, b, start, len, kvh, t);
  const int bytes = ht.rows > 0 ? (ht.rows - 1) * (int)p.k_st + kRowBytes : 0;
  auto rk = make_rsrc(ht.k, bytes);
  uint8_t* dst = out + (((int64_t)b * p.Hkv + kvh) * o_rows + t) * kRowBytes;
  for (int i = threadIdx.x; i < 16 * kChunks; i += kWave) {
    const int r = i / kChunks, ch = i - r * kChunks;
    Chunk<16> x = buf_load<16>(rk, r * (int)p.k_st + 16 * ch);
    *(u32x4*)(dst + r * kRowBytes + 16 * ch) = u32x4{x.w[0], x.w[1], x.w[2], x.w[3]};
  }
}

__global__ __launch_bounds__(64) void fp8_table_kernel(uint32_t* out) {
  // Codes 4l .. 4l+3 through both widening routes.  The raw 16-bit results are
  // stored as produced (the host widens them to fp32), so the table exercises
  // exactly the instruction sequence the decode kernels use.
  const int l = threadIdx.x;
  const uint32_t w = (uint32_t)(4 * l) | ((uint32_t)(4 * l + 1) << 8) | ((uint32_t)(4 * l + 2) << 16) |
                     ((uint32_t)(4 * l + 3) << 24);
  const u32x2 h = e4m3x4_to<false>(w);
  const u32x2 bb = e4m3x4_to<true>(w);
  *(u32x2*)(out + 2 * l) = h;
  *(u32x2*)(out + 128 + 2 * l) = bb;
}

// ---------------------------------------------------------------------------
// KV write path: scatter new tokens' K/V rows into the page pools
// ---------------------------------------------------------------------------
// Token i of the batch goes to page slots[i] / page_size, row slots[i] %
// page_size, of every KV head (fskernels/paged_attn/paged_kv_cache.py:117-130
// does this per token with two indexed copies).  Each thread moves one
// 8-element column group of one (token, head) row: consecutive threads cover a
// row, then the next head, then the next token, so both the source read and
// the pool write are contiguous 16-byte accesses (8 bytes for e4m3 pools).
// Division by a divisor d fixed per launch, for dividends below 2^31:
// q = (x * m) >> s with s = 31 + ceil(log2 d), m = ceil(2^s / d).  The error
// term (m d - 2^s) x / (d 2^s) stays below 1/d, so q == x / d exactly.
struct WriteParams {
  const uint8_t* src[2];               // K, V: [n, Hkv, D] rows
  int64_t s_st[2], s_sh[2];            // token / head strides, bytes
  uint8_t* pool[2];                    // [P, Hkv, page_size, D]
  int64_t p_sp[2], p_sh[2], p_st[2];   // page / head / row strides, bytes
  const float* scale[2];               // e4m3 pools: quantisation scale, or null
  const int64_t* slots;                // [n] page * page_size + row; < 0: skip
  uint32_t n_slots;                    // num_pages * page_size (< 2^31)
  uint32_t rows;                       // n * Hkv
  FastDiv hkv, page;                   // divisors Hkv and page_size
  FastDiv groups;                      // divisor D / 8: column groups per row
  uint32_t rows_per_block;             // kWriteThreads / groups
  int32_t* bt;                         // block-table updates: bt[upd[2j]] = upd[2j+1]
  int64_t bt_numel;
  const int64_t* upd;
  int n_upd;
};

constexpr int kWriteThreads = 256;
// Workgroups per CU for each of the K and V planes, and the cache policy of
// the row loads and stores (1: non-temporal, each row is read once and
// written once).  A thread stores one row per step; with non-temporal access
// that measured fastest (W0 206.5 -> 199.7 us, W1 162.3 -> 155.1 us against
// four rows loaded before their stores and the default policy).
#ifndef FSK_WRITE_BLOCKS_PER_CU
#define FSK_WRITE_BLOCKS_PER_CU 16
#endif
#ifndef FSK_WRITE_NT
#define FSK_WRITE_NT 1
#endif

template <typename T>
__device__ __forceinline__ T row_load(const T* p) {
  if constexpr (FSK_WRITE_NT) return __builtin_nontemporal_load(p);
  else return *p;
}
template <typename T>
__device__ __forceinline__ void row_store(T* p, T x) {
  if constexpr (FSK_WRITE_NT) __builtin_nontemporal_store(x, p);
  else *p = x;
}

// One thread's share of a row in flight: its slot and its 8 source elements
// (raw bits; f32 sources in two halves).
struct WriteRow {
  int64_t slot;
  uint32_t i, h;  // token and head of the row
  u32x4 raw[2];
};

// Issues the loads of row `row` (< rows): the slot and the source elements
// together, so a row costs one memory round trip before its store.
template <int kSrc>
__device__ __forceinline__ WriteRow write_row_issue(FastDiv hkv, const int64_t* slots, const uint8_t* src,
                                                    int64_t s_st, int64_t s_sh, uint32_t row) {
  WriteRow w;
  w.i = fdiv(row, hkv);
  w.h = row - w.i * hkv.d;
  w.slot = slots[w.i];
  const uint8_t* a = src + w.i * s_st + w.h * s_sh;
  w.raw[0] = row_load((const u32x4*)a);
  if constexpr (kSrc == kF32) w.raw[1] = row_load((const u32x4*)(a + 16));
  return w;
}

template <int kSrc>
__device__ __forceinline__ void widen8(const WriteRow& w, float (&x)[8]) {
  if constexpr (kSrc == kF32) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t b = w.raw[j >> 2][j & 3];
      x[j] = u2f(b);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // The element goes through a scalar: this compiler lowers
      // __builtin_bit_cast of a vector-element operand to a load from the
      // vector's first element.
      const uint32_t b = w.raw[0][j];
      if constexpr (kSrc == kF16) {
        const f16x2 hx = __builtin_bit_cast(f16x2, b);
        x[2 * j] = (float)hx[0];
        x[2 * j + 1] = (float)hx[1];
      } else {
        x[2 * j] = bf16_lo_to_f32(b);
        x[2 * j + 1] = bf16_hi_to_f32(b);
      }
    }
  }
}

// x / s rounded to fp32, for fp32 x and a scale s (finite, nonzero), from
// rs = RN64(1 / s) as RN32(RN64(x * rs)).  This equals the correctly rounded
// fp32 quotient: with x = X 2^a and s = S 2^b (X, S odd, < 2^24) the exact
// quotient is never an fp32 rounding midpoint (a midpoint has 25 significant
// bits, so m s = x would need an odd factor >= 2^24 + 1 in X) and lies at a
// relative distance >= 1 / (2 S 2^24) >= 2^-49 from every midpoint, while the
// two binary64 roundings perturb it by at most 2^-52 (1 + 2^-53) relative.
// Quotients in the fp32 subnormal range may differ, but they all quantise to
// a signed zero below.  Costs a convert, a multiply and a convert instead of
// the ten-instruction fp32 division sequence.
__device__ __forceinline__ float div_by_scale(float x, double rs) {
  return (float)((double)x * rs);
}

// Four fp32 values -> four e4m3fn codes (round to nearest even, as torch's
// float8_e4m3fn cast).  With a scale the values are first divided by it
// (rs = 1 / scale in binary64, see div_by_scale) and clamped to +-448 (the
// quantiser of fskernels/triton/triton_gqa_decode_hf_fp8.py:13-16); without one
// they are cast as they are, so magnitudes above 464 encode NaN as the cast
// does.  NaN inputs are left to nan_codes.
template <bool kScaled>
__device__ __forceinline__ uint32_t encode_e4m3x4(const float* x, double rs) {
  float y[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    y[j] = x[j];
    if constexpr (kScaled) y[j] = fminf(fmaxf(div_by_scale(x[j], rs), -E4M3_MAX_F), E4M3_MAX_F);
  }
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], w, true);
  return (uint32_t)w;
}

// NaN inputs take 0x7F with the input's sign bit, as torch's cast gives them.
__device__ __forceinline__ uint32_t nan_codes(uint32_t u, const float* x) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (x[j] != x[j]) {
      const uint32_t code = 0x7Fu | ((f2u(x[j]) >> 31) << 7);
      u = (u & ~(0xFFu << (8 * j))) | (code << (8 * j));
    }
  }
  return u;
}

template <int kPool>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (kPool == kF16) return pack_f16x2(a, b);
  else return pack_bf16x2(a, b);
}

template <int kSrc, int kPool, bool kScaled>
__device__ __forceinline__ void write_row_put(const WriteRow& w, uint32_t n_slots, FastDiv page_div, uint8_t* pool,
                                              int64_t p_sp, int64_t p_sh, int64_t p_st, double rscale) {
  if (w.slot < 0 || w.slot >= (int64_t)n_slots) return;  // skipped slot
  const uint32_t page = fdiv((uint32_t)w.slot, page_div);
  const uint32_t r = (uint32_t)w.slot - page * page_div.d;
  uint8_t* dst = pool + page * p_sp + w.h * p_sh + r * p_st;
  if constexpr (kPool == kSrc) {
    row_store((u32x4*)dst, w.raw[0]);  // same type: a bit-exact copy
  } else {
    float x[8];
    widen8<kSrc>(w, x);
    if constexpr (kPool == kE4M3) {
      u32x2 codes{encode_e4m3x4<kScaled>(x, rscale), encode_e4m3x4<kScaled>(x + 4, rscale)};
      // The NaN fix-up only where the wave holds a NaN: the quantising
      // write is VALU-bound enough that per-code selects cost it ~2 %.
      bool nan = false;
#pragma unroll
      for (int j = 0; j < 8; ++j) nan = nan || x[j] != x[j];
      if (__builtin_amdgcn_ballot_w64(nan) != 0) {
        codes[0] = nan_codes(codes[0], x);
        codes[1] = nan_codes(codes[1], x + 4);
      }
      row_store((u32x2*)dst, codes);
    } else {
      row_store((u32x4*)dst, u32x4{pack2<kPool>(x[0], x[1]), pack2<kPool>(x[2], x[3]), pack2<kPool>(x[4], x[5]),
                                   pack2<kPool>(x[6], x[7])});
    }
  }
}

template <int kSrc, int kPool, bool kScaled>
__global__ __launch_bounds__(kWriteThreads) void kv_write_kernel(WriteParams p) {
  const int kv = blockIdx.y;
  // The kernel arguments, read in one batch: the asm takes them all in
  // SGPRs, so their loads go out together and are waited for once, not one
  // round trip after another behind the branches that first use them.
  const uint8_t* src0 = p.src[kv];
  const int64_t s_st = p.s_st[kv], s_sh = p.s_sh[kv];
  uint8_t* pool0 = p.pool[kv];
  const int64_t p_sp = p.p_sp[kv], p_sh = p.p_sh[kv], p_st = p.p_st[kv];
  const float* scale = p.scale[kv];
  const int64_t* slots = p.slots;
  const FastDiv hkv = p.hkv, page = p.page, groups = p.groups;
  const uint32_t n_slots = p.n_slots, rows = p.rows, rows_per_block = p.rows_per_block;
  const int64_t* upd = p.upd;
  const int n_upd = p.n_upd;
  asm volatile("" ::"s"(src0), "s"(s_st), "s"(s_sh), "s"(pool0), "s"(p_sp), "s"(p_sh), "s"(p_st), "s"(scale),
               "s"(slots), "s"(hkv.m), "s"(hkv.s), "s"(hkv.d), "s"(page.m), "s"(page.s), "s"(page.d),
               "s"(groups.m), "s"(groups.s), "s"(groups.d), "s"(n_slots), "s"(rows), "s"(rows_per_block), "s"(upd),
               "s"(n_upd));
  // Block-table updates (workgroup (0, 0)): the first kWriteThreads are
  // loaded with the first rows and stored after them, so they add no round
  // trip to the launch (the decode kernels read both after it ends).
  const bool upd_block = blockIdx.x == 0 && kv == 0;
  int64_t upd_idx = -1;
  int32_t upd_val = 0;
  if (upd_block && (int)threadIdx.x < n_upd) {
    upd_idx = upd[2 * threadIdx.x];
    // (the low word of the int64 value, all the store keeps: a whole-pair
    // load would leave a dead register the first row's loads wait for)
    upd_val = ((const int32_t*)upd)[4 * threadIdx.x + 2];
  }
  constexpr int kSrcBytes = (kSrc == kF32) ? 32 : 16;   // 8 source elements
  constexpr int kDstBytes = (kPool == kE4M3) ? 8 : 16;  // 8 pool elements
  // A block covers rows_per_block (token, head) rows per step, `groups`
  // threads per row; the row stride between a thread's steps is fixed, so its
  // column group never changes.
  const uint32_t lrow = fdiv(threadIdx.x, groups);
  const uint32_t first = blockIdx.x * rows_per_block + lrow;
  if (lrow < rows_per_block && first < rows) {
    const uint32_t g = threadIdx.x - lrow * groups.d;
    const uint8_t* src = src0 + g * kSrcBytes;
    uint8_t* pool = pool0 + g * kDstBytes;
    const uint32_t step = gridDim.x * rows_per_block;
    // The first row's loads go out before the scale's, whose reciprocal
    // (a binary64 division) the encoding needs only once the row is in.
    WriteRow w = write_row_issue<kSrc>(hkv, slots, src, s_st, s_sh, first);
    __builtin_amdgcn_sched_barrier(0);
    double rscale = 1.0;
    if constexpr (kScaled) rscale = 1.0 / (double)*scale;
    for (uint32_t row = first;;) {
      write_row_put<kSrc, kPool, kScaled>(w, n_slots, page, pool, p_sp, p_sh, p_st, rscale);
      row += step;
      if (row >= rows) break;
      w = write_row_issue<kSrc>(hkv, slots, src, s_st, s_sh, row);
    }
  }
  if (upd_block) {
    if (upd_idx >= 0 && upd_idx < p.bt_numel) p.bt[upd_idx] = upd_val;
    for (int j = threadIdx.x + kWriteThreads; j < n_upd; j += kWriteThreads) {
      const int64_t idx = upd[2 * j];
      if (idx >= 0 && idx < p.bt_numel) p.bt[idx] = (int32_t)upd[2 * j + 1];
    }
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

struct Options {
  int chunk_tokens = 0;         // 0: automatic
  int waves_per_cu = 8;         // largest persistent grid (workgroups per CU)
  int target_waves_per_cu = 4;  // automatic split: units of work per CU
  int xcd_skew = 3;             // automatic split: extra share of the even XCDs, in % (see item_of)
  int chunk_pref = 2432;        // automatic split: longest chunk before one doubling of the count (16-bit tokens)
  int qk_engine = 0;            // 0: QK and PV on the matrix cores; 1: the VALU tile (A/B measurement)
  int head_pairs = 1;           // varlen, head_dim 64: neighbouring KV heads as one 128-wide row (see pair_shape)
  int seg_tokens = 96;          // lead-in per sequence in the work stream where boundaries are common (tokens)
} g_opt;

// Event triples of timed decode calls (the partial kernel's start and end and
// the reduce kernel's end, stamped by the dispatches themselves).
struct Timing {
  bool enabled = false;
  int every = 1;       // record on every n-th decode call
  int64_t calls = 0;
  std::vector<hipEvent_t> ev;  // 3 per recorded call
  std::vector<hipEvent_t> spare;
} g_timing;

bool timing_this_call() {
  if (!g_timing.enabled) return false;
  return (g_timing.calls++ % g_timing.every) == 0;
}

hipEvent_t timing_event() {
  hipEvent_t e = nullptr;
  if (!g_timing.spare.empty()) {
    e = g_timing.spare.back();
    g_timing.spare.pop_back();
  } else if (hipEventCreate(&e) != hipSuccess) {
    e = nullptr;
  }
  return e;
}

// Three events for this call if it is a timed one, else nulls.
void timing_events(hipEvent_t ev[3]) {
  ev[0] = ev[1] = ev[2] = nullptr;
  if (!timing_this_call()) return;
  for (int i = 0; i < 3; ++i) ev[i] = timing_event();
  if (!ev[0] || !ev[1] || !ev[2]) {
    for (int i = 0; i < 3; ++i)
      if (ev[i]) g_timing.spare.push_back(ev[i]);
    ev[0] = ev[1] = ev[2] = nullptr;
    g_timing.enabled = false;  // could not create events: stop timing rather than mis-pair
  }
}

// Keeps a launched call's events for fsk_kernel_timing, or returns them to
// the spares when the call did not launch.
void timing_keep(hipEvent_t ev[3], bool launched) {
  if (!ev[0]) return;
  for (int i = 0; i < 3; ++i) (launched ? g_timing.ev : g_timing.spare).push_back(ev[i]);
}

void timing_clear() {
  for (hipEvent_t e : g_timing.ev) g_timing.spare.push_back(e);
  g_timing.ev.clear();
}

int elem_bytes(int dt) {
  switch (dt) {
    case FSK_F16: case FSK_BF16: return 2;
    case FSK_F32: return 4;
    case FSK_E4M3: return 1;
    default: return 0;
  }
}

int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t align256(int64_t x) { return (x + 255) & ~(int64_t)255; }

constexpr int kChunkMin = 128;   // floor of an automatic split (tokens; short streams go down to kShortChunk)
constexpr int kSegTokensMax = 256;  // largest lead-in per sequence (tokens)
constexpr int kChunkMax = 4096;  // largest split: 256 pages of 16 tokens per paged unit (the page window)

// Longest padded token stream a call can have (each sequence is padded to a
// multiple of at most 128 tokens on the device).
int64_t stream_bound(int layout, int B, int64_t kv_extent, int page_size) {
  constexpr int64_t kSlack = 128 + kSegTokensMax;  // padding and lead-in per sequence
  if (layout == FSK_LAYOUT_VARLEN) return kv_extent + kSlack * (int64_t)B;
  if (layout == FSK_LAYOUT_PAGED) return (int64_t)B * (kv_extent * page_size + kSlack);
  return (int64_t)B * (kv_extent + kSlack);
}

// Partials a call can produce with split size `chunk` (host-side bound): the
// stream's chunks plus one more per sequence boundary.
int64_t unit_bound(int layout, int B, int64_t kv_extent, int page_size, int chunk) {
  return cdiv(stream_bound(layout, B, kv_extent, page_size), chunk) + B + 1;
}

// Chunks the device can plan for a stream of at most `stream` tokens: a
// split never has more than its target count of chunks (doubled once past
// chunk_pref and then while the chunks would exceed chunk_max, as
// split_geometry does; a longer bound doubles at least as often), plus one
// from an XCD-skewed split's even count.
int64_t chunk_bound(int64_t target_units, int chunk_pref, int chunk_max, int64_t stream) {
  int64_t t = target_units;
  if (t < cdiv(stream, chunk_pref)) t *= 2;
  const int64_t need = cdiv(stream, chunk_max);
  while (t < need && t < ((int64_t)1 << 24)) t *= 2;
  return t + 1;
}

// Split policy of one call: a fixed split when the caller (or the
// chunk_tokens option) asks for one, else bounds for the device-side choice
// and a workspace capacity that always holds the chunk_pref split.
struct SplitPlan {
  int chunk_min, chunk_max, chunk_pref, target_units;
  int64_t u_max;
};
SplitPlan plan_split(int layout, int B, int64_t nh, int64_t kv_extent, int page_size, int chunk_tokens, int cus,
                     int kv_bytes) {
  SplitPlan sp;
  const int fixed = chunk_tokens > 0 ? chunk_tokens : chunk_tokens == 0 ? g_opt.chunk_tokens : 0;
  if (fixed > 0) {
    sp.chunk_min = sp.chunk_max = sp.chunk_pref = fixed;
    sp.target_units = 1;
    sp.u_max = unit_bound(layout, B, kv_extent, page_size, fixed);
    return sp;
  }
  // chunk_tokens < 0: an automatic split of chunks of at most -chunk_tokens
  // tokens (the dense entry points' split-count hint)
  // (below 128 tokens the floor is the short-stream one, so that a cap never
  // makes a split coarser than the uncapped choice)
  sp.chunk_max = chunk_tokens < 0 && chunk_tokens > -kChunkMax ? -chunk_tokens : kChunkMax;
  sp.chunk_min = sp.chunk_max >= kChunkMin ? kChunkMin : std::min(kShortChunk, sp.chunk_max);
  // Chunks longer than chunk_pref 16-bit tokens' worth of KV bytes are split
  // once, up to one item per wave of a grid of 8 per CU (head_dim 128, 8 KV
  // heads, B x 4096 tokens: B=80, 96, 128 from 217, 258, 345 us in the partial
  // kernel to 206, 245, 321 us; C3's 2351-token chunks stay: halving them cost
  // 3-4 us, as did halving the 2560-3200-token chunks of B=160, 200 x 4096 again).
  const int pref = g_opt.chunk_pref * 2 / kv_bytes / 128 * 128;
  sp.chunk_pref = std::max(sp.chunk_min, std::min(sp.chunk_max, pref));
  const int64_t target = std::max<int64_t>(1, (int64_t)cus * g_opt.target_waves_per_cu / nh);
  sp.target_units = (int)std::min<int64_t>(target, 1 << 20);
  const int64_t cap = std::max<int64_t>(4 * target, 256);
  // Room for short-stream splits (chunks down to kShortChunk, at most 32 per
  // sequence on average) only where the device can choose them: the
  // workspace bound also sizes the persistent grid.
  int64_t u_plan = unit_bound(layout, B, kv_extent, page_size, sp.chunk_min);
  if (stream_bound(layout, B, kv_extent, page_size) < target * kChunkMin)
    u_plan = std::max(u_plan, std::min(unit_bound(layout, B, kv_extent, page_size, kShortChunk),
                                       33 * (int64_t)B + 1));
  // The workspace holds every split the doubling can reach (at most
  // chunk_bound chunks, plus one partial per sequence boundary), so that its
  // capacity never makes the chunk count uneven over the grid.
  const int64_t u_split =
      chunk_bound(sp.target_units, sp.chunk_pref, sp.chunk_max, stream_bound(layout, B, kv_extent, page_size)) + B + 1;
  sp.u_max = std::max(u_split, std::min(u_plan, cap));
  return sp;
}

// Varlen decodes at head_dim 64 with an even number of KV heads and at most
// 8 query heads per KV head take neighbouring KV heads in pairs (partial_kernel
// at D = 128) when the heads of a token row are packed; the split is planned
// for head_dim and head count alone, so the workspace size does not depend on
// the strides.
bool pair_shape(int layout, int D, int Hkv, int G) {
  return layout == FSK_LAYOUT_VARLEN && D == 64 && Hkv % 2 == 0 && G <= 8;
}
// Head slots per chunk the split is planned for.
int64_t plan_heads(int layout, int D, int Hkv, int G) {
  return pair_shape(layout, D, Hkv, G) ? Hkv / 2 : (int64_t)Hkv * ((G + 15) / 16);
}

struct WsLayout {
  int64_t plan_off, ml_off, acc_off, total;
};
WsLayout ws_layout(int B, int Hkv, int G, int D, int64_t u_max) {
  WsLayout w;
  w.plan_off = 0;
  w.ml_off = align256(4 * (int64_t)(B + 1));
  w.acc_off = w.ml_off + align256(u_max * Hkv * G * 2 * 4);
  w.total = w.acc_off + align256(u_max * Hkv * G * (int64_t)D * 4);
  return w;
}

struct Common {
  int layout;
  const void* q; int64_t q_sb, q_sh;
  const void* k; int64_t k_s0, k_sh, k_st;
  const void* v; int64_t v_s0, v_sh, v_st;
  const int32_t* lens; const int32_t* starts;
  const int32_t* bt; int64_t bt_sb; int max_blocks, num_pages, page_size;
  int64_t kv_extent;
  const float* s_aux; int sink_mode;
  const float *q_scale, *k_scale, *v_scale;
  void* out; int64_t o_sb, o_sh;
  int B, Hq, Hkv, D, q_dt, kv_dt, o_dt;
  float sm_scale;
  void* ws; int64_t ws_bytes; int chunk;
  hipStream_t stream;
  void* scores; int nblk;  // block scores [B, Hq, nblk] in the output dtype, or null
  bool no_timing;          // never stamp this call (no event creation: the allocation-free entry)
  bool lens_on_host;       // lens is host memory: the plan is built here (make_host_plan)
};

bool aligned(const void* p, int a) { return ((uintptr_t)p % a) == 0; }

// Extra workspace of a call with block scores: raw block maxima + lengths.
int64_t score_ws_bytes(int B, int Hq, int nblk) {
  return align256((int64_t)B * Hq * nblk * 4) + align256(4 * (int64_t)B);
}

// Bounds on batch and query heads: keep every size product (batch x heads x
// blocks or units x 4 bytes) inside int64.
constexpr int kMaxBatch = 16384;
constexpr int kMaxQHeads = 1 << 16;
constexpr int64_t kMaxStride = (int64_t)1 << 40;

int validate(const Common& c) {
  if (c.B < 0 || c.Hq <= 0 || c.Hkv <= 0) return fail(FSK_ERR_INVALID, "batch/heads must be positive");
  if (c.Hq > kMaxQHeads) return fail(FSK_ERR_UNSUPPORTED, "num_q_heads above 65536");
  if (c.Hq % c.Hkv != 0) return fail(FSK_ERR_INVALID, "num_q_heads must be a multiple of num_kv_heads");
  if (c.D != 64 && c.D != 128 && c.D != 256) return fail(FSK_ERR_UNSUPPORTED, "head_dim must be 64, 128 or 256");
  // An empty varlen/dense KV (extent 0: every sequence empty) reads no row, so
  // its k/v may be null, as an empty tensor's data pointer is.
  const bool kv_empty = c.layout != FSK_LAYOUT_PAGED && c.kv_extent == 0;
  if (!c.q || !c.lens || !c.out || (!kv_empty && (!c.k || !c.v))) return fail(FSK_ERR_INVALID, "null tensor pointer");
  if (c.sink_mode != FSK_SINK_EXP && c.sink_mode != FSK_SINK_LINEAR) return fail(FSK_ERR_INVALID, "bad sink_mode");
  if (c.o_dt != FSK_F16 && c.o_dt != FSK_BF16 && c.o_dt != FSK_F32) return fail(FSK_ERR_UNSUPPORTED, "out dtype must be f16, bf16 or f32");
  if (c.kv_dt == FSK_E4M3) {
    if (c.q_dt != FSK_F16 && c.q_dt != FSK_BF16 && !(c.q_dt == FSK_E4M3 && c.layout == FSK_LAYOUT_DENSE))
      return fail(FSK_ERR_UNSUPPORTED, "e4m3 KV needs f16/bf16 q (e4m3 q only on the dense layout)");
    if (!c.k_scale || !c.v_scale) return fail(FSK_ERR_INVALID, "e4m3 KV needs k_scale and v_scale");
  } else if (c.kv_dt == FSK_F16 || c.kv_dt == FSK_BF16) {
    if (c.q_dt != c.kv_dt) return fail(FSK_ERR_UNSUPPORTED, "q and f16/bf16 KV must share a dtype");
  } else {
    return fail(FSK_ERR_UNSUPPORTED, "KV dtype must be f16, bf16 or e4m3");
  }
  if (c.q_dt == FSK_E4M3 && !c.q_scale) return fail(FSK_ERR_INVALID, "e4m3 q needs q_scale");
  if (!(c.sm_scale == c.sm_scale) || !std::isfinite(c.sm_scale)) return fail(FSK_ERR_INVALID, "sm_scale must be finite");
  // Strides (elements) are non-negative and below 2^40, so the byte products
  // below stay inside int64.
  for (const int64_t st : {c.q_sb, c.q_sh, c.k_s0, c.k_sh, c.k_st, c.v_s0, c.v_sh, c.v_st, c.o_sb, c.o_sh, c.bt_sb}) {
    if (st < 0) return fail(FSK_ERR_INVALID, "negative stride");
    if (st >= kMaxStride) return fail(FSK_ERR_UNSUPPORTED, "stride above 2^40 elements");
  }
  const int qe = elem_bytes(c.q_dt), ke = elem_bytes(c.kv_dt), oe = elem_bytes(c.o_dt);
  // Row starts must be 16-byte aligned (8 for e4m3 q) for the vector loads.
  const int qa = (c.q_dt == FSK_E4M3) ? 8 : 16;
  if (!aligned(c.q, qa) || (c.q_sb * qe) % qa || (c.q_sh * qe) % qa) return fail(FSK_ERR_INVALID, "q rows must be 16-byte aligned");
  if (!aligned(c.k, 16) || !aligned(c.v, 16) || (c.k_st * ke) % 16 || (c.v_st * ke) % 16 || (c.k_sh * ke) % 16 ||
      (c.v_sh * ke) % 16 || (c.k_s0 * ke) % 16 || (c.v_s0 * ke) % 16)
    return fail(FSK_ERR_INVALID, "k/v rows must be 16-byte aligned");
  if (c.k_st < c.D || c.v_st < c.D) return fail(FSK_ERR_INVALID, "k/v token stride must be >= head_dim");
  if ((c.k_st * ke) * 16 >= (int64_t)1 << 31 || (c.v_st * ke) * 16 >= (int64_t)1 << 31)
    return fail(FSK_ERR_UNSUPPORTED, "k/v token stride too large");
  if (!aligned(c.out, 4 * oe) || (c.o_sb * oe) % (4 * oe) || (c.o_sh * oe) % (4 * oe))
    return fail(FSK_ERR_INVALID, "out rows must be aligned to 4 elements");
  if (c.kv_extent < 0 || c.kv_extent >= ((int64_t)1 << 31)) return fail(FSK_ERR_UNSUPPORTED, "kv extent out of int32 range");
  if (c.layout == FSK_LAYOUT_PAGED) {
    if (!c.bt) return fail(FSK_ERR_INVALID, "null block_table");
    if (c.page_size <= 0 || c.page_size % 16) return fail(FSK_ERR_UNSUPPORTED, "page_size must be a positive multiple of 16");
    if (c.num_pages <= 0) return fail(FSK_ERR_INVALID, "num_pages must be positive");
    if (c.max_blocks < 0 || c.bt_sb < c.max_blocks) return fail(FSK_ERR_INVALID, "bad block_table shape");
    if ((int64_t)c.max_blocks * c.page_size >= ((int64_t)1 << 31)) return fail(FSK_ERR_UNSUPPORTED, "block table too wide");
  }
  if (c.B > kMaxBatch) return fail(FSK_ERR_UNSUPPORTED, "batch above 16384");
  if (stream_bound(c.layout, c.B, c.kv_extent, c.page_size > 0 ? c.page_size : 16) >= ((int64_t)1 << 31) - 4096)
    return fail(FSK_ERR_UNSUPPORTED, "total token extent of the batch above 2^31");
  if (c.scores) {
    if (c.layout == FSK_LAYOUT_DENSE) return fail(FSK_ERR_UNSUPPORTED, "block scores on the varlen and paged layouts only");
    if (c.nblk <= 0 || c.nblk > (1 << 24)) return fail(FSK_ERR_INVALID, "score_blocks must be in [1, 2^24]");
    if (!aligned(c.scores, elem_bytes(c.o_dt))) return fail(FSK_ERR_INVALID, "scores must be aligned to the output dtype");
    if (c.chunk % 128) return fail(FSK_ERR_INVALID, "with block scores chunk_tokens must be a multiple of 128");
  }
  return FSK_OK;
}

// Stream of a launch, and the events (or null) that the dispatch itself
// timestamps at the kernel's start and end (timing calls only).
struct Launch {
  hipStream_t s;
  hipEvent_t start, stop;
};

template <typename K, typename... Args>
void launch(K kernel, dim3 grid, dim3 block, uint32_t lds, const Launch& L, Args... args) {
  if (L.start || L.stop) hipExtLaunchKernelGGL(kernel, grid, block, lds, L.s, L.start, L.stop, 0, args...);
  else hipLaunchKernelGGL(kernel, grid, block, lds, L.s, args...);
}

template <int D, int kQ, int kKV, int kLayout, bool kScores>
void launch_partial(const Params& p, int grid, const Launch& s) {
  launch(partial_kernel<D, kQ, kKV, kLayout, kScores>, dim3(grid), dim3(64), 8 * (p.B + 1), s, p.lens, p.starts,
         p.B, p);
}

template <int D, int kLayout, bool kScores>
int dispatch_qkv(const Params& p, int grid, int q_dt, int kv_dt, const Launch& s) {
  if (kv_dt == FSK_F16) launch_partial<D, kF16, kF16, kLayout, kScores>(p, grid, s);
  else if (kv_dt == FSK_BF16) launch_partial<D, kBF16, kBF16, kLayout, kScores>(p, grid, s);
  else if (q_dt == FSK_F16) launch_partial<D, kF16, kE4M3, kLayout, kScores>(p, grid, s);
  else if (q_dt == FSK_BF16) launch_partial<D, kBF16, kE4M3, kLayout, kScores>(p, grid, s);
  else if constexpr (kLayout == kDense) launch_partial<D, kE4M3, kE4M3, kLayout, kScores>(p, grid, s);
  else return fail(FSK_ERR_UNSUPPORTED, "e4m3 q only on the dense layout");
  return FSK_OK;
}

template <int D, int kQ, int kKV, int kLayout>
void launch_partial_hp(const Params& p, const HostPlan& hp, int grid, const Launch& s) {
  launch(partial_kernel<D, kQ, kKV, kLayout, false, false, HostPlan>, dim3(grid), dim3(64), 0, s,
         (const int32_t*)nullptr, (const int32_t*)nullptr, p.B, p, hp);
}

template <int D, int kLayout>
int dispatch_qkv_hp(const Params& p, const HostPlan& hp, int grid, int q_dt, int kv_dt, const Launch& s) {
  if (kv_dt == FSK_F16) launch_partial_hp<D, kF16, kF16, kLayout>(p, hp, grid, s);
  else if (kv_dt == FSK_BF16) launch_partial_hp<D, kBF16, kBF16, kLayout>(p, hp, grid, s);
  else if (q_dt == FSK_F16) launch_partial_hp<D, kF16, kE4M3, kLayout>(p, hp, grid, s);
  else if (q_dt == FSK_BF16) launch_partial_hp<D, kBF16, kE4M3, kLayout>(p, hp, grid, s);
  else return fail(FSK_ERR_UNSUPPORTED, "e4m3 q only on the dense layout");
  return FSK_OK;
}

template <int D>
int dispatch_layout_hp(int layout, const Params& p, const HostPlan& hp, int grid, int q_dt, int kv_dt,
                       const Launch& s) {
  return layout == FSK_LAYOUT_VARLEN ? dispatch_qkv_hp<D, kVarlen>(p, hp, grid, q_dt, kv_dt, s)
                                     : dispatch_qkv_hp<D, kPaged>(p, hp, grid, q_dt, kv_dt, s);
}

// The VALU-tile kernels (option qk_engine = 1; f16, D = 128, paged or varlen).
int launch_valu(int layout, const Params& p, int grid, const Launch& s) {
  if (layout == FSK_LAYOUT_PAGED)
    launch(partial_kernel<128, kF16, kF16, kPaged, false, true>, dim3(grid), dim3(64), 8 * (p.B + 1), s, p.lens,
           p.starts, p.B, p);
  else
    launch(partial_kernel<128, kF16, kF16, kVarlen, false, true>, dim3(grid), dim3(64), 8 * (p.B + 1), s, p.lens,
           p.starts, p.B, p);
  return FSK_OK;
}

template <int D>
int dispatch_layout(int layout, bool scores, const Params& p, int grid, int q_dt, int kv_dt, const Launch& s) {
  if (layout == FSK_LAYOUT_VARLEN)
    return scores ? dispatch_qkv<D, kVarlen, true>(p, grid, q_dt, kv_dt, s)
                  : dispatch_qkv<D, kVarlen, false>(p, grid, q_dt, kv_dt, s);
  if (layout == FSK_LAYOUT_PAGED)
    return scores ? dispatch_qkv<D, kPaged, true>(p, grid, q_dt, kv_dt, s)
                  : dispatch_qkv<D, kPaged, false>(p, grid, q_dt, kv_dt, s);
  return dispatch_qkv<D, kDense, false>(p, grid, q_dt, kv_dt, s);
}

template <int D, int kRows>
void launch_reduce_rows(const ReduceParams& rp, int B, int o_dt, const Launch& s) {
  dim3 grid(rp.Hq / kRows, B);
  dim3 block(kReduceThreads);
  if (o_dt == FSK_F16) launch(reduce_kernel<D, kF16, kRows>, grid, block, 0, s, rp);
  else if (o_dt == FSK_BF16) launch(reduce_kernel<D, kBF16, kRows>, grid, block, 0, s, rp);
  else launch(reduce_kernel<D, kF32, kRows>, grid, block, 0, s, rp);
}

// Four query heads per workgroup when the batch has at least twice as many
// sequences as the split has chunks (a few partials per row): a quarter of
// the workgroups, each merging 8 units per round trip and row (D = 128).
template <int D>
void launch_reduce(const ReduceParams& rp, int B, int o_dt, bool rows4, const Launch& s) {
  if (rows4 && rp.Hq % 4 == 0 && !rp.scores) launch_reduce_rows<D, 4>(rp, B, o_dt, s);
  else launch_reduce_rows<D, 1>(rp, B, o_dt, s);
}

FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while (((uint64_t)1 << l) < d) ++l;
  const uint64_t two_s = (uint64_t)1 << (31 + l);
  return FastDiv{d, (uint32_t)((two_s + d - 1) / d), 31 + l};
}

// The split policy's per-call constants (see SplitArgs): target_units <=
// 2^20, chunk bounds <= 2^24, 0 <= u_max < 2^31.
SplitArgs make_split_args(int chunk_min, int chunk_max, int chunk_pref, int target_units, int64_t u_max, int B,
                          int xcd_skew, int head_slots) {
  SplitArgs a;
  const uint64_t lim = (uint64_t)1 << 31;
  a.chunk_min = (uint32_t)chunk_min;
  a.chunk_max = (uint32_t)chunk_max;
  a.pref_total = (uint32_t)std::min<uint64_t>((uint64_t)target_units * (uint64_t)chunk_pref, lim);
  a.max_total = (uint32_t)std::min<uint64_t>((uint64_t)target_units * (uint64_t)chunk_max, lim);
  a.short_units = (uint32_t)std::min<uint64_t>(32 * (uint64_t)std::max(B, 0), 0xFFFFFFFFull);
  const int64_t cap = u_max > (int64_t)B + 1 ? u_max - B - 1 : 0;
  a.cap = (uint32_t)cap;
  a.target = make_fastdiv((uint32_t)target_units);
  a.target_half = make_fastdiv((uint32_t)std::max(target_units / 2, 1));
  a.cap_div = make_fastdiv((uint32_t)std::max<int64_t>(cap, 1));
  a.k_cap = 0;
  while (((uint64_t)target_units << a.k_cap) < ((uint64_t)1 << 24)) ++a.k_cap;
  a.xcd_skew = (uint32_t)xcd_skew;
  a.nh7 = (uint32_t)head_slots & 7;
  return a;
}

// The plan build_plan computes on the device, computed here from host
// lengths (varlen: cu_seqlens [B+1]; paged: seq_lens [B]) with the same
// clamps, split rule (split_geometry, chunk_of) and prefix sums, so a
// host-planned call does exactly what the device-planned one does.
int make_host_plan(const Common& c, const Params& p, HostPlan& hp) {
  if (c.B > kHostPlanMax)
    return fail(FSK_ERR_UNSUPPORTED, "host lengths: at most " + std::to_string(kHostPlanMax) + " sequences a call");
  memset(&hp, 0, sizeof(hp));
  auto clampi = [](int x, int lo, int hi) { return x < lo ? lo : (x > hi ? hi : x); };
  constexpr int kA = 32;  // stream padding of the plain decode kernels
  uint32_t total = 0;     // < 2^31 - 4096: validate bounds the stream
  int nonempty = 0, ref = -1;
  bool varied = false;
  for (int b = 0; b < c.B; ++b) {
    int start = 0, len;
    if (c.layout == FSK_LAYOUT_VARLEN) {
      start = clampi(c.lens[b], 0, p.kv_extent);
      len = clampi(c.lens[b + 1], start, p.kv_extent) - start;
    } else {
      len = clampi(c.lens[b], 0, p.max_blocks * p.page_size);
    }
    hp.start[b] = start;
    hp.len[b] = len;
    total += (uint32_t)((len + kA - 1) / kA * kA);
    if (len > 0) {
      ++nonempty;
      if (ref < 0) ref = len;
      varied = varied || len != ref;
    }
  }
  const uint32_t seg = (uint32_t)p.seg_tokens;
  int X = 0;
  Split sp;
  if (seg > 0 && varied) {
    sp = split_geometry(total + (uint32_t)nonempty * seg, p.split, kA);
    if (sp.n <= 8 * nonempty || (uint32_t)sp.c_e <= seg) X = (int)seg;
    else sp = split_geometry(total, p.split, kA);
  } else {
    sp = split_geometry(total, p.split, kA);
  }
  int carry_f = 0, carry_u = 0;
  for (int b = 0; b < c.B; ++b) {
    const int len = hp.len[b];
    const int fs = carry_f + X;  // the sequence's first token in the stream
    const int n = len > 0 ? chunk_of(sp, fs + len - 1) - chunk_of(sp, fs) + 1 : 0;
    hp.flat[b] = carry_f;
    hp.pre[b] = std::min(carry_u, p.u_max);
    carry_f += (len + kA - 1) / kA * kA + (len > 0 ? X : 0);
    carry_u += n;
  }
  for (int b = c.B; b < kHostPlanMax; ++b) {
    hp.flat[b] = carry_f;
    hp.pre[b] = std::min(carry_u, p.u_max);
  }
  hp.pre_end = std::min(carry_u, p.u_max);
  hp.c_e = sp.c_e; hp.c_o = sp.c_o; hp.n = sp.n; hp.paired = sp.paired; hp.m = sp.m;
  hp.seg_x = X;
  return FSK_OK;
}

int run_decode(const Common& c) {
  int st = validate(c);
  if (st != FSK_OK) return st;
  if (c.B == 0) return FSK_OK;
  const int G = c.Hq / c.Hkv;
  const int n_hb = (G + 15) / 16;
  const int cus = device_cus();
  if (c.chunk % 32 != 0) return fail(FSK_ERR_INVALID, "chunk_tokens must be a multiple of 32");
  const SplitPlan sp = plan_split(c.layout, c.B, plan_heads(c.layout, c.D, c.Hkv, G), c.kv_extent, c.page_size,
                                  c.chunk, cus, elem_bytes(c.kv_dt));
  const bool pair =
      g_opt.head_pairs && pair_shape(c.layout, c.D, c.Hkv, G) && !c.scores && c.k_sh == 64 && c.v_sh == 64;
  if (c.layout == FSK_LAYOUT_PAGED && sp.chunk_max > kChunkMax)
    return fail(FSK_ERR_UNSUPPORTED, "paged decode takes chunk_tokens <= 4096");
  const int64_t u_max = sp.u_max;
  if (u_max >= ((int64_t)1 << 31) / (c.Hkv * (int64_t)n_hb)) return fail(FSK_ERR_UNSUPPORTED, "too many work units");
  const WsLayout wl = ws_layout(c.B, c.Hkv, G, c.D, u_max);
  const int64_t need = wl.total + (c.scores ? score_ws_bytes(c.B, c.Hq, c.nblk) : 0);
  if (!c.ws || c.ws_bytes < need || !aligned(c.ws, 256))
    return fail(FSK_ERR_WORKSPACE, c.scores ? "workspace missing, unaligned or smaller than fsk_workspace_bytes() + "
                                              "fsk_score_workspace_bytes()"
                                            : "workspace missing, unaligned or smaller than fsk_workspace_bytes()");

  const int qe = elem_bytes(c.q_dt), ke = elem_bytes(c.kv_dt), oe = elem_bytes(c.o_dt);
  Params p;
  memset(&p, 0, sizeof(p));
  p.q = (const uint8_t*)c.q;
  p.q_sb = c.q_sb * qe; p.q_sh = c.q_sh * qe;
  p.k = (const uint8_t*)c.k; p.v = (const uint8_t*)c.v;
  p.k_s0 = c.k_s0 * ke; p.k_sh = c.k_sh * ke; p.k_st = c.k_st * ke;
  p.v_s0 = c.v_s0 * ke; p.v_sh = c.v_sh * ke; p.v_st = c.v_st * ke;
  p.lens = c.lens; p.starts = c.starts;
  p.block_table = c.bt; p.bt_sb = c.bt_sb; p.max_blocks = c.max_blocks;
  p.num_pages = c.num_pages; p.page_size = c.page_size > 0 ? c.page_size : 16;
  p.page = make_fastdiv((uint32_t)p.page_size);
  p.kv_extent = (int)c.kv_extent;
  p.q_scale = c.q_scale; p.k_scale = c.k_scale; p.v_scale = c.v_scale;
  p.score_scale = c.sm_scale * kLog2e;
  p.B = c.B; p.Hkv = c.Hkv; p.G = G; p.n_hb = n_hb;
  p.pair = pair ? 1 : 0;
  p.n_items_h = pair ? c.Hkv / 2 : c.Hkv * n_hb;
  p.nh_div = make_fastdiv((uint32_t)p.n_items_h);
  p.hb_div = make_fastdiv((uint32_t)p.n_hb);
  p.hkv_div = make_fastdiv((uint32_t)c.Hkv);
  // The skew is not applied to a fixed split, nor at head_dim 256: there the
  // even and odd XCDs stream at the same rate (16-bit KV: partial kernel
  // 3-4 % slower with it, paged and varlen; e4m3: no difference).
  const int xcd_skew = (sp.chunk_min == sp.chunk_max || c.D > 128) ? 0 : g_opt.xcd_skew;
  p.split = make_split_args(sp.chunk_min, sp.chunk_max, sp.chunk_pref, sp.target_units, u_max, c.B, xcd_skew,
                            p.n_items_h);
  p.seg_tokens = g_opt.seg_tokens;
  p.u_max = (int)u_max;
  uint8_t* ws = (uint8_t*)c.ws;
  p.plan = (int32_t*)(ws + wl.plan_off);
  p.part_ml = (float*)(ws + wl.ml_off);
  p.part_acc = (float*)(ws + wl.acc_off);
  if (c.scores) {
    p.nblk = c.nblk;
    p.blk_max = (float*)(ws + wl.total);
    p.lens_out = (int32_t*)(ws + wl.total + align256((int64_t)c.B * c.Hq * c.nblk * 4));
  }

  const bool valu = g_opt.qk_engine == 1;
  if (valu && !(c.D == 128 && c.q_dt == FSK_F16 && c.kv_dt == FSK_F16 && G <= kValuHeads && !c.scores &&
                c.layout != FSK_LAYOUT_DENSE))
    return fail(FSK_ERR_UNSUPPORTED, "qk_engine 1 (VALU tile) covers f16 q and KV, head_dim 128, at most 4 query "
                                     "heads per KV head, the paged and varlen layouts and no block scores");
  HostPlan hp;
  if (c.lens_on_host) {
    if (c.scores || valu || c.layout == FSK_LAYOUT_DENSE)
      return fail(FSK_ERR_UNSUPPORTED, "host lengths: paged and varlen decode without block scores");
    st = make_host_plan(c, p, hp);
    if (st != FSK_OK) return st;
    p.lens = nullptr;  // (host memory: the kernel takes the plan instead)
  }

  // Workgroups that can find a work item: no more than the workspace holds,
  // nor than the split can plan (a grid of 8 per CU for 4 items per CU made
  // C4's decode step ~0.25 µs longer; the other configs were unchanged).
  const int64_t w_max =
      std::min<int64_t>(u_max * c.Hkv * n_hb,
                        chunk_bound(sp.target_units, sp.chunk_pref, sp.chunk_max,
                                    stream_bound(c.layout, c.B, c.kv_extent, p.page_size)) * p.n_items_h);
  const int64_t grid64 = std::min<int64_t>(w_max, (int64_t)cus * g_opt.waves_per_cu);
  const int grid = (int)std::max<int64_t>(grid64, 1);

  (void)hipGetLastError();
  // Timed calls: the partial kernel's dispatch stamps its start and end, the
  // reduce's its end (no separate event records around the launches).
  hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
  if (!c.no_timing) timing_events(ev);
  int rc;
  const bool sc = c.scores != nullptr;
  const Launch lp{c.stream, ev[0], ev[1]};
  if (c.lens_on_host) {
    if (c.D == 64 && !pair) rc = dispatch_layout_hp<64>(c.layout, p, hp, grid, c.q_dt, c.kv_dt, lp);
    else if (c.D <= 128) rc = dispatch_layout_hp<128>(c.layout, p, hp, grid, c.q_dt, c.kv_dt, lp);
    else rc = dispatch_layout_hp<256>(c.layout, p, hp, grid, c.q_dt, c.kv_dt, lp);
  } else if (valu) rc = launch_valu(c.layout, p, grid, lp);
  else if (c.D == 64 && !pair) rc = dispatch_layout<64>(c.layout, sc, p, grid, c.q_dt, c.kv_dt, lp);
  else if (c.D <= 128) rc = dispatch_layout<128>(c.layout, sc, p, grid, c.q_dt, c.kv_dt, lp);
  else rc = dispatch_layout<256>(c.layout, sc, p, grid, c.q_dt, c.kv_dt, lp);
  if (rc != FSK_OK) {
    timing_keep(ev, false);
    return rc;
  }

  ReduceParams rp;
  rp.plan = p.plan; rp.part_ml = p.part_ml; rp.part_acc = p.part_acc;
  rp.s_aux = c.s_aux; rp.sink_mode = c.sink_mode;
  rp.out = (uint8_t*)c.out; rp.o_sb = c.o_sb * oe; rp.o_sh = c.o_sh * oe;
  rp.Hq = c.Hq; rp.Hkv = c.Hkv; rp.G = G;
  rp.blk_max = p.blk_max; rp.lens = p.lens_out; rp.scores = (uint8_t*)c.scores; rp.nblk = c.nblk;
  const Launch lr{c.stream, nullptr, ev[2]};
  const bool rows4 = sp.chunk_min != sp.chunk_max && (int64_t)c.B >= 2 * (int64_t)sp.target_units;
  if (c.D == 64) launch_reduce<64>(rp, c.B, c.o_dt, rows4, lr);
  else if (c.D == 128) launch_reduce<128>(rp, c.B, c.o_dt, rows4, lr);
  else launch_reduce<256>(rp, c.B, c.o_dt, rows4, lr);
  timing_keep(ev, true);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(FSK_ERR_HIP, std::string("kernel launch failed: ") + hipGetErrorString(e));
  return FSK_OK;
}


template <int kSrc, int kPool, bool kScaled>
void launch_write(const WriteParams& p, dim3 grid, const Launch& s) {
  launch(kv_write_kernel<kSrc, kPool, kScaled>, grid, dim3(kWriteThreads), 0, s, p);
}

template <int kSrc>
void dispatch_write(const WriteParams& p, int pool_dt, bool scaled, dim3 grid, const Launch& s) {
  if (pool_dt == FSK_F16) launch_write<kSrc, kF16, false>(p, grid, s);
  else if (pool_dt == FSK_BF16) launch_write<kSrc, kBF16, false>(p, grid, s);
  else if (scaled) launch_write<kSrc, kE4M3, true>(p, grid, s);
  else launch_write<kSrc, kE4M3, false>(p, grid, s);
}

struct WriteArgs {
  const void* src[2]; int64_t s_st[2], s_sh[2];
  const int64_t* slots; int64_t n;
  void* pool[2]; int64_t p_sp[2], p_sh[2], p_st[2];
  int num_pages, page_size, Hkv, D, src_dt, pool_dt;
  const float* scale[2];
  int32_t* bt; int64_t bt_numel; const int64_t* upd; int64_t n_upd;
  hipStream_t stream;
};

int run_write(const WriteArgs& a) {
  if (a.n < 0 || a.n_upd < 0) return fail(FSK_ERR_INVALID, "negative count");
  if (a.n >= ((int64_t)1 << 31)) return fail(FSK_ERR_UNSUPPORTED, "batch too large for one call");
  if (a.Hkv <= 0 || a.D <= 0) return fail(FSK_ERR_INVALID, "num_kv_heads and head_dim must be positive");
  if (a.Hkv > kMaxQHeads) return fail(FSK_ERR_UNSUPPORTED, "num_kv_heads above 65536");
  if (a.D % 8 || a.D > 8 * kWriteThreads) return fail(FSK_ERR_UNSUPPORTED, "head_dim must be a multiple of 8, at most 2048");
  if (a.page_size <= 0 || a.num_pages <= 0) return fail(FSK_ERR_INVALID, "page_size and num_pages must be positive");
  if (a.src_dt != FSK_F16 && a.src_dt != FSK_BF16 && a.src_dt != FSK_F32)
    return fail(FSK_ERR_UNSUPPORTED, "new K/V must be f16, bf16 or f32");
  if (a.pool_dt != FSK_F16 && a.pool_dt != FSK_BF16 && a.pool_dt != FSK_E4M3)
    return fail(FSK_ERR_UNSUPPORTED, "pools must be f16, bf16 or e4m3");
  const bool scaled = a.scale[0] || a.scale[1];
  if (scaled && (!a.scale[0] || !a.scale[1])) return fail(FSK_ERR_INVALID, "pass both k_scale and v_scale or neither");
  if (scaled && a.pool_dt != FSK_E4M3) return fail(FSK_ERR_INVALID, "scales apply to e4m3 pools only");
  if (a.n_upd > 0 && (!a.bt || !a.upd || a.bt_numel <= 0)) return fail(FSK_ERR_INVALID, "block-table updates need block_table");
  if (a.n_upd >= (1 << 30)) return fail(FSK_ERR_UNSUPPORTED, "too many block-table updates");
  const int se = elem_bytes(a.src_dt), pe = elem_bytes(a.pool_dt);
  const int pa = pe == 1 ? 8 : 16;
  for (int kv = 0; kv < 2; ++kv) {
    if (a.n > 0 && (!a.src[kv] || !a.pool[kv])) return fail(FSK_ERR_INVALID, "null tensor pointer");
    for (const int64_t st : {a.s_st[kv], a.s_sh[kv], a.p_sp[kv], a.p_sh[kv], a.p_st[kv]}) {
      if (st < 0) return fail(FSK_ERR_INVALID, "negative stride");
      if (st >= kMaxStride) return fail(FSK_ERR_UNSUPPORTED, "stride above 2^40 elements");
    }
    if (!aligned(a.src[kv], 16) || (a.s_st[kv] * se) % 16 || (a.s_sh[kv] * se) % 16)
      return fail(FSK_ERR_INVALID, "new K/V rows must be 16-byte aligned");
    if (!aligned(a.pool[kv], pa) || (a.p_sp[kv] * pe) % pa || (a.p_sh[kv] * pe) % pa || (a.p_st[kv] * pe) % pa)
      return fail(FSK_ERR_INVALID, "pool rows must be aligned to 8 elements' bytes");
    if (a.page_size > 1 && a.p_st[kv] < a.D) return fail(FSK_ERR_INVALID, "pool row stride must be >= head_dim");
  }
  if (a.n && a.slots == nullptr) return fail(FSK_ERR_INVALID, "null slot_mapping");
  const int64_t total = a.n * a.Hkv * (int64_t)(a.D / 8);  // (< 2^55 with the bounds above)
  if (total >= ((int64_t)1 << 31)) return fail(FSK_ERR_UNSUPPORTED, "batch too large for one call");
  if ((int64_t)a.num_pages * a.page_size >= ((int64_t)1 << 31)) return fail(FSK_ERR_UNSUPPORTED, "pool above 2^31 slots");
  if (total == 0 && a.n_upd == 0) return FSK_OK;

  WriteParams p;
  memset(&p, 0, sizeof(p));
  for (int kv = 0; kv < 2; ++kv) {
    p.src[kv] = (const uint8_t*)a.src[kv];
    p.s_st[kv] = a.s_st[kv] * se; p.s_sh[kv] = a.s_sh[kv] * se;
    p.pool[kv] = (uint8_t*)a.pool[kv];
    p.p_sp[kv] = a.p_sp[kv] * pe; p.p_sh[kv] = a.p_sh[kv] * pe; p.p_st[kv] = a.p_st[kv] * pe;
    p.scale[kv] = a.scale[kv];
  }
  p.slots = a.slots;
  p.n_slots = (uint32_t)((int64_t)a.num_pages * a.page_size);
  p.rows = (uint32_t)(a.n * a.Hkv);
  p.hkv = make_fastdiv((uint32_t)a.Hkv);
  p.page = make_fastdiv((uint32_t)a.page_size);
  p.groups = make_fastdiv((uint32_t)(a.D / 8));
  p.rows_per_block = (uint32_t)(kWriteThreads / (a.D / 8));
  p.bt = a.bt; p.bt_numel = a.bt_numel; p.upd = a.upd; p.n_upd = (int)a.n_upd;
  const int64_t blocks = std::min<int64_t>(std::max<int64_t>(cdiv(p.rows, p.rows_per_block), 1),
                                           (int64_t)device_cus() * FSK_WRITE_BLOCKS_PER_CU);
  const dim3 grid((unsigned)blocks, 2);
  (void)hipGetLastError();
  // Timed calls: the write kernel's dispatch stamps its start and end (the
  // third event, recorded after it, keeps the record in triples).
  hipEvent_t ev[3];
  timing_events(ev);
  const Launch lw{a.stream, ev[0], ev[1]};
  if (a.src_dt == FSK_F16) dispatch_write<kF16>(p, a.pool_dt, scaled, grid, lw);
  else if (a.src_dt == FSK_BF16) dispatch_write<kBF16>(p, a.pool_dt, scaled, grid, lw);
  else dispatch_write<kF32>(p, a.pool_dt, scaled, grid, lw);
  timing_keep(ev, !ev[0] || hipEventRecord(ev[2], a.stream) == hipSuccess);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(FSK_ERR_HIP, std::string("kernel launch failed: ") + hipGetErrorString(e));
  return FSK_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

const char* fsk_last_error(void) { return g_err.c_str(); }

int fsk_version(void) { return 1; }

int fsk_set_option(const char* name, int64_t value) {
  if (!name) return fail(FSK_ERR_INVALID, "null option name");
  if (!strcmp(name, "chunk_tokens")) {
    if (value < 0 || value % 32 || value > (1 << 20)) return fail(FSK_ERR_INVALID, "chunk_tokens: 0 or a multiple of 32");
    g_opt.chunk_tokens = (int)value;
    return FSK_OK;
  }
  if (!strcmp(name, "seg_tokens")) {
    if (value < 0 || value > kSegTokensMax || value % 32)
      return fail(FSK_ERR_INVALID, "seg_tokens: a multiple of 32 in [0, 256]");
    g_opt.seg_tokens = (int)value;
    return FSK_OK;
  }
  if (!strcmp(name, "waves_per_cu")) {
    if (value < 1 || value > 64) return fail(FSK_ERR_INVALID, "waves_per_cu in [1, 64]");
    g_opt.waves_per_cu = (int)value;
    return FSK_OK;
  }
  if (!strcmp(name, "head_pairs")) {
    if (value != 0 && value != 1) return fail(FSK_ERR_INVALID, "head_pairs is 0 or 1");
    g_opt.head_pairs = (int)value;
    return FSK_OK;
  }
  if (!strcmp(name, "qk_engine")) {
    if (value != 0 && value != 1) return fail(FSK_ERR_INVALID, "qk_engine is 0 (MFMA) or 1 (VALU)");
    g_opt.qk_engine = (int)value;
    return FSK_OK;
  }
  if (!strcmp(name, "chunk_pref")) {
    if (value < kChunkMin || value > kChunkMax || value % 128)
      return fail(FSK_ERR_INVALID, "chunk_pref must be a multiple of 128 in [128, 4096]");
    g_opt.chunk_pref = (int)value;
    return FSK_OK;
  }
  if (!strcmp(name, "xcd_skew")) {
    if (value < 0 || value > 50) return fail(FSK_ERR_INVALID, "xcd_skew in [0, 50]");
    g_opt.xcd_skew = (int)value;
    return FSK_OK;
  }
  if (!strcmp(name, "target_waves_per_cu")) {
    if (value < 1 || value > 256) return fail(FSK_ERR_INVALID, "target_waves_per_cu in [1, 256]");
    g_opt.target_waves_per_cu = (int)value;
    return FSK_OK;
  }
  return fail(FSK_ERR_INVALID, std::string("unknown option ") + name);
}

int fsk_enable_kernel_timing(int every_n) {
  if (every_n < 0) return fail(FSK_ERR_INVALID, "every_n must be >= 0");
  timing_clear();
  g_timing.enabled = every_n != 0;
  g_timing.every = every_n > 0 ? every_n : 1;
  g_timing.calls = 0;
  return FSK_OK;
}

int fsk_kernel_timing(double* partial_ms, double* total_ms, int64_t* calls) {
  if (!partial_ms || !total_ms || !calls) return fail(FSK_ERR_INVALID, "null pointer");
  *partial_ms = *total_ms = 0.0;
  *calls = 0;
  const size_t n = g_timing.ev.size() / 3 * 3;
  if (n) {
    hipError_t e = hipEventSynchronize(g_timing.ev[n - 1]);
    if (e != hipSuccess) {
      timing_clear();
      return fail(FSK_ERR_HIP, std::string("hipEventSynchronize: ") + hipGetErrorString(e));
    }
  }
  for (size_t i = 0; i < n; i += 3) {
    float a = 0.f, b = 0.f;
    if (hipEventElapsedTime(&a, g_timing.ev[i], g_timing.ev[i + 1]) != hipSuccess ||
        hipEventElapsedTime(&b, g_timing.ev[i], g_timing.ev[i + 2]) != hipSuccess) {
      timing_clear();
      return fail(FSK_ERR_HIP, "hipEventElapsedTime failed");
    }
    *partial_ms += a;
    *total_ms += b;
    *calls += 1;
  }
  timing_clear();
  return FSK_OK;
}

int64_t fsk_workspace_bytes(int layout, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                            int64_t kv_extent, int page_size, int chunk_tokens) {
  if (layout < 0 || layout > 2) return fail(FSK_ERR_INVALID, "bad layout");
  if (batch < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads || kv_extent < 0)
    return fail(FSK_ERR_INVALID, "bad shape");
  if (num_q_heads > kMaxQHeads) return fail(FSK_ERR_UNSUPPORTED, "num_q_heads above 65536");
  if (batch > kMaxBatch) return fail(FSK_ERR_UNSUPPORTED, "batch above 16384");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return fail(FSK_ERR_UNSUPPORTED, "head_dim must be 64, 128 or 256");
  if (layout == FSK_LAYOUT_PAGED && (page_size <= 0 || page_size % 16)) return fail(FSK_ERR_UNSUPPORTED, "page_size must be a positive multiple of 16");
  if (chunk_tokens % 32) return fail(FSK_ERR_INVALID, "chunk_tokens: a multiple of 32");
  const int G = num_q_heads / num_kv_heads;
  const int B = batch > 0 ? batch : 1;
  // sized for 16-bit KV: the smallest chunk_pref, so the most chunks
  const SplitPlan sp = plan_split(layout, B, plan_heads(layout, head_dim, num_kv_heads, G), kv_extent, page_size,
                                  chunk_tokens, device_cus(), 2);
  const int64_t u_max = sp.u_max;
  return ws_layout(B, num_kv_heads, G, head_dim, u_max).total;
}

int64_t fsk_score_workspace_bytes(int batch, int num_q_heads, int score_blocks) {
  if (batch < 0 || num_q_heads <= 0 || score_blocks <= 0 || score_blocks > (1 << 24))
    return fail(FSK_ERR_INVALID, "bad shape");
  if (num_q_heads > kMaxQHeads) return fail(FSK_ERR_UNSUPPORTED, "num_q_heads above 65536");
  if (batch > kMaxBatch) return fail(FSK_ERR_UNSUPPORTED, "batch above 16384");
  return score_ws_bytes(batch > 0 ? batch : 1, num_q_heads, score_blocks);
}

int fsk_decode_varlen_scores(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k,
                             int64_t k_stride_t, int64_t k_stride_h, const void* v, int64_t v_stride_t,
                             int64_t v_stride_h, const int32_t* cu_seqlens, int64_t total_tokens, const float* s_aux,
                             int sink_mode, const float* k_scale, const float* v_scale, void* out,
                             int64_t o_stride_b, int64_t o_stride_h, int batch, int num_q_heads, int num_kv_heads,
                             int head_dim, int q_dtype, int kv_dtype, int out_dtype, float sm_scale,
                             void* workspace, int64_t workspace_bytes, int chunk_tokens, void* scores,
                             int score_blocks, void* stream) {
  if (!scores) return fail(FSK_ERR_INVALID, "null scores");
  Common c;
  memset(&c, 0, sizeof(c));
  c.layout = FSK_LAYOUT_VARLEN;
  c.q = q; c.q_sb = q_stride_b; c.q_sh = q_stride_h;
  c.k = k; c.k_st = k_stride_t; c.k_sh = k_stride_h;
  c.v = v; c.v_st = v_stride_t; c.v_sh = v_stride_h;
  c.lens = cu_seqlens; c.kv_extent = total_tokens;
  c.s_aux = s_aux; c.sink_mode = sink_mode; c.k_scale = k_scale; c.v_scale = v_scale;
  c.out = out; c.o_sb = o_stride_b; c.o_sh = o_stride_h;
  c.B = batch; c.Hq = num_q_heads; c.Hkv = num_kv_heads; c.D = head_dim;
  c.q_dt = q_dtype; c.kv_dt = kv_dtype; c.o_dt = out_dtype; c.sm_scale = sm_scale;
  c.ws = workspace; c.ws_bytes = workspace_bytes; c.chunk = chunk_tokens; c.stream = (hipStream_t)stream;
  c.scores = scores; c.nblk = score_blocks;
  return run_decode(c);
}

int fsk_decode_paged_scores(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_pool,
                            int64_t k_stride_p, int64_t k_stride_h, int64_t k_stride_t, const void* v_pool,
                            int64_t v_stride_p, int64_t v_stride_h, int64_t v_stride_t, const int32_t* block_table,
                            int64_t bt_stride_b, int max_blocks, const int32_t* seq_lens, int num_pages,
                            int page_size, const float* s_aux, int sink_mode, const float* k_scale,
                            const float* v_scale, void* out, int64_t o_stride_b, int64_t o_stride_h, int batch,
                            int num_q_heads, int num_kv_heads, int head_dim, int q_dtype, int kv_dtype,
                            int out_dtype, float sm_scale, void* workspace, int64_t workspace_bytes,
                            int chunk_tokens, void* scores, int score_blocks, void* stream) {
  if (!scores) return fail(FSK_ERR_INVALID, "null scores");
  Common c;
  memset(&c, 0, sizeof(c));
  c.layout = FSK_LAYOUT_PAGED;
  c.q = q; c.q_sb = q_stride_b; c.q_sh = q_stride_h;
  c.k = k_pool; c.k_s0 = k_stride_p; c.k_sh = k_stride_h; c.k_st = k_stride_t;
  c.v = v_pool; c.v_s0 = v_stride_p; c.v_sh = v_stride_h; c.v_st = v_stride_t;
  c.bt = block_table; c.bt_sb = bt_stride_b; c.max_blocks = max_blocks;
  c.lens = seq_lens; c.num_pages = num_pages; c.page_size = page_size; c.kv_extent = max_blocks;
  c.s_aux = s_aux; c.sink_mode = sink_mode; c.k_scale = k_scale; c.v_scale = v_scale;
  c.out = out; c.o_sb = o_stride_b; c.o_sh = o_stride_h;
  c.B = batch; c.Hq = num_q_heads; c.Hkv = num_kv_heads; c.D = head_dim;
  c.q_dt = q_dtype; c.kv_dt = kv_dtype; c.o_dt = out_dtype; c.sm_scale = sm_scale;
  c.ws = workspace; c.ws_bytes = workspace_bytes; c.chunk = chunk_tokens; c.stream = (hipStream_t)stream;
  c.scores = scores; c.nblk = score_blocks;
  return run_decode(c);
}

}  // extern "C"

namespace {
int decode_varlen(bool host_lens, const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k,
                  int64_t k_stride_t, int64_t k_stride_h, const void* v, int64_t v_stride_t, int64_t v_stride_h,
                  const int32_t* cu_seqlens, int64_t total_tokens, const float* s_aux, int sink_mode,
                  const float* k_scale, const float* v_scale, void* out, int64_t o_stride_b, int64_t o_stride_h,
                  int batch, int num_q_heads, int num_kv_heads, int head_dim, int q_dtype, int kv_dtype,
                  int out_dtype, float sm_scale, void* workspace, int64_t workspace_bytes, int chunk_tokens,
                  void* stream) {
  Common c;
  memset(&c, 0, sizeof(c));
  c.layout = FSK_LAYOUT_VARLEN;
  c.q = q; c.q_sb = q_stride_b; c.q_sh = q_stride_h;
  c.k = k; c.k_st = k_stride_t; c.k_sh = k_stride_h;
  c.v = v; c.v_st = v_stride_t; c.v_sh = v_stride_h;
  c.lens = cu_seqlens; c.kv_extent = total_tokens; c.lens_on_host = host_lens;
  c.s_aux = s_aux; c.sink_mode = sink_mode; c.k_scale = k_scale; c.v_scale = v_scale;
  c.out = out; c.o_sb = o_stride_b; c.o_sh = o_stride_h;
  c.B = batch; c.Hq = num_q_heads; c.Hkv = num_kv_heads; c.D = head_dim;
  c.q_dt = q_dtype; c.kv_dt = kv_dtype; c.o_dt = out_dtype; c.sm_scale = sm_scale;
  c.ws = workspace; c.ws_bytes = workspace_bytes; c.chunk = chunk_tokens; c.stream = (hipStream_t)stream;
  return run_decode(c);
}

int decode_paged(bool host_lens, const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_pool,
                 int64_t k_stride_p, int64_t k_stride_h, int64_t k_stride_t, const void* v_pool, int64_t v_stride_p,
                 int64_t v_stride_h, int64_t v_stride_t, const int32_t* block_table, int64_t bt_stride_b,
                 int max_blocks, const int32_t* seq_lens, int num_pages, int page_size, const float* s_aux,
                 int sink_mode, const float* k_scale, const float* v_scale, void* out, int64_t o_stride_b,
                 int64_t o_stride_h, int batch, int num_q_heads, int num_kv_heads, int head_dim, int q_dtype,
                 int kv_dtype, int out_dtype, float sm_scale, void* workspace, int64_t workspace_bytes,
                 int chunk_tokens, void* stream) {
  Common c;
  memset(&c, 0, sizeof(c));
  c.layout = FSK_LAYOUT_PAGED;
  c.q = q; c.q_sb = q_stride_b; c.q_sh = q_stride_h;
  c.k = k_pool; c.k_s0 = k_stride_p; c.k_sh = k_stride_h; c.k_st = k_stride_t;
  c.v = v_pool; c.v_s0 = v_stride_p; c.v_sh = v_stride_h; c.v_st = v_stride_t;
  c.bt = block_table; c.bt_sb = bt_stride_b; c.max_blocks = max_blocks;
  c.lens = seq_lens; c.num_pages = num_pages; c.page_size = page_size; c.kv_extent = max_blocks;
  c.lens_on_host = host_lens;
  c.s_aux = s_aux; c.sink_mode = sink_mode; c.k_scale = k_scale; c.v_scale = v_scale;
  c.out = out; c.o_sb = o_stride_b; c.o_sh = o_stride_h;
  c.B = batch; c.Hq = num_q_heads; c.Hkv = num_kv_heads; c.D = head_dim;
  c.q_dt = q_dtype; c.kv_dt = kv_dtype; c.o_dt = out_dtype; c.sm_scale = sm_scale;
  c.ws = workspace; c.ws_bytes = workspace_bytes; c.chunk = chunk_tokens; c.stream = (hipStream_t)stream;
  return run_decode(c);
}
}  // namespace

extern "C" {

#define FSK_VARLEN_PARAMS                                                                                          \
  const void *q, int64_t q_stride_b, int64_t q_stride_h, const void *k, int64_t k_stride_t, int64_t k_stride_h,   \
      const void *v, int64_t v_stride_t, int64_t v_stride_h, const int32_t *cu_seqlens, int64_t total_tokens,     \
      const float *s_aux, int sink_mode, const float *k_scale, const float *v_scale, void *out, int64_t o_stride_b, \
      int64_t o_stride_h, int batch, int num_q_heads, int num_kv_heads, int head_dim, int q_dtype, int kv_dtype,   \
      int out_dtype, float sm_scale, void *workspace, int64_t workspace_bytes, int chunk_tokens, void *stream
#define FSK_VARLEN_ARGS                                                                                            \
  q, q_stride_b, q_stride_h, k, k_stride_t, k_stride_h, v, v_stride_t, v_stride_h, cu_seqlens, total_tokens, s_aux, \
      sink_mode, k_scale, v_scale, out, o_stride_b, o_stride_h, batch, num_q_heads, num_kv_heads, head_dim,        \
      q_dtype, kv_dtype, out_dtype, sm_scale, workspace, workspace_bytes, chunk_tokens, stream
#define FSK_PAGED_PARAMS                                                                                           \
  const void *q, int64_t q_stride_b, int64_t q_stride_h, const void *k_pool, int64_t k_stride_p,                  \
      int64_t k_stride_h, int64_t k_stride_t, const void *v_pool, int64_t v_stride_p, int64_t v_stride_h,         \
      int64_t v_stride_t, const int32_t *block_table, int64_t bt_stride_b, int max_blocks, const int32_t *seq_lens, \
      int num_pages, int page_size, const float *s_aux, int sink_mode, const float *k_scale,                      \
      const float *v_scale, void *out, int64_t o_stride_b, int64_t o_stride_h, int batch, int num_q_heads,        \
      int num_kv_heads, int head_dim, int q_dtype, int kv_dtype, int out_dtype, float sm_scale, void *workspace,  \
      int64_t workspace_bytes, int chunk_tokens, void *stream
#define FSK_PAGED_ARGS                                                                                             \
  q, q_stride_b, q_stride_h, k_pool, k_stride_p, k_stride_h, k_stride_t, v_pool, v_stride_p, v_stride_h,          \
      v_stride_t, block_table, bt_stride_b, max_blocks, seq_lens, num_pages, page_size, s_aux, sink_mode, k_scale, \
      v_scale, out, o_stride_b, o_stride_h, batch, num_q_heads, num_kv_heads, head_dim, q_dtype, kv_dtype,         \
      out_dtype, sm_scale, workspace, workspace_bytes, chunk_tokens, stream

int fsk_decode_varlen(FSK_VARLEN_PARAMS) { return decode_varlen(false, FSK_VARLEN_ARGS); }
int fsk_decode_varlen_host(FSK_VARLEN_PARAMS) { return decode_varlen(true, FSK_VARLEN_ARGS); }
int fsk_decode_paged(FSK_PAGED_PARAMS) { return decode_paged(false, FSK_PAGED_ARGS); }
int fsk_decode_paged_host(FSK_PAGED_PARAMS) { return decode_paged(true, FSK_PAGED_ARGS); }

}  // extern "C"

namespace {
// Device address of `scratch` on the current device, looked up once per device
// (with that device current) and kept; null on failure (g_err says why).
std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {nullptr};

void* noalloc_scratch() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    fail(FSK_ERR_HIP, std::string("hipGetDevice: ") + hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= 64) {
    fail(FSK_ERR_UNSUPPORTED, "device index above 63");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      fail(FSK_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}
}  // namespace

extern "C" {

int fsk_decode_paged_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_pool,
                             int64_t k_stride_p, int64_t k_stride_h, int64_t k_stride_t, const void* v_pool,
                             int64_t v_stride_p, int64_t v_stride_h, int64_t v_stride_t,
                             const int32_t* block_table, int64_t bt_stride_b, int max_blocks,
                             const int32_t* seq_lens, int num_pages, int page_size, const float* s_aux,
                             int sink_mode, const float* k_scale, const float* v_scale, void* out,
                             int64_t o_stride_b, int64_t o_stride_h, int batch, int num_q_heads,
                             int num_kv_heads, int head_dim, int q_dtype, int kv_dtype, int out_dtype,
                             float sm_scale, int chunk_tokens, void* stream) {
  // The workspace this call needs, from the same sizing as fsk_workspace_bytes
  // (argument errors are reported by the decode's own validation below).
  const int64_t need = fsk_workspace_bytes(FSK_LAYOUT_PAGED, batch, num_q_heads, num_kv_heads, head_dim,
                                           max_blocks, page_size, chunk_tokens);
  if (need < 0) return (int)need;
  if (need > (int64_t)FSK_NOALLOC_SCRATCH_BYTES)
    return fail(FSK_ERR_UNSUPPORTED, "fsk_decode_paged_noalloc: this call needs " + std::to_string(need) +
                                         " bytes of workspace, above the " +
                                         std::to_string((long long)FSK_NOALLOC_SCRATCH_BYTES) +
                                         "-byte device scratch; use fsk_decode_paged with a workspace");
  void* ws = noalloc_scratch();
  if (!ws) return FSK_ERR_HIP;
  Common c;
  memset(&c, 0, sizeof(c));
  c.layout = FSK_LAYOUT_PAGED;
  c.q = q; c.q_sb = q_stride_b; c.q_sh = q_stride_h;
  c.k = k_pool; c.k_s0 = k_stride_p; c.k_sh = k_stride_h; c.k_st = k_stride_t;
  c.v = v_pool; c.v_s0 = v_stride_p; c.v_sh = v_stride_h; c.v_st = v_stride_t;
  c.bt = block_table; c.bt_sb = bt_stride_b; c.max_blocks = max_blocks;
  c.lens = seq_lens; c.num_pages = num_pages; c.page_size = page_size; c.kv_extent = max_blocks;
  c.s_aux = s_aux; c.sink_mode = sink_mode; c.k_scale = k_scale; c.v_scale = v_scale;
  c.out = out; c.o_sb = o_stride_b; c.o_sh = o_stride_h;
  c.B = batch; c.Hq = num_q_heads; c.Hkv = num_kv_heads; c.D = head_dim;
  c.q_dt = q_dtype; c.kv_dt = kv_dtype; c.o_dt = out_dtype; c.sm_scale = sm_scale;
  c.ws = ws; c.ws_bytes = FSK_NOALLOC_SCRATCH_BYTES; c.chunk = chunk_tokens; c.stream = (hipStream_t)stream;
  c.no_timing = true;
  return run_decode(c);
}

int fsk_decode_dense(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k, int64_t k_stride_b,
                     int64_t k_stride_h, int64_t k_stride_t, const void* v, int64_t v_stride_b, int64_t v_stride_h,
                     int64_t v_stride_t, int64_t max_seqlen, const int32_t* cache_lens,
                     const int32_t* start_offsets, const float* s_aux, int sink_mode, const float* q_scale,
                     const float* k_scale, const float* v_scale, void* out, int64_t o_stride_b,
                     int64_t o_stride_h, int batch, int num_q_heads, int num_kv_heads, int head_dim, int q_dtype,
                     int kv_dtype, int out_dtype, float sm_scale, void* workspace, int64_t workspace_bytes,
                     int chunk_tokens, void* stream) {
  Common c;
  memset(&c, 0, sizeof(c));
  c.layout = FSK_LAYOUT_DENSE;
  c.q = q; c.q_sb = q_stride_b; c.q_sh = q_stride_h;
  c.k = k; c.k_s0 = k_stride_b; c.k_sh = k_stride_h; c.k_st = k_stride_t;
  c.v = v; c.v_s0 = v_stride_b; c.v_sh = v_stride_h; c.v_st = v_stride_t;
  c.kv_extent = max_seqlen; c.lens = cache_lens; c.starts = start_offsets;
  c.s_aux = s_aux; c.sink_mode = sink_mode; c.q_scale = q_scale; c.k_scale = k_scale; c.v_scale = v_scale;
  c.out = out; c.o_sb = o_stride_b; c.o_sh = o_stride_h;
  c.B = batch; c.Hq = num_q_heads; c.Hkv = num_kv_heads; c.D = head_dim;
  c.q_dt = q_dtype; c.kv_dt = kv_dtype; c.o_dt = out_dtype; c.sm_scale = sm_scale;
  c.ws = workspace; c.ws_bytes = workspace_bytes; c.chunk = chunk_tokens; c.stream = (hipStream_t)stream;
  return run_decode(c);
}

int fsk_paged_gather(const void* pool, int64_t stride_p, int64_t stride_h, int64_t stride_t,
                     const int32_t* block_table, int64_t bt_stride_b, int max_blocks, const int32_t* seq_lens,
                     int num_pages, int page_size, int batch, int num_kv_heads, int head_dim, int dtype, void* out,
                     void* stream) {
  if (!pool || !block_table || !seq_lens || !out) return fail(FSK_ERR_INVALID, "null pointer");
  if (batch < 0 || num_kv_heads <= 0 || max_blocks < 0 || num_pages <= 0 || bt_stride_b < max_blocks)
    return fail(FSK_ERR_INVALID, "bad shape");
  if (page_size <= 0 || page_size % 16) return fail(FSK_ERR_UNSUPPORTED, "page_size must be a positive multiple of 16");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return fail(FSK_ERR_UNSUPPORTED, "head_dim must be 64, 128 or 256");
  if (batch > kMaxBatch || num_kv_heads > kMaxQHeads) return fail(FSK_ERR_UNSUPPORTED, "batch or num_kv_heads too large");
  for (const int64_t st : {stride_p, stride_h, stride_t, bt_stride_b}) {
    if (st < 0) return fail(FSK_ERR_INVALID, "negative stride");
    if (st >= kMaxStride) return fail(FSK_ERR_UNSUPPORTED, "stride above 2^40 elements");
  }
  const int e = elem_bytes(dtype);
  if (e != 1 && e != 2) return fail(FSK_ERR_UNSUPPORTED, "dtype must be f16, bf16 or e4m3");
  if (!aligned(pool, 16) || !aligned(out, 16) || (stride_p * e) % 16 || (stride_h * e) % 16 || (stride_t * e) % 16 ||
      stride_t < head_dim)
    return fail(FSK_ERR_INVALID, "pool rows must be 16-byte aligned and non-overlapping");
  if ((int64_t)max_blocks * page_size >= ((int64_t)1 << 31)) return fail(FSK_ERR_UNSUPPORTED, "block table too wide");
  if (batch == 0 || max_blocks == 0) return FSK_OK;
  Params p;
  memset(&p, 0, sizeof(p));
  p.k = p.v = (const uint8_t*)pool;
  p.k_s0 = p.v_s0 = stride_p * e; p.k_sh = p.v_sh = stride_h * e; p.k_st = p.v_st = stride_t * e;
  p.lens = seq_lens; p.block_table = block_table; p.bt_sb = bt_stride_b; p.max_blocks = max_blocks;
  p.num_pages = num_pages; p.page_size = page_size; p.B = batch; p.Hkv = num_kv_heads;
  const int64_t rows = (int64_t)max_blocks * page_size;
  dim3 grid((unsigned)(rows / 16), num_kv_heads, batch);
  hipStream_t s = (hipStream_t)stream;
  (void)hipGetLastError();
  if (e == 2) {
    if (head_dim == 64) hipLaunchKernelGGL((paged_gather_kernel<64, 2>), grid, dim3(64), 0, s, p, (uint8_t*)out, rows);
    else if (head_dim == 128) hipLaunchKernelGGL((paged_gather_kernel<128, 2>), grid, dim3(64), 0, s, p, (uint8_t*)out, rows);
    else hipLaunchKernelGGL((paged_gather_kernel<256, 2>), grid, dim3(64), 0, s, p, (uint8_t*)out, rows);
  } else {
    if (head_dim == 64) hipLaunchKernelGGL((paged_gather_kernel<64, 1>), grid, dim3(64), 0, s, p, (uint8_t*)out, rows);
    else if (head_dim == 128) hipLaunchKernelGGL((paged_gather_kernel<128, 1>), grid, dim3(64), 0, s, p, (uint8_t*)out, rows);
    else hipLaunchKernelGGL((paged_gather_kernel<256, 1>), grid, dim3(64), 0, s, p, (uint8_t*)out, rows);
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(FSK_ERR_HIP, std::string("kernel launch failed: ") + hipGetErrorString(err));
  return FSK_OK;
}

#ifdef FSK_WAVE_STAMPS
int fsk_debug_wave_stamps(uint64_t* out, int waves) {
  if (!out || waves < 0 || waves > kStampWaves) return fail(FSK_ERR_INVALID, "null pointer or waves out of range");
  const hipError_t e = hipMemcpyFromSymbol(out, HIP_SYMBOL(g_wave_stamps), sizeof(uint64_t) * kStampSlots * (size_t)waves);
  if (e != hipSuccess) return fail(FSK_ERR_HIP, std::string("hipMemcpyFromSymbol: ") + hipGetErrorString(e));
  return FSK_OK;
}

int fsk_debug_clear_wave_stamps(void) {
  static const uint64_t zeros[kStampWaves * kStampSlots] = {0};
  const hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(g_wave_stamps), zeros, sizeof(zeros));
  if (e != hipSuccess) return fail(FSK_ERR_HIP, std::string("hipMemcpyToSymbol: ") + hipGetErrorString(e));
  return FSK_OK;
}
#endif

int fsk_fp8_decode_table(uint16_t* out, void* stream) {
  if (!out || !aligned(out, 8)) return fail(FSK_ERR_INVALID, "null or unaligned pointer");
  (void)hipGetLastError();
  hipLaunchKernelGGL(fp8_table_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, (uint32_t*)out);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(FSK_ERR_HIP, std::string("kernel launch failed: ") + hipGetErrorString(err));
  return FSK_OK;
}

int fsk_debug_split(int64_t total, int chunk_min, int chunk_max, int chunk_pref, int target_units, int64_t u_max,
                    int batch, int xcd_skew, int head_slots, int align, int32_t* geometry, int32_t* chunk_start,
                    int32_t* item_chunk, int32_t* item_slot, int32_t* token_chunk) {
  if (!geometry) return fail(FSK_ERR_INVALID, "null geometry");
  if (total < 0 || total >= ((int64_t)1 << 31) - 4096) return fail(FSK_ERR_INVALID, "total out of range");
  if (align != 32 && align != 128) return fail(FSK_ERR_INVALID, "align must be 32 or 128");
  if (chunk_min < 32 || chunk_min % align || chunk_max < chunk_min || chunk_max % align || chunk_max > (1 << 24))
    return fail(FSK_ERR_INVALID, "chunk bounds must be multiples of align with 32 <= chunk_min <= chunk_max");
  if (chunk_pref < chunk_min || chunk_pref > chunk_max)
    return fail(FSK_ERR_INVALID, "chunk_pref must lie in [chunk_min, chunk_max]");
  if (target_units < 1 || target_units > (1 << 20) || u_max < 0 || u_max >= ((int64_t)1 << 31) || batch < 0 || xcd_skew < 0 || xcd_skew > 50 ||
      head_slots < 1 || head_slots > (1 << 16))
    return fail(FSK_ERR_INVALID, "bad split arguments");
  const SplitArgs a =
      make_split_args(chunk_min, chunk_max, chunk_pref, target_units, u_max, batch, xcd_skew, head_slots);
  const Split sp = split_geometry((uint32_t)total, a, (uint32_t)align);
  geometry[0] = sp.c_e;
  geometry[1] = sp.c_o;
  geometry[2] = sp.n;
  geometry[3] = sp.paired;
  if (chunk_start)
    for (int j = 0; j < sp.n; ++j) chunk_start[j] = chunk_lo(sp, j);
  if (item_chunk && item_slot) {
    const int64_t W = (int64_t)sp.n * head_slots;
    if (W >= ((int64_t)1 << 31)) return fail(FSK_ERR_UNSUPPORTED, "too many work items");
    const FastDiv nh = make_fastdiv((uint32_t)head_slots);
    for (int64_t w = 0; w < W; ++w) {
      int jc, hh;
      item_of(sp, (uint32_t)w, nh, jc, hh);
      item_chunk[w] = jc;
      item_slot[w] = hh;
    }
  }
  if (token_chunk)
    for (int64_t x = 0; x < total; ++x) token_chunk[x] = chunk_of(sp, (int)x);
  return FSK_OK;
}

int fsk_paged_write(const void* k_new, int64_t k_stride_t, int64_t k_stride_h, const void* v_new,
                    int64_t v_stride_t, int64_t v_stride_h, const int64_t* slot_mapping, int64_t num_tokens,
                    void* k_pool, int64_t k_stride_p, int64_t kp_stride_h, int64_t kp_stride_t, void* v_pool,
                    int64_t v_stride_p, int64_t vp_stride_h, int64_t vp_stride_t, int num_pages, int page_size,
                    int num_kv_heads, int head_dim, int src_dtype, int pool_dtype, const float* k_scale,
                    const float* v_scale, int32_t* block_table, int64_t bt_numel, const int64_t* bt_updates,
                    int64_t num_bt_updates, void* stream) {
  WriteArgs a;
  memset(&a, 0, sizeof(a));
  a.src[0] = k_new; a.s_st[0] = k_stride_t; a.s_sh[0] = k_stride_h;
  a.src[1] = v_new; a.s_st[1] = v_stride_t; a.s_sh[1] = v_stride_h;
  a.slots = slot_mapping; a.n = num_tokens;
  a.pool[0] = k_pool; a.p_sp[0] = k_stride_p; a.p_sh[0] = kp_stride_h; a.p_st[0] = kp_stride_t;
  a.pool[1] = v_pool; a.p_sp[1] = v_stride_p; a.p_sh[1] = vp_stride_h; a.p_st[1] = vp_stride_t;
  a.num_pages = num_pages; a.page_size = page_size; a.Hkv = num_kv_heads; a.D = head_dim;
  a.src_dt = src_dtype; a.pool_dt = pool_dtype; a.scale[0] = k_scale; a.scale[1] = v_scale;
  a.bt = block_table; a.bt_numel = bt_numel; a.upd = bt_updates; a.n_upd = num_bt_updates;
  a.stream = (hipStream_t)stream;
  return run_write(a);
}

}  // extern "C"
