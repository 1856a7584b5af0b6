/*
 * fsk_decode.h -- C ABI of the MI355X (gfx950) GQA flash-decode library.
 *
 * One query token per sequence attends over that sequence's KV cache.  Query
 * head h reads KV head h / (num_q_heads / num_kv_heads).  Three KV layouts are
 * supported, each with fp16 / bf16 / fp8-e4m3 KV:
 *
 *   varlen : k[T, Hkv, D], sequence b owns rows [cu_seqlens[b], cu_seqlens[b+1])
 *   paged  : k_pool[P, Hkv, page_size, D], token t of sequence b lives in page
 *            block_table[b, t / page_size] at row t % page_size
 *   dense  : k[B, Hkv, S_max, D], sequence b attends rows
 *            [start_offsets[b], cache_lens[b])
 *
 * Every entry point validates its arguments on the host before any HIP call,
 * returns FSK_OK (0) or a negative status, and keeps a thread-local message
 * readable through fsk_last_error().  The library never allocates device
 * memory in these entry points: outputs and the split-KV workspace are passed
 * in (size it with fsk_workspace_bytes).  Work is enqueued on `stream` without
 * host synchronisation, so every call can be captured into a HIP graph.
 *
 * Strides are in ELEMENTS of the tensor they describe; the innermost (head_dim)
 * stride must be 1.  Lengths, offsets, block tables and scales are read on the
 * device; out-of-range values are clamped so that no access leaves the tensors
 * described by the sizes passed here.
 */
#ifndef FSK_DECODE_H
#define FSK_DECODE_H

#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define FSK_API __attribute__((visibility("default")))
#else
#define FSK_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define FSK_OK 0
#define FSK_ERR_INVALID (-1)     /* bad argument: null pointer, shape, stride */
#define FSK_ERR_UNSUPPORTED (-2) /* valid but not implemented (head_dim, dtype) */
#define FSK_ERR_WORKSPACE (-3)   /* workspace missing or too small */
#define FSK_ERR_HIP (-4)         /* HIP runtime error at launch */

/* Element types. */
#define FSK_F16 0
#define FSK_BF16 1
#define FSK_F32 2
#define FSK_E4M3 3 /* OCP float8 e4m3fn (torch.float8_e4m3fn) */

/* Sink folding.  With s = q.k * sm_scale over the sequence and a per-q-head
 * sink value z:
 *   FSK_SINK_EXP    : out = sum_t e^{s_t} v_t / (sum_t e^{s_t} + e^{z})
 *                     (z is an extra logit with a zero value vector; the
 *                     semantics of the reference's test oracles)
 *   FSK_SINK_LINEAR : out = sum_t e^{s_t - m} v_t / (sum_t e^{s_t - m} + z),
 *                     m = max_t s_t (the fold done by the reference kernels)
 */
#define FSK_SINK_EXP 0
#define FSK_SINK_LINEAR 1

/* KV layouts (argument of fsk_workspace_bytes). */
#define FSK_LAYOUT_VARLEN 0
#define FSK_LAYOUT_PAGED 1
#define FSK_LAYOUT_DENSE 2

/* Message of the last failed call on this thread ("" if none). */
FSK_API const char *fsk_last_error(void);

/* Library ABI version, currently 1. */
FSK_API int fsk_version(void);

/* Bytes of device workspace a decode call needs.
 *   kv_extent: varlen -> total rows T of k/v;
 *              paged  -> block_table width (max blocks per sequence);
 *              dense  -> S_max (dim 2 of the cache).
 *   page_size: paged layout only (ignored otherwise).
 *   chunk_tokens: a multiple of 32: > 0 a fixed split size in tokens, 0 the
 *              split the library picks for this shape, < 0 that automatic
 *              split with chunks of at most -chunk_tokens tokens (the dense
 *              entry points' split-count hint).  The decode entry points take
 *              the same values.
 * Returns the byte count (> 0) or a negative status. */
FSK_API int64_t fsk_workspace_bytes(int layout, int batch, int num_q_heads, int num_kv_heads,
                            int head_dim, int64_t kv_extent, int page_size,
                            int chunk_tokens);

/* Varlen GQA decode.
 * Replaces: fskernels/triton/triton_gqa_decode.py:126-155 (flash_decode_gqa_varlen
 *           + _flash_decode_gqa_varlen_kernel launch, :142-154) and
 *           fskernels/cuda/flash_decode_cuda.cu:168-188 (launch_flash_decode_gqa).
 * q [B, Hq, D], k/v [T, Hkv, D], cu_seqlens int32 [B+1], s_aux fp32 [Hq] or
 * NULL, out [B, Hq, D].  k/v may be fp16, bf16 or e4m3 (then k_scale/v_scale are
 * device fp32 scalars, dequantised value = code * scale). */
FSK_API int fsk_decode_varlen(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                      const void *k, int64_t k_stride_t, int64_t k_stride_h,
                      const void *v, int64_t v_stride_t, int64_t v_stride_h,
                      const int32_t *cu_seqlens, int64_t total_tokens,
                      const float *s_aux, int sink_mode,
                      const float *k_scale, const float *v_scale,
                      void *out, int64_t o_stride_b, int64_t o_stride_h,
                      int batch, int num_q_heads, int num_kv_heads, int head_dim,
                      int q_dtype, int kv_dtype, int out_dtype, float sm_scale,
                      void *workspace, int64_t workspace_bytes, int chunk_tokens,
                      void *stream);

/* Paged GQA decode.
 * Replaces: fskernels/paged_attn/triton_paged_attn.py:96-125 (paged_flash_decode
 *           + _paged_flash_decode_kernel launch, :112-124).
 * k_pool/v_pool [P, Hkv, page_size, D] (a per-layer view of PagedKVCache's
 * pools, fskernels/paged_attn/paged_kv_cache.py:46-51), block_table int32
 * [B, max_blocks] (row stride bt_stride_b), seq_lens int32 [B].  page_size must
 * be a multiple of 16. */
FSK_API int fsk_decode_paged(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                     const void *k_pool, int64_t k_stride_p, int64_t k_stride_h,
                     int64_t k_stride_t,
                     const void *v_pool, int64_t v_stride_p, int64_t v_stride_h,
                     int64_t v_stride_t,
                     const int32_t *block_table, int64_t bt_stride_b, int max_blocks,
                     const int32_t *seq_lens, int num_pages, int page_size,
                     const float *s_aux, int sink_mode,
                     const float *k_scale, const float *v_scale,
                     void *out, int64_t o_stride_b, int64_t o_stride_h,
                     int batch, int num_q_heads, int num_kv_heads, int head_dim,
                     int q_dtype, int kv_dtype, int out_dtype, float sm_scale,
                     void *workspace, int64_t workspace_bytes, int chunk_tokens,
                     void *stream);

/* Varlen and paged decode with the lengths in host memory: cu_seqlens
 * (int32 [B+1]) / seq_lens (int32 [B]) are HOST pointers, read during the
 * call; everything else as fsk_decode_varlen / fsk_decode_paged, with the
 * same results bit for bit.  The work plan that the device-length entry
 * points build on the GPU from the lengths (a memory round trip and the
 * split's arithmetic at the start of every workgroup) is built here on the
 * host and passed in the kernel arguments.  For callers that already hold
 * the lengths on the host: a serving loop (PagedKVCache keeps them, as the
 * reference's does, fskernels/paged_attn/paged_kv_cache.py:59, :139-141),
 * and the reference's own varlen bindings, which copy cu_seqlens to the host
 * on every call (fskernels/cuda/flash_decode_api.cpp:22,
 * fskernels/triton/triton_gqa_decode.py:135).  No block scores; at most 64
 * sequences (FSK_ERR_UNSUPPORTED beyond).  Under HIP-graph capture the plan
 * is captured with the call: a replay decodes the captured lengths. */
FSK_API int fsk_decode_varlen_host(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                      const void *k, int64_t k_stride_t, int64_t k_stride_h,
                      const void *v, int64_t v_stride_t, int64_t v_stride_h,
                      const int32_t *cu_seqlens, int64_t total_tokens,
                      const float *s_aux, int sink_mode,
                      const float *k_scale, const float *v_scale,
                      void *out, int64_t o_stride_b, int64_t o_stride_h,
                      int batch, int num_q_heads, int num_kv_heads, int head_dim,
                      int q_dtype, int kv_dtype, int out_dtype, float sm_scale,
                      void *workspace, int64_t workspace_bytes, int chunk_tokens,
                      void *stream);
FSK_API int fsk_decode_paged_host(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                     const void *k_pool, int64_t k_stride_p, int64_t k_stride_h,
                     int64_t k_stride_t,
                     const void *v_pool, int64_t v_stride_p, int64_t v_stride_h,
                     int64_t v_stride_t,
                     const int32_t *block_table, int64_t bt_stride_b, int max_blocks,
                     const int32_t *seq_lens, int num_pages, int page_size,
                     const float *s_aux, int sink_mode,
                     const float *k_scale, const float *v_scale,
                     void *out, int64_t o_stride_b, int64_t o_stride_h,
                     int batch, int num_q_heads, int num_kv_heads, int head_dim,
                     int q_dtype, int kv_dtype, int out_dtype, float sm_scale,
                     void *workspace, int64_t workspace_bytes, int chunk_tokens,
                     void *stream);
#define FSK_HOST_PLAN_MAX_BATCH 64

/* Allocation-free paged decode.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP-graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments and
 * results as fsk_decode_paged, without workspace / workspace_bytes: the
 * workspace is a device array of FSK_NOALLOC_SCRATCH_BYTES bytes inside the
 * library's GPU code object.  It is allocated with that code object, so every
 * device on which any kernel of this library has been loaded holds it (also
 * in processes that never call this entry point), until the process ends.
 * The first call on a device looks up the array's address on that device
 * (hipGetSymbolAddress) and keeps it; that call and all later ones may run
 * under HIP-graph capture.  The call allocates nothing and frees nothing.
 * It returns FSK_ERR_UNSUPPORTED, launching nothing, when the shape needs
 * more workspace than that (fsk_workspace_bytes(FSK_LAYOUT_PAGED, ...) tells
 * how much; the M0 shape, B=4 x 32768 tokens, Hq=32, Hkv=8, D=128, needs
 * 8,519,936 bytes, 8.5 MB).  Every call on one device shares that device's array:
 * calls that overlap on one device (two streams, two threads, or two entries
 * of one graph that may run concurrently) race and give wrong results;
 * serialise them.  Nothing in the array needs to start at zero (each call
 * writes its plan and every partial its reduce reads), so no clearing is
 * issued. */
#define FSK_NOALLOC_SCRATCH_BYTES (32ll << 20)
FSK_API int fsk_decode_paged_noalloc(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                     const void *k_pool, int64_t k_stride_p, int64_t k_stride_h,
                     int64_t k_stride_t,
                     const void *v_pool, int64_t v_stride_p, int64_t v_stride_h,
                     int64_t v_stride_t,
                     const int32_t *block_table, int64_t bt_stride_b, int max_blocks,
                     const int32_t *seq_lens, int num_pages, int page_size,
                     const float *s_aux, int sink_mode,
                     const float *k_scale, const float *v_scale,
                     void *out, int64_t o_stride_b, int64_t o_stride_h,
                     int batch, int num_q_heads, int num_kv_heads, int head_dim,
                     int q_dtype, int kv_dtype, int out_dtype, float sm_scale,
                     int chunk_tokens, void *stream);

/* Block scores: the varlen / paged decode plus, per sequence b, query head h
 * and 128-token block j of the sequence, the largest final attention
 * probability of a token of that block:
 *   S[b, h, j] = max_{t in [128 j, 128 j + 128) and t < len_b} p_t,
 * p_t = softmax weight of token t (the sink folded into the denominator as
 * sink_mode says); S = 0 for blocks at or past the sequence end.
 * Replaces: the S output of fskernels/tilelang/tilelang_gqa_decode.py:40-132
 *           (block maxima :102-103, normalised :123-124, stored :129-130),
 *           which that module's flash_decode_gqa_varlen computes and drops (:170).
 * scores: [B, Hq, score_blocks] contiguous, in out_dtype; blocks past
 * score_blocks are not stored.  The workspace must hold
 * fsk_workspace_bytes(...) + fsk_score_workspace_bytes(B, Hq, score_blocks)
 * bytes, and a nonzero chunk_tokens must be a multiple of 128.  Other
 * arguments as fsk_decode_varlen / fsk_decode_paged. */
FSK_API int64_t fsk_score_workspace_bytes(int batch, int num_q_heads, int score_blocks);
FSK_API int fsk_decode_varlen_scores(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                      const void *k, int64_t k_stride_t, int64_t k_stride_h,
                      const void *v, int64_t v_stride_t, int64_t v_stride_h,
                      const int32_t *cu_seqlens, int64_t total_tokens,
                      const float *s_aux, int sink_mode,
                      const float *k_scale, const float *v_scale,
                      void *out, int64_t o_stride_b, int64_t o_stride_h,
                      int batch, int num_q_heads, int num_kv_heads, int head_dim,
                      int q_dtype, int kv_dtype, int out_dtype, float sm_scale,
                      void *workspace, int64_t workspace_bytes, int chunk_tokens,
                      void *scores, int score_blocks, void *stream);
FSK_API int fsk_decode_paged_scores(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                     const void *k_pool, int64_t k_stride_p, int64_t k_stride_h,
                     int64_t k_stride_t,
                     const void *v_pool, int64_t v_stride_p, int64_t v_stride_h,
                     int64_t v_stride_t,
                     const int32_t *block_table, int64_t bt_stride_b, int max_blocks,
                     const int32_t *seq_lens, int num_pages, int page_size,
                     const float *s_aux, int sink_mode,
                     const float *k_scale, const float *v_scale,
                     void *out, int64_t o_stride_b, int64_t o_stride_h,
                     int batch, int num_q_heads, int num_kv_heads, int head_dim,
                     int q_dtype, int kv_dtype, int out_dtype, float sm_scale,
                     void *workspace, int64_t workspace_bytes, int chunk_tokens,
                     void *scores, int score_blocks, void *stream);

/* Dense (HF static cache) GQA decode.
 * Replaces: fskernels/triton/triton_gqa_decode_hf.py:146-211
 *           (flash_decode_gqa_hf_dense_optimized: partial :186-199 + reduce
 *           :201-209) and fskernels/triton/triton_gqa_decode_hf_fp8.py:164-227
 *           (flash_decode_gqa_hf_fp8; q_dtype FSK_E4M3 with q_scale reproduces
 *           its q = fp16(fp32(q8) * scale_q), :47-50).
 * k/v [B, Hkv, S_max, D]; cache_lens int32 [B]; start_offsets int32 [B] or
 * NULL (all zero). */
FSK_API int fsk_decode_dense(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                     const void *k, int64_t k_stride_b, int64_t k_stride_h,
                     int64_t k_stride_t,
                     const void *v, int64_t v_stride_b, int64_t v_stride_h,
                     int64_t v_stride_t, int64_t max_seqlen,
                     const int32_t *cache_lens, const int32_t *start_offsets,
                     const float *s_aux, int sink_mode, const float *q_scale,
                     const float *k_scale, const float *v_scale,
                     void *out, int64_t o_stride_b, int64_t o_stride_h,
                     int batch, int num_q_heads, int num_kv_heads, int head_dim,
                     int q_dtype, int kv_dtype, int out_dtype, float sm_scale,
                     void *workspace, int64_t workspace_bytes, int chunk_tokens,
                     void *stream);

/* KV write path: store a batch of new tokens' K/V into the page pools.
 * Replaces: fskernels/paged_attn/paged_kv_cache.py:109-132 (PagedKVCache.append_kv:
 *           block-table store :122-124 and the two indexed row copies :129-130),
 *           batched over tokens and fused into one launch.
 * k_new/v_new [n, Hkv, D] (token stride, head stride; head_dim contiguous,
 * 16-byte aligned rows) in f16, bf16 or f32.  slot_mapping int64 [n]: token i
 * is written to page slot_mapping[i] / page_size, row slot_mapping[i] %
 * page_size, of every head; a negative slot or one >= num_pages * page_size
 * skips the token.  Pools [P, Hkv, page_size, D] in f16, bf16 or e4m3:
 *   - f16/bf16 pools: the source is copied (same dtype: bit-exact) or cast
 *     with round-to-nearest-even;
 *   - e4m3 pools with k_scale/v_scale (device fp32 scalars, finite and > 0):
 *     code = e4m3(clamp(x / scale, -448, 448)), the quantiser of
 *     fskernels/triton/triton_gqa_decode_hf_fp8.py:13-16 with a fixed scale;
 *   - e4m3 pools without scales: a plain e4m3fn cast (|x| > 464 -> NaN).
 *   NaN inputs encode as 0x7F | sign, like torch's float8_e4m3fn cast.
 * Optionally the same launch stores block-table entries:
 * block_table[bt_updates[2j]] = (int32)bt_updates[2j+1] for j < num_bt_updates
 * (flat element indices; indices outside [0, bt_numel) are skipped).  The
 * writes are ordered before later work on `stream`; tokens that share a slot
 * race. */
FSK_API int fsk_paged_write(const void *k_new, int64_t k_stride_t, int64_t k_stride_h,
                    const void *v_new, int64_t v_stride_t, int64_t v_stride_h,
                    const int64_t *slot_mapping, int64_t num_tokens,
                    void *k_pool, int64_t k_stride_p, int64_t k_stride_h_pool,
                    int64_t k_stride_t_pool,
                    void *v_pool, int64_t v_stride_p, int64_t v_stride_h_pool,
                    int64_t v_stride_t_pool,
                    int num_pages, int page_size, int num_kv_heads, int head_dim,
                    int src_dtype, int pool_dtype,
                    const float *k_scale, const float *v_scale,
                    int32_t *block_table, int64_t bt_numel,
                    const int64_t *bt_updates, int64_t num_bt_updates,
                    void *stream);

/* Debug: gather a paged pool into a dense [B, Hkv, max_blocks*page_size, D]
 * tensor through the decode kernels' own page-addressing routine; rows at or
 * past seq_lens[b] are written as zero.  Bit-exact copy of the element bytes.
 * Checks the page-addressing contract of
 * fskernels/paged_attn/triton_paged_attn.py:57-69. */
FSK_API int fsk_paged_gather(const void *pool, int64_t stride_p, int64_t stride_h,
                     int64_t stride_t, const int32_t *block_table,
                     int64_t bt_stride_b, int max_blocks, const int32_t *seq_lens,
                     int num_pages, int page_size, int batch, int num_kv_heads,
                     int head_dim, int dtype, void *out, void *stream);

/* Debug: decode all 256 e4m3 codes with the kernels' in-register dequant
 * routines and store the raw 16-bit results.  out[0..255]: fp16 bit pattern
 * of code i; out[256..511]: bf16 bit pattern of code i (out 8-byte aligned).
 * Widened to fp32 on the host, both must equal the e4m3fn -> fp32 cast the
 * reference relies on (fskernels/triton/triton_gqa_decode_hf_fp8.py:71-73,
 * :90-92). */
FSK_API int fsk_fp8_decode_table(uint16_t *out, void *stream);

/* Debug: the chunk geometry and work-item mapping of the decode kernels'
 * device-side plan, computed on the host by the same functions, for a stream
 * of `total` padded tokens (each sequence padded to `align` = 32, or 128 with
 * block scores).  chunk_min / chunk_max / chunk_pref / target_units / u_max /
 * xcd_skew are the split policy a decode call passes to its kernel; head_slots = work items
 * per chunk.  geometry[0..3] = long chunk, short chunk (equal without an XCD
 * skew), chunk count n, XCD pairing flag.  Optional outputs (null to skip):
 * chunk_start[n]; item_chunk[n * head_slots] and item_slot[...] (the chunk
 * and head slot of work item w); token_chunk[total] (the chunk holding
 * stream position x).  No GPU needed.  The split follows the reference's
 * split-KV partition (fskernels/triton/triton_gqa_decode_hf.py:52-54), with
 * the chunk count chosen for this GPU. */
FSK_API int fsk_debug_split(int64_t total, int chunk_min, int chunk_max,
                            int chunk_pref, int target_units, int64_t u_max,
                            int batch,
                            int xcd_skew, int head_slots, int align,
                            int32_t *geometry, int32_t *chunk_start,
                            int32_t *item_chunk, int32_t *item_slot,
                            int32_t *token_chunk);

/* Tuning knobs for benchmarking sweeps:
 *   "chunk_tokens"        fixed split size in tokens (0: chosen on the device)
 *   "waves_per_cu"        largest persistent grid, workgroups per CU (default
 *                         8; the grid also stops at the work items the split
 *                         can plan)
 *   "target_waves_per_cu" automatic split: units of work per CU (default 4)
 *   "xcd_skew"            automatic split: extra share of the even XCDs, in %
 *                         (0..50, default 3; 0 = equal chunks; not applied at
 *                         head_dim 256, nor to a fixed chunk_tokens split)
 *   "chunk_pref"          automatic split: chunks longer than this many
 *                         tokens of 16-bit KV (twice as many of e4m3) make
 *                         the chunk count double once (multiple of 128 in
 *                         128..4096, default 2432)
 *   "seg_tokens"          work-stream positions laid before each sequence when
 *                         non-empty lengths differ and there are at most 8
 *                         chunks per sequence or the chunks are no longer
 *                         than this, so that items holding a sequence
 *                         boundary carry fewer tokens (multiple of 32 in
 *                         0..256, default 96; 0 = none)
 *   "head_pairs"          1 (default): varlen decodes at head_dim 64 with
 *                         packed heads read KV heads 2i and 2i+1 as one
 *                         128-wide row; 0: one KV head per wave
 *   "qk_engine"           0 (default): QK and PV on the matrix cores (MFMA);
 *                         1: the VALU formulation of the tile, for A/B
 *                         measurement (f16 q and KV, head_dim 128, at most 4
 *                         query heads per KV head, paged and varlen layouts,
 *                         no block scores; other calls return
 *                         FSK_ERR_UNSUPPORTED)
 * The options are process-wide and not synchronised: set them before
 * decoding from several threads.  Returns FSK_OK or FSK_ERR_INVALID for an
 * unknown name or bad value. */
FSK_API int fsk_set_option(const char *name, int64_t value);

/* Profiling hook (no counterpart in the reference; used by the benchmark;
 * process-wide, for one thread at a time).
 * With every_n > 0, every n-th decode or write call launches its kernels with
 * HIP events that the dispatches stamp (hipExtLaunchKernel): for a decode,
 * the split-KV partial kernel's start and end and the reduce kernel's end;
 * for a write, the write kernel's start and end.  every_n = 0 disables the
 * hook.  A timed launch costs ~20 us of extra host time, so time steps with
 * the hook off.  Not for use under HIP graph capture.  fsk_kernel_timing()
 * waits for the recorded events, returns the summed first-kernel and
 * first-kernel-start-to-last-kernel-end milliseconds and the number of
 * recorded calls, and clears the record. */
FSK_API int fsk_enable_kernel_timing(int every_n);
FSK_API int fsk_kernel_timing(double *partial_ms, double *total_ms, int64_t *calls);

/* Instrumented builds only (libfsk_decode_stamps.so, compiled with
 * -DFSK_WAVE_STAMPS; bench.py --wave-stamps): the partial kernel's per-wave
 * timeline of the last decode call.  out receives 16 uint64 per workgroup w
 * < waves: s_memrealtime (100 MHz) at the wave's start, plan done, first tile
 * in registers, last epilogue issued and exit (0 where a stage did not
 * happen), the number of segments processed, the XCC id, the HW_ID register,
 * and (paged) the first item's page-window and Q loads issued and arrived;
 * slots 10-15 are unused.  No reference counterpart (measurement only). */
#ifdef FSK_WAVE_STAMPS
FSK_API int fsk_debug_wave_stamps(uint64_t *out, int waves);
FSK_API int fsk_debug_clear_wave_stamps(void);
#endif

#ifdef __cplusplus
}
#endif

#endif /* FSK_DECODE_H */
