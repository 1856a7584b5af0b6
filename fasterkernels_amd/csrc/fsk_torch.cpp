// fsk_torch.cpp -- torch-tensor binding of libfsk_decode.so (Python module
// fasterkernels_amd._fsk_torch).
//
// A decode or KV-write call crosses from Python to C++ once.  The tensor
// checks (device, rank, dtype, shapes), the packed copies a strided input
// needs, the output and workspace allocations (torch's caching allocator)
// and the C-ABI call all happen here, so that a small decode costs its two
// kernel launches plus a few microseconds of host work.  The C ABI
// (include/fsk_decode.h) validates every argument itself.  Both the checks
// here and its status codes raise the exceptions the Python entry points
// document: ValueError for a bad argument, NotImplementedError for an
// unsupported case, RuntimeError for a tensor off the GPU or a HIP failure.
//
// The caller passes the HIP stream handle (torch's current stream of the
// tensors' device); the device guard makes that device current for the call.
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>

#include <cmath>
#include <cstdint>
#include <string>

#include "fsk_decode.h"

namespace {

// A failure with a library status code (or kRuntime / kType for checks of the
// binding itself), raised as the matching Python exception.
struct FskFailure {
  int code;
  std::string msg;
};
constexpr int kRuntime = -100;  // RuntimeError (tensor off the GPU, wrong device)

[[noreturn]] void raise(int code, const std::string& msg) { throw FskFailure{code, msg}; }

void check(int status) {
  if (status != FSK_OK) raise(status, fsk_last_error());
}

std::string shape_str(const at::Tensor& t) {
  std::string s = "(";
  for (int64_t i = 0; i < t.dim(); ++i) s += (i ? ", " : "") + std::to_string(t.size(i));
  return s + (t.dim() == 1 ? ",)" : ")");
}

int dtype_code(at::ScalarType t, const char* name) {
  switch (t) {
    case at::kHalf: return FSK_F16;
    case at::kBFloat16: return FSK_BF16;
    case at::kFloat: return FSK_F32;
    case at::kFloat8_e4m3fn: return FSK_E4M3;
    default: raise(FSK_ERR_UNSUPPORTED, std::string(name) + ": unsupported dtype " + c10::toString(t));
  }
}

at::ScalarType code_dtype(int64_t code) {
  switch (code) {
    case FSK_F16: return at::kHalf;
    case FSK_BF16: return at::kBFloat16;
    case FSK_F32: return at::kFloat;
    case FSK_E4M3: return at::kFloat8_e4m3fn;
    default: raise(FSK_ERR_UNSUPPORTED, "unsupported output dtype code " + std::to_string(code));
  }
}

void on_gpu(const at::Tensor& t, const char* name) {
  if (!t.defined()) raise(FSK_ERR_INVALID, std::string(name) + " is undefined");
  if (!t.is_cuda()) raise(kRuntime, std::string(name) + " must be on a GPU (HIP) device");
}

void on_device(const at::Tensor& t, const char* name, const c10::Device& dev) {
  on_gpu(t, name);
  if (t.device() != dev)
    raise(kRuntime, std::string(name) + " is on " + t.device().str() + ", expected " + dev.str());
}

// The tensor itself when its innermost dim is contiguous and every row starts
// 16-byte aligned (what the kernels' vector loads need), else a packed copy.
at::Tensor rows16(const at::Tensor& t) {
  const int64_t es = t.element_size();
  bool ok = t.stride(-1) == 1 && reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0;
  for (int64_t i = 0; ok && i + 1 < t.dim(); ++i) ok = (t.stride(i) * es) % 16 == 0;
  return ok ? t : t.contiguous();
}

at::Tensor int32_contig(const at::Tensor& t, const char* name, const c10::Device& dev) {
  on_device(t, name, dev);
  if (t.scalar_type() == at::kInt && t.is_contiguous()) return t;
  return t.to(at::kInt).contiguous();
}

const void* ptr_or_null(const c10::optional<at::Tensor>& t) { return t && t->defined() ? t->data_ptr() : nullptr; }

// Sequence lengths: a device tensor, or host memory (then the work plan is
// built on the host: the *_host entry points).  Host lengths that the host
// path does not take (block scores, more than FSK_HOST_PLAN_MAX_BATCH
// sequences) are copied to the device instead.
struct Lengths {
  at::Tensor t;
  bool host;
};
Lengths lengths(const at::Tensor& t, const char* name, const c10::Device& dev, bool host_ok) {
  if (!t.defined()) raise(FSK_ERR_INVALID, std::string(name) + " is undefined");
  if (t.is_cuda()) return {int32_contig(t, name, dev), false};
  if (t.device().type() != c10::kCPU)
    raise(kRuntime, std::string(name) + " must be on the GPU or in host memory, got " + t.device().str());
  const at::Tensor h = t.to(at::kInt).contiguous();
  if (host_ok) return {h, true};
  return {h.to(dev), false};
}

c10::optional<at::Tensor> sinks(const c10::optional<at::Tensor>& s, int64_t hq, const c10::Device& dev) {
  if (!s || !s->defined()) return c10::nullopt;
  on_device(*s, "s_aux", dev);
  if (s->numel() != hq)
    raise(FSK_ERR_INVALID, "s_aux must have num_q_heads=" + std::to_string(hq) + " entries, got " + shape_str(*s));
  if (s->scalar_type() == at::kFloat && s->is_contiguous()) return *s;
  return s->reshape({hq}).to(at::kFloat).contiguous();
}

// A per-tensor scale: a one-element device tensor, widened to fp32.
c10::optional<at::Tensor> scale(const c10::optional<at::Tensor>& s, const char* name, const c10::Device& dev) {
  if (!s || !s->defined()) return c10::nullopt;
  on_device(*s, name, dev);
  if (s->numel() != 1) raise(FSK_ERR_INVALID, std::string(name) + " must hold a single per-tensor scale");
  return s->scalar_type() == at::kFloat ? *s : s->to(at::kFloat);
}

at::Tensor check_q(const at::Tensor& q) {
  on_gpu(q, "q");
  if (q.dim() != 3) raise(FSK_ERR_INVALID, "q must be [batch, num_q_heads, head_dim], got " + shape_str(q));
  return rows16(q);
}

at::Tensor kv_tensor(const at::Tensor& t, const char* name, const c10::Device& dev, int64_t dims,
                     const char* layout) {
  on_device(t, name, dev);
  if (t.dim() != dims) raise(FSK_ERR_INVALID, std::string(name) + " must be " + layout);
  return rows16(t);
}

at::ScalarType out_dtype(int64_t code, const at::Tensor& q) { return code < 0 ? q.scalar_type() : code_dtype(code); }

float softmax_scale(c10::optional<double> s, int64_t d) {
  return s ? (float)*s : (float)(1.0 / std::sqrt((double)d));
}

// Block-score output: the reduce kernel writes it as a contiguous
// [batch, num_q_heads, n] array in the output dtype.
bool score_tensor(const c10::optional<at::Tensor>& s, int64_t B, int64_t Hq, at::ScalarType odt,
                  const c10::Device& dev) {
  if (!s || !s->defined()) return false;
  on_device(*s, "scores", dev);
  if (s->dim() != 3 || s->size(0) != B || s->size(1) != Hq || s->size(2) < 1 || !s->is_contiguous() ||
      s->scalar_type() != odt)
    raise(FSK_ERR_INVALID, "scores must be a contiguous [" + std::to_string(B) + ", " + std::to_string(Hq) +
                               ", n] tensor of the output dtype, got " + shape_str(*s));
  return true;
}

at::Tensor workspace(int64_t nbytes, const at::Tensor& like) {
  if (nbytes < 0) check((int)nbytes);
  return at::empty({nbytes}, like.options().dtype(at::kByte));
}

void* stream_ptr(int64_t stream) { return reinterpret_cast<void*>(static_cast<intptr_t>(stream)); }

// ---------------------------------------------------------------------------
// paged (fskernels/paged_attn/triton_paged_attn.py:96-125)
// ---------------------------------------------------------------------------
at::Tensor paged(const at::Tensor& q_in, const at::Tensor& k_pool, const at::Tensor& v_pool,
                 const at::Tensor& block_table, const at::Tensor& seq_lens, int64_t page_size,
                 const c10::optional<at::Tensor>& s_aux, const c10::optional<at::Tensor>& k_scale,
                 const c10::optional<at::Tensor>& v_scale, int64_t out_code, int64_t sink_mode,
                 c10::optional<double> sm_scale, int64_t chunk_tokens, const c10::optional<at::Tensor>& scores,
                 int64_t stream) {
  const at::Tensor q = check_q(q_in);
  const c10::Device dev = q.device();
  const c10::DeviceGuard guard(dev);
  const at::Tensor k = kv_tensor(k_pool, "k_pool", dev, 4, "[num_pages, num_kv_heads, page_size, head_dim]");
  const at::Tensor v = kv_tensor(v_pool, "v_pool", dev, 4, "[num_pages, num_kv_heads, page_size, head_dim]");
  const int64_t B = q.size(0), Hq = q.size(1), D = q.size(2);
  const int64_t P = k.size(0), Hkv = k.size(1), PS = k.size(2);
  if (v.sizes() != k.sizes() || k.size(3) != D) raise(FSK_ERR_INVALID, "k_pool / v_pool shapes disagree with q");
  if (page_size != PS)
    raise(FSK_ERR_INVALID, "page_size=" + std::to_string(page_size) + " but the pools hold " + std::to_string(PS) +
                               "-token pages");
  on_device(block_table, "block_table", dev);
  if (block_table.dim() != 2 || block_table.size(0) < B) raise(FSK_ERR_INVALID, "block_table must be [batch, max_blocks]");
  at::Tensor bt = block_table.scalar_type() == at::kInt ? block_table : block_table.to(at::kInt);
  if (bt.stride(1) != 1) bt = bt.contiguous();
  const bool with_scores_arg = scores && scores->defined();
  const Lengths ln = lengths(seq_lens, "seq_lens", dev, !with_scores_arg && B <= FSK_HOST_PLAN_MAX_BATCH);
  const at::Tensor& lens = ln.t;
  if (lens.numel() < B) raise(FSK_ERR_INVALID, "seq_lens must have one entry per sequence");
  const auto sk = sinks(s_aux, Hq, dev);
  const auto ks = scale(k_scale, "k_scale", dev), vs = scale(v_scale, "v_scale", dev);
  const at::Tensor out = at::empty({B, Hq, D}, q.options().dtype(out_dtype(out_code, q)));
  const int64_t max_blocks = bt.size(1);
  int64_t nbytes = fsk_workspace_bytes(FSK_LAYOUT_PAGED, (int)B, (int)Hq, (int)Hkv, (int)D, max_blocks, (int)PS,
                                       (int)chunk_tokens);
  if (nbytes < 0) check((int)nbytes);
  const bool with_scores = score_tensor(scores, B, Hq, out.scalar_type(), dev);
  if (with_scores) {
    const int64_t extra = fsk_score_workspace_bytes((int)B, (int)Hq, (int)scores->size(2));
    if (extra < 0) check((int)extra);
    nbytes += extra;
  }
  const at::Tensor ws = workspace(nbytes, q);
  const int qd = dtype_code(q.scalar_type(), "q"), kd = dtype_code(k.scalar_type(), "k_pool");
  const int od = dtype_code(out.scalar_type(), "out_dtype");
  const float scl = softmax_scale(sm_scale, D);
  const float* sp = static_cast<const float*>(ptr_or_null(sk));
  const float* ksp = static_cast<const float*>(ptr_or_null(ks));
  const float* vsp = static_cast<const float*>(ptr_or_null(vs));
  int st;
  if (!with_scores) {
    auto entry = ln.host ? fsk_decode_paged_host : fsk_decode_paged;
    st = entry(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
                          k.stride(2), v.data_ptr(), v.stride(0), v.stride(1), v.stride(2), bt.data_ptr<int32_t>(),
                          bt.stride(0), (int)max_blocks, lens.data_ptr<int32_t>(), (int)P, (int)PS, sp,
                          (int)sink_mode, ksp, vsp, out.data_ptr(), out.stride(0), out.stride(1), (int)B, (int)Hq,
                          (int)Hkv, (int)D, qd, kd, od, scl, ws.data_ptr(), nbytes, (int)chunk_tokens,
                          stream_ptr(stream));
  } else {
    st = fsk_decode_paged_scores(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
                                 k.stride(2), v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
                                 bt.data_ptr<int32_t>(), bt.stride(0), (int)max_blocks, lens.data_ptr<int32_t>(),
                                 (int)P, (int)PS, sp, (int)sink_mode, ksp, vsp, out.data_ptr(), out.stride(0),
                                 out.stride(1), (int)B, (int)Hq, (int)Hkv, (int)D, qd, kd, od, scl, ws.data_ptr(),
                                 nbytes, (int)chunk_tokens, scores->data_ptr(), (int)scores->size(2),
                                 stream_ptr(stream));
  }
  check(st);
  return out;
}

// ---------------------------------------------------------------------------
// varlen (fskernels/triton/triton_gqa_decode.py:126-155)
// ---------------------------------------------------------------------------
at::Tensor varlen(const at::Tensor& q_in, const at::Tensor& k_varlen, const at::Tensor& v_varlen,
                  const at::Tensor& cu_seqlens_k, const c10::optional<at::Tensor>& s_aux,
                  const c10::optional<at::Tensor>& k_scale, const c10::optional<at::Tensor>& v_scale, int64_t out_code,
                  int64_t sink_mode, c10::optional<double> sm_scale, int64_t chunk_tokens,
                  const c10::optional<at::Tensor>& scores, int64_t stream) {
  const at::Tensor q = check_q(q_in);
  const c10::Device dev = q.device();
  const c10::DeviceGuard guard(dev);
  const at::Tensor k = kv_tensor(k_varlen, "k_varlen", dev, 3, "[total_tokens, num_kv_heads, head_dim]");
  const at::Tensor v = kv_tensor(v_varlen, "v_varlen", dev, 3, "[total_tokens, num_kv_heads, head_dim]");
  const int64_t B = q.size(0), Hq = q.size(1), D = q.size(2);
  const int64_t T = k.size(0), Hkv = k.size(1);
  if (v.sizes() != k.sizes() || k.size(2) != D) raise(FSK_ERR_INVALID, "k_varlen / v_varlen shapes disagree with q");
  const bool with_scores_arg = scores && scores->defined();
  const Lengths ln = lengths(cu_seqlens_k, "cu_seqlens_k", dev, !with_scores_arg && B <= FSK_HOST_PLAN_MAX_BATCH);
  const at::Tensor& cu = ln.t;
  if (cu.numel() != B + 1)
    raise(FSK_ERR_INVALID, "cu_seqlens_k must have batch+1=" + std::to_string(B + 1) + " entries");
  const auto sk = sinks(s_aux, Hq, dev);
  const auto ks = scale(k_scale, "k_scale", dev), vs = scale(v_scale, "v_scale", dev);
  const at::Tensor out = at::empty({B, Hq, D}, q.options().dtype(out_dtype(out_code, q)));
  int64_t nbytes = fsk_workspace_bytes(FSK_LAYOUT_VARLEN, (int)B, (int)Hq, (int)Hkv, (int)D, T, 16, (int)chunk_tokens);
  if (nbytes < 0) check((int)nbytes);
  const bool with_scores = score_tensor(scores, B, Hq, out.scalar_type(), dev);
  if (with_scores) {
    const int64_t extra = fsk_score_workspace_bytes((int)B, (int)Hq, (int)scores->size(2));
    if (extra < 0) check((int)extra);
    nbytes += extra;
  }
  const at::Tensor ws = workspace(nbytes, q);
  const int qd = dtype_code(q.scalar_type(), "q"), kd = dtype_code(k.scalar_type(), "k_varlen");
  const int od = dtype_code(out.scalar_type(), "out_dtype");
  const float scl = softmax_scale(sm_scale, D);
  const float* sp = static_cast<const float*>(ptr_or_null(sk));
  const float* ksp = static_cast<const float*>(ptr_or_null(ks));
  const float* vsp = static_cast<const float*>(ptr_or_null(vs));
  int st;
  if (!with_scores) {
    auto entry = ln.host ? fsk_decode_varlen_host : fsk_decode_varlen;
    st = entry(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
                           v.data_ptr(), v.stride(0), v.stride(1), cu.data_ptr<int32_t>(), T, sp, (int)sink_mode, ksp,
                           vsp, out.data_ptr(), out.stride(0), out.stride(1), (int)B, (int)Hq, (int)Hkv, (int)D, qd,
                           kd, od, scl, ws.data_ptr(), nbytes, (int)chunk_tokens, stream_ptr(stream));
  } else {
    st = fsk_decode_varlen_scores(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
                                  v.data_ptr(), v.stride(0), v.stride(1), cu.data_ptr<int32_t>(), T, sp,
                                  (int)sink_mode, ksp, vsp, out.data_ptr(), out.stride(0), out.stride(1), (int)B,
                                  (int)Hq, (int)Hkv, (int)D, qd, kd, od, scl, ws.data_ptr(), nbytes,
                                  (int)chunk_tokens, scores->data_ptr(), (int)scores->size(2), stream_ptr(stream));
  }
  check(st);
  return out;
}

// ---------------------------------------------------------------------------
// dense HF cache (fskernels/triton/triton_gqa_decode_hf.py:146-211,
// fskernels/triton/triton_gqa_decode_hf_fp8.py:164-227)
// ---------------------------------------------------------------------------
at::Tensor dense(const at::Tensor& q_in, const at::Tensor& k_cache, const at::Tensor& v_cache,
                 const at::Tensor& cache_lens, const c10::optional<at::Tensor>& start_k_offsets,
                 const c10::optional<at::Tensor>& s_aux, const c10::optional<at::Tensor>& q_scale,
                 const c10::optional<at::Tensor>& k_scale, const c10::optional<at::Tensor>& v_scale, int64_t out_code,
                 int64_t sink_mode, c10::optional<double> sm_scale, int64_t chunk_tokens, int64_t stream) {
  const at::Tensor q = check_q(q_in);
  const c10::Device dev = q.device();
  const c10::DeviceGuard guard(dev);
  const at::Tensor k = kv_tensor(k_cache, "k_cache", dev, 4, "[batch, num_kv_heads, max_seqlen, head_dim]");
  const at::Tensor v = kv_tensor(v_cache, "v_cache", dev, 4, "[batch, num_kv_heads, max_seqlen, head_dim]");
  const int64_t B = q.size(0), Hq = q.size(1), D = q.size(2);
  const int64_t Hkv = k.size(1), S = k.size(2);
  if (v.sizes() != k.sizes() || k.size(3) != D || k.size(0) < B)
    raise(FSK_ERR_INVALID, "k_cache / v_cache shapes disagree with q");
  const at::Tensor lens = int32_contig(cache_lens, "cache_lens", dev);
  if (lens.numel() < B) raise(FSK_ERR_INVALID, "cache_lens must have one entry per sequence");
  c10::optional<at::Tensor> starts;
  if (start_k_offsets && start_k_offsets->defined()) {
    starts = int32_contig(*start_k_offsets, "start_k_offsets", dev);
    if (starts->numel() < B) raise(FSK_ERR_INVALID, "start_k_offsets must have one entry per sequence");
  }
  const auto sk = sinks(s_aux, Hq, dev);
  const auto qs = scale(q_scale, "scale_q", dev), ks = scale(k_scale, "scale_k", dev);
  const auto vs = scale(v_scale, "scale_v", dev);
  const at::Tensor out = at::empty({B, Hq, D}, q.options().dtype(out_dtype(out_code, q)));
  const int64_t nbytes =
      fsk_workspace_bytes(FSK_LAYOUT_DENSE, (int)B, (int)Hq, (int)Hkv, (int)D, S, 16, (int)chunk_tokens);
  const at::Tensor ws = workspace(nbytes, q);
  const int st = fsk_decode_dense(
      q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1), k.stride(2), v.data_ptr(),
      v.stride(0), v.stride(1), v.stride(2), S, lens.data_ptr<int32_t>(),
      starts ? starts->data_ptr<int32_t>() : nullptr, static_cast<const float*>(ptr_or_null(sk)), (int)sink_mode,
      static_cast<const float*>(ptr_or_null(qs)), static_cast<const float*>(ptr_or_null(ks)),
      static_cast<const float*>(ptr_or_null(vs)), out.data_ptr(), out.stride(0), out.stride(1), (int)B, (int)Hq,
      (int)Hkv, (int)D, dtype_code(q.scalar_type(), "q"), dtype_code(k.scalar_type(), "k_cache"),
      dtype_code(out.scalar_type(), "out_dtype"), softmax_scale(sm_scale, D), ws.data_ptr(), nbytes,
      (int)chunk_tokens, stream_ptr(stream));
  check(st);
  return out;
}

// ---------------------------------------------------------------------------
// KV write (fskernels/paged_attn/paged_kv_cache.py:117-130, batched)
// ---------------------------------------------------------------------------
at::Tensor new_rows(const at::Tensor& t_in, const char* name) {
  at::Tensor t = t_in;
  if (t.dim() == 4) {
    if (t.size(2) != 1)
      raise(FSK_ERR_INVALID, std::string(name) + " as [n, Hkv, 1, D] must have a single position, got " + shape_str(t));
    t = t.select(2, 0);
  }
  if (t.dim() != 3) raise(FSK_ERR_INVALID, std::string(name) + " must be [n, Hkv, D] or [n, Hkv, 1, D], got " + shape_str(t));
  const auto dt = t.scalar_type();
  if (dt != at::kHalf && dt != at::kBFloat16 && dt != at::kFloat)
    raise(FSK_ERR_UNSUPPORTED, std::string(name) + ": dtype " + c10::toString(dt) + " (f16, bf16 or f32 expected)");
  return rows16(t);
}

void kv_write(const at::Tensor& k_in, const at::Tensor& v_in, const at::Tensor& k_pool, const at::Tensor& v_pool,
           const at::Tensor& slot_mapping, const c10::optional<at::Tensor>& k_scale,
           const c10::optional<at::Tensor>& v_scale, const c10::optional<at::Tensor>& block_table,
           const c10::optional<at::Tensor>& bt_updates, int64_t stream) {
  for (const auto* pt : {&k_pool, &v_pool}) {
    const char* name = pt == &k_pool ? "k_pool" : "v_pool";
    on_gpu(*pt, name);
    if (pt->dim() != 4)
      raise(FSK_ERR_INVALID, std::string(name) + " must be [P, Hkv, page_size, D], got " + shape_str(*pt));
    const auto dt = pt->scalar_type();
    if (dt != at::kHalf && dt != at::kBFloat16 && dt != at::kFloat8_e4m3fn)
      raise(FSK_ERR_UNSUPPORTED, std::string(name) + ": dtype " + c10::toString(dt) + " (f16, bf16 or e4m3 expected)");
    if (pt->stride(-1) != 1) raise(FSK_ERR_INVALID, std::string(name) + " must have a contiguous head_dim");
  }
  const c10::Device dev = k_pool.device();
  const c10::DeviceGuard guard(dev);
  if (v_pool.device() != dev || v_pool.sizes() != k_pool.sizes() || v_pool.scalar_type() != k_pool.scalar_type())
    raise(FSK_ERR_INVALID, "k_pool and v_pool must match in shape, dtype and device");
  const int64_t P = k_pool.size(0), Hkv = k_pool.size(1), PS = k_pool.size(2), D = k_pool.size(3);
  const at::Tensor k = new_rows(k_in, "k"), v = new_rows(v_in, "v");
  on_device(k, "k", dev);
  on_device(v, "v", dev);
  const int64_t n = k.size(0);
  if (k.size(1) != Hkv || k.size(2) != D || v.sizes() != k.sizes() || v.scalar_type() != k.scalar_type())
    raise(FSK_ERR_INVALID, "k/v must be [" + std::to_string(n) + ", " + std::to_string(Hkv) + ", " +
                               std::to_string(D) + "] of one dtype, got " + shape_str(k) + " / " + shape_str(v));
  on_device(slot_mapping, "slot_mapping", dev);
  if (slot_mapping.scalar_type() != at::kLong || slot_mapping.numel() != n)
    raise(FSK_ERR_INVALID, "slot_mapping must be int64 with " + std::to_string(n) + " entries");
  const at::Tensor slots =
      slot_mapping.dim() == 1 && slot_mapping.is_contiguous() ? slot_mapping : slot_mapping.reshape({n}).contiguous();
  for (const auto* s : {&k_scale, &v_scale}) {
    if (*s && (*s)->defined()) {
      const char* name = s == &k_scale ? "k_scale" : "v_scale";
      if ((*s)->scalar_type() != at::kFloat || (*s)->numel() != 1)
        raise(FSK_ERR_INVALID, std::string(name) + " must be a one-element fp32 device tensor");
      on_device(**s, name, dev);
    }
  }
  int32_t* bt_ptr = nullptr;
  int64_t bt_numel = 0, n_upd = 0;
  at::Tensor upd;
  if (bt_updates && bt_updates->defined() && bt_updates->numel()) {
    if (!block_table || !block_table->defined()) raise(FSK_ERR_INVALID, "bt_updates need block_table");
    on_device(*block_table, "block_table", dev);
    on_device(*bt_updates, "bt_updates", dev);
    if (block_table->scalar_type() != at::kInt || !block_table->is_contiguous())
      raise(FSK_ERR_INVALID, "block_table must be a contiguous int32 tensor");
    if (bt_updates->scalar_type() != at::kLong || bt_updates->dim() != 2 || bt_updates->size(1) != 2)
      raise(FSK_ERR_INVALID, "bt_updates must be int64 [m, 2]");
    upd = bt_updates->contiguous();
    bt_ptr = block_table->data_ptr<int32_t>();
    bt_numel = block_table->numel();
    n_upd = upd.size(0);
  }
  const int st = fsk_paged_write(
      k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1), slots.data_ptr<int64_t>(), n,
      k_pool.data_ptr(), k_pool.stride(0), k_pool.stride(1), k_pool.stride(2), v_pool.data_ptr(), v_pool.stride(0),
      v_pool.stride(1), v_pool.stride(2), (int)P, (int)PS, (int)Hkv, (int)D, dtype_code(k.scalar_type(), "k"),
      dtype_code(k_pool.scalar_type(), "k_pool"), static_cast<const float*>(ptr_or_null(k_scale)),
      static_cast<const float*>(ptr_or_null(v_scale)), bt_ptr, bt_numel,
      n_upd ? upd.data_ptr<int64_t>() : nullptr, n_upd, stream_ptr(stream));
  check(st);
}

}  // namespace

PYBIND11_MODULE(_fsk_torch, m) {
  m.doc() = "torch-tensor binding of libfsk_decode.so (one C++ call per decode or KV write)";
  pybind11::register_exception_translator([](std::exception_ptr p) {
    try {
      if (p) std::rethrow_exception(p);
    } catch (const FskFailure& f) {
      PyObject* type = PyExc_RuntimeError;
      if (f.code == FSK_ERR_INVALID) type = PyExc_ValueError;
      else if (f.code == FSK_ERR_UNSUPPORTED) type = PyExc_NotImplementedError;
      std::string msg = f.msg;
      if (f.code == FSK_ERR_HIP) msg = "libfsk_decode status " + std::to_string(f.code) + ": " + msg;
      PyErr_SetString(type, msg.c_str());
    }
  });
  namespace py = pybind11;
  m.def("paged", &paged, py::arg("q"), py::arg("k_pool"), py::arg("v_pool"), py::arg("block_table"),
        py::arg("seq_lens"), py::arg("page_size"), py::arg("s_aux"), py::arg("k_scale"), py::arg("v_scale"),
        py::arg("out_code"), py::arg("sink_mode"), py::arg("sm_scale"), py::arg("chunk_tokens"), py::arg("scores"),
        py::arg("stream"));
  m.def("varlen", &varlen, py::arg("q"), py::arg("k"), py::arg("v"), py::arg("cu_seqlens"), py::arg("s_aux"),
        py::arg("k_scale"), py::arg("v_scale"), py::arg("out_code"), py::arg("sink_mode"), py::arg("sm_scale"),
        py::arg("chunk_tokens"), py::arg("scores"), py::arg("stream"));
  m.def("dense", &dense, py::arg("q"), py::arg("k"), py::arg("v"), py::arg("cache_lens"), py::arg("start_k_offsets"),
        py::arg("s_aux"), py::arg("q_scale"), py::arg("k_scale"), py::arg("v_scale"), py::arg("out_code"),
        py::arg("sink_mode"), py::arg("sm_scale"), py::arg("chunk_tokens"), py::arg("stream"));
  m.def("kv_write", &kv_write, py::arg("k"), py::arg("v"), py::arg("k_pool"), py::arg("v_pool"), py::arg("slot_mapping"),
        py::arg("k_scale"), py::arg("v_scale"), py::arg("block_table"), py::arg("bt_updates"), py::arg("stream"));
}
