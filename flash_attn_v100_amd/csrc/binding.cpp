// PyTorch-ROCm extension exposing the reference module's Python API
// (module `flash_attn_v100`, flash_attn.cpp:224-255) on top of the C ABI in
// include/flash_attn_mi355x.h.
//
// Each function keeps the reference's positional signature, its argument
// validation (same conditions, same messages, raised as RuntimeError through
// TORCH_CHECK) and its output contract, then calls one fa_* entry point on the
// caller's current HIP stream (the `_stream` variants: on the given stream).
#include <torch/extension.h>

#include <ATen/hip/impl/HIPCachingAllocatorMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <cmath>
#include <tuple>
#include <vector>

#include "flash_attn_mi355x.h"

namespace {

using c10::hip::HIPGuardMasqueradingAsCUDA;
using c10::hip::HIPStreamGuardMasqueradingAsCUDA;

// Validation macros and helpers with the reference's conditions and messages
// (flash_attn_kernel.cu:15-30, :122-249).
#define CHECK_CUDA(x) TORCH_CHECK(x.device().is_cuda(), #x " must be a CUDA tensor")
#define CHECK_CONTIGUOUS(x) TORCH_CHECK(x.is_contiguous(), #x " must be a contiguous tensor")
#define CHECK_INPUT(x) \
  CHECK_CUDA(x);       \
  CHECK_CONTIGUOUS(x)
#define CHECK_DIM(x, expected_dim) TORCH_CHECK(x.dim() == expected_dim, #x " must be a " #expected_dim "D tensor")
#define CHECK_SAME_DEVICE(x, y) TORCH_CHECK(x.device() == y.device(), #x " and " #y " must be on the same device")
#define CHECK_SAME_DTYPE(x, y) TORCH_CHECK(x.dtype() == y.dtype(), #x " and " #y " must have the same dtype")

constexpr int64_t kMaxD = 128;       // MAX_D (flash_attn_kernel.cu:35)
constexpr int64_t kMaxDLarge = 256;  // MAX_D_LARGE (flash_attn_kernel.cu:36)
constexpr int64_t kPage = 16;        // PAGE_BLOCK_SIZE (flash_attn_kernel.cu:3389)

void check_fa(int rc) {
  TORCH_CHECK(rc == FA_OK, "flash_attn_v100 (MI355X): ", fa_last_error());
}

void* cur_stream() { return static_cast<void*>(c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream()); }

int to_int(int64_t x, const char* what) {
  TORCH_CHECK(x >= 0 && x <= INT32_MAX, what, " out of int32 range");
  return static_cast<int>(x);
}

// Shape agreement between q, k and v, as rule tables: each rule names one
// dimension (or the whole shape), the tensor pairs that must agree on it, and
// the message the reference raises when they do not.  The conditions and
// messages follow the reference's validators (flash_attn_kernel.cu:122-249);
// the table form is this build's own.
constexpr unsigned kQK = 1u, kQV = 2u, kKV = 4u;  // pairs: (q, k), (q, v), (k, v)
constexpr int kWholeShape = -1;

struct Agree {
  int dim;         // dimension index, or kWholeShape
  unsigned pairs;  // kQK | kQV | kKV
  const char* msg;
};

// self-attention: q, k, v of one shape
constexpr Agree kMhaRules[] = {{kWholeShape, kQK, "q and k must have the same shape"},
                               {kWholeShape, kQV, "q and v must have the same shape"}};
// MHA decode: q [B, H, 1, D] against k, v [B, H, N, D]
constexpr Agree kDecodeMhaRules[] = {{0, kQK | kQV, "q, k, v batch size must match"},
                                     {1, kQK | kQV, "q, k, v head count must match"},
                                     {3, kQK | kQV, "q, k, v head dimension must match"},
                                     {2, kKV, "k and v sequence length must match"}};
// GQA prefill: k, v may have fewer heads than q
constexpr Agree kPrefillGqaRules[] = {{0, kQK | kQV, "q, k, v batch size must match"},
                                      {1, kKV, "k and v must have the same number of heads"},
                                      {2, kQK | kQV, "q, k, v sequence length must match"},
                                      {3, kQK | kQV, "q, k, v head dimension must match"}};
// GQA decode
constexpr Agree kDecodeGqaRules[] = {{0, kQK | kQV, "q, k, v batch size must match"},
                                     {1, kKV, "k and v must have the same number of heads"},
                                     {2, kKV, "k and v sequence length must match"},
                                     {3, kQK | kQV, "q, k, v head dimension must match"}};
// packed varlen: [total, H, D] each
constexpr Agree kVarlenRules[] = {{0, kQK | kQV, "k and v total length must match q"},
                                  {1, kQK | kQV, "k and v head count must match q"},
                                  {2, kQK | kQV, "k and v head dimension must match q"}};

template <size_t N>
void check_qkv(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, int64_t ndim,
               const Agree (&rules)[N]) {
  const at::Tensor* t[3] = {&q, &k, &v};
  const char* name[3] = {"q", "k", "v"};
  for (int i = 0; i < 3; ++i) TORCH_CHECK(t[i]->dim() == ndim, name[i], " must be a ", ndim, "D tensor");
  for (int i = 1; i < 3; ++i) TORCH_CHECK(t[i]->device() == q.device(), "q and ", name[i], " must be on the same device");
  for (int i = 1; i < 3; ++i) TORCH_CHECK(t[i]->dtype() == q.dtype(), "q and ", name[i], " must have the same dtype");
  static constexpr int kPair[3][2] = {{0, 1}, {0, 2}, {1, 2}};
  for (const Agree& r : rules) {
    bool ok = true;
    for (int pi = 0; pi < 3; ++pi) {
      if (!(r.pairs & (1u << pi))) continue;
      const at::Tensor& a = *t[kPair[pi][0]];
      const at::Tensor& b = *t[kPair[pi][1]];
      ok = ok && (r.dim == kWholeShape ? a.sizes() == b.sizes() : a.size(r.dim) == b.size(r.dim));
    }
    TORCH_CHECK(ok, r.msg);
  }
}

void check_mha_input_shapes(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v) {
  check_qkv(q, k, v, 4, kMhaRules);
}
void check_decode_mha_input_shapes(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v) {
  check_qkv(q, k, v, 4, kDecodeMhaRules);
}
void check_prefill_gqa_input_shapes(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v) {
  check_qkv(q, k, v, 4, kPrefillGqaRules);
}
void check_decode_gqa_input_shapes(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v) {
  check_qkv(q, k, v, 4, kDecodeGqaRules);
}
void check_varlen_prefill_input_shapes(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                       const at::Tensor& cu_seqlens) {
  CHECK_DIM(cu_seqlens, 1);
  CHECK_SAME_DEVICE(q, cu_seqlens);
  check_qkv(q, k, v, 3, kVarlenRules);
}

void check_cache_len(int cache_len, int64_t seq_len) {
  TORCH_CHECK(cache_len >= 0, "cache_len must be non-negative");
  TORCH_CHECK(cache_len < seq_len, "cache_len must be less than sequence length");
}

void check_decode_gqa_output_tensor(const at::Tensor& out, const at::Tensor& q) {
  CHECK_INPUT(out);
  CHECK_DIM(out, 4);
  CHECK_SAME_DEVICE(out, q);
  CHECK_SAME_DTYPE(out, q);
  TORCH_CHECK(out.size(0) == q.size(0), "out batch size must match q");
  TORCH_CHECK(out.size(1) == q.size(1), "out head count must match q");
  TORCH_CHECK(out.size(2) == 1, "out sequence length must be 1 for decode mode");
  TORCH_CHECK(out.size(3) == q.size(3), "out head dimension must match q");
}

void check_prefill_gqa_output_tensor(const at::Tensor& out, const at::Tensor& q) {
  CHECK_INPUT(out);
  CHECK_DIM(out, 4);
  CHECK_SAME_DEVICE(out, q);
  CHECK_SAME_DTYPE(out, q);
  TORCH_CHECK(out.sizes() == q.sizes(), "out shape must match q shape for prefill mode");
}

// Split-KV workspace.  The kernels leave its arrival counters at zero after
// every call, so a buffer is zero-filled once, when allocated, and then serves
// any number of calls issued in order on one stream.  Two pools:
//  * eager calls: one buffer per (device, stream), least recently used first
//    out once a device holds kMaxEagerWorkspaces of them (a server that makes
//    a stream per request does not accumulate buffers).  A dropped or
//    outgrown buffer returns to the caching allocator, which hands it only to
//    later allocations on the same stream, i.e. after the calls already queued
//    there.
//  * calls under graph capture: one buffer per (device, capturing stream),
//    never shared with eager calls and never released: a captured graph keeps
//    the buffer's address, so an outgrown one is retired but kept alive.
//    Graphs captured on one stream share that buffer and must be replayed in
//    order, not concurrently with each other.
// The GIL serialises every use of these pools.
constexpr size_t kMaxEagerWorkspaces = 8;

struct WorkspaceEntry {
  int device;
  uintptr_t stream;
  at::Tensor buf;
  uint64_t last_use;
};

struct WorkspacePools {
  std::vector<WorkspaceEntry> eager;
  std::vector<WorkspaceEntry> captured;
  std::vector<at::Tensor> retired;  // outgrown capture buffers, still referenced by graphs
  uint64_t tick = 0;
};

bool stream_is_capturing(void* stream) {
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  const hipError_t err = hipStreamIsCapturing(static_cast<hipStream_t>(stream), &status);
  TORCH_CHECK(err == hipSuccess, "hipStreamIsCapturing: ", hipGetErrorString(err));
  return status != hipStreamCaptureStatusNone;
}

at::Tensor decode_workspace(const at::Tensor& q, int B, int H_Q, int H_KV, int max_len, int D) {
  // Deliberately leaked: destroying tensors after the HIP runtime shut down at exit is unsafe.
  static auto& pools = *new WorkspacePools();
  const size_t bytes = fa_decode_workspace_size(B, H_Q, H_KV, max_len, D);
  if (bytes == 0) return at::Tensor();
  void* stream = cur_stream();
  const int device = q.device().index();
  const uintptr_t sid = reinterpret_cast<uintptr_t>(stream);
  const bool capturing = stream_is_capturing(stream);
  auto& pool = capturing ? pools.captured : pools.eager;
  const uint64_t now = ++pools.tick;
  for (auto& e : pool) {
    if (e.device != device || e.stream != sid) continue;
    if (static_cast<size_t>(e.buf.numel()) >= bytes) {
      e.last_use = now;
      return e.buf;
    }
    // Grow geometrically.
    const size_t alloc = std::max(bytes, static_cast<size_t>(e.buf.numel()) * 2);
    at::Tensor grown = at::zeros({static_cast<int64_t>(alloc)}, q.options().dtype(at::kByte));
    if (capturing) pools.retired.push_back(e.buf);
    e.buf = grown;
    e.last_use = now;
    return grown;
  }
  if (!capturing) {
    size_t on_device = 0;
    WorkspaceEntry* lru = nullptr;
    for (auto& e : pool) {
      if (e.device != device) continue;
      ++on_device;
      if (!lru || e.last_use < lru->last_use) lru = &e;
    }
    if (on_device >= kMaxEagerWorkspaces && lru) {
      *lru = pool.back();
      pool.pop_back();
    }
  }
  at::Tensor ws = at::zeros({static_cast<int64_t>(bytes)}, q.options().dtype(at::kByte));
  pool.push_back(WorkspaceEntry{device, sid, ws, now});
  return ws;
}

void* ws_ptr(const at::Tensor& ws) { return ws.defined() ? ws.data_ptr() : nullptr; }
size_t ws_bytes(const at::Tensor& ws) { return ws.defined() ? static_cast<size_t>(ws.numel()) : 0; }

// ---------------------------------------------------------------------------
// Prefill

void launch_prefill(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, at::Tensor& out, bool causal) {
  check_fa(fa_prefill_fp16(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), to_int(q.size(0), "B"),
                           to_int(q.size(1), "H_Q"), to_int(k.size(1), "H_KV"), to_int(q.size(2), "N"),
                           to_int(q.size(3), "D"), causal ? 1 : 0, cur_stream()));
}

// forward_prefill_gqa_fp16 (flash_attn_kernel.cu:2740-2768)
at::Tensor forward_prefill_gqa_fp16(at::Tensor q, at::Tensor k, at::Tensor v, bool causal) {
  CHECK_INPUT(q);
  CHECK_INPUT(k);
  CHECK_INPUT(v);
  check_prefill_gqa_input_shapes(q, k, v);
  TORCH_CHECK(q.dtype() == at::kHalf, "q, k, v must be float16");
  const auto H_Q = q.size(1), N = q.size(2), D = q.size(3), H_KV = k.size(1);
  TORCH_CHECK(H_Q >= H_KV, "H_Q must be >= H_KV");
  TORCH_CHECK(H_Q % H_KV == 0, "H_Q must be divisible by H_KV");
  TORCH_CHECK(D <= kMaxDLarge, "D must be <= MAX_D_LARGE(256)");
  TORCH_CHECK(k.size(2) == N, "k sequence length must match q");
  TORCH_CHECK(v.size(2) == N, "v sequence length must match q");
  HIPGuardMasqueradingAsCUDA guard(q.device());
  auto out = at::empty_like(q);
  launch_prefill(q, k, v, out, causal);
  return out;
}

// forward_prefill_gqa_fp16_out (flash_attn_kernel.cu:2770-2794)
at::Tensor forward_prefill_gqa_fp16_out(at::Tensor out, at::Tensor q, at::Tensor k, at::Tensor v, bool causal) {
  CHECK_INPUT(q);
  CHECK_INPUT(k);
  CHECK_INPUT(v);
  check_prefill_gqa_input_shapes(q, k, v);
  check_prefill_gqa_output_tensor(out, q);
  TORCH_CHECK(q.dtype() == at::kHalf, "q, k, v must be float16");
  TORCH_CHECK(q.size(1) >= k.size(1), "H_Q must be >= H_KV");
  TORCH_CHECK(q.size(1) % k.size(1) == 0, "H_Q must be divisible by H_KV");
  TORCH_CHECK(q.size(3) <= kMaxDLarge, "D must be <= MAX_D_LARGE(256)");
  HIPGuardMasqueradingAsCUDA guard(q.device());
  launch_prefill(q, k, v, out, causal);
  return out;
}

// forward_fp16 (flash_attn_kernel.cu:1915-1962)
at::Tensor forward_fp16(at::Tensor q, at::Tensor k, at::Tensor v, bool causal) {
  CHECK_INPUT(q);
  CHECK_INPUT(k);
  CHECK_INPUT(v);
  check_mha_input_shapes(q, k, v);
  TORCH_CHECK(q.dtype() == at::kHalf, "q, k, v must be float16");
  TORCH_CHECK(q.size(3) <= kMaxDLarge, "D must be less than or equal to MAX_D_LARGE(256)");
  if (q.size(3) > kMaxD) return forward_prefill_gqa_fp16(q, k, v, causal);
  HIPGuardMasqueradingAsCUDA guard(q.device());
  auto out = at::empty_like(q);
  launch_prefill(q, k, v, out, causal);
  return out;
}

// forward_fp16_warp (flash_attn_kernel.cu:1440-1484): same math as forward_fp16.
at::Tensor forward_fp16_warp(at::Tensor q, at::Tensor k, at::Tensor v, bool causal) {
  CHECK_INPUT(q);
  CHECK_INPUT(k);
  CHECK_INPUT(v);
  check_mha_input_shapes(q, k, v);
  TORCH_CHECK(q.dtype() == at::kHalf, "q, k, v must be float16");
  TORCH_CHECK(q.size(3) <= kMaxD, "D must be less than or equal to MAX_D(128)");
  HIPGuardMasqueradingAsCUDA guard(q.device());
  auto out = at::empty_like(q);
  launch_prefill(q, k, v, out, causal);
  return out;
}

// forward_fp16_wmma (flash_attn_kernel.cu:2425-2468): the reference's tensor-core
// variant; on gfx950 the one MFMA prefill kernel serves both names.
at::Tensor forward_fp16_wmma(at::Tensor q, at::Tensor k, at::Tensor v, bool causal) {
  CHECK_INPUT(q);
  CHECK_INPUT(k);
  CHECK_INPUT(v);
  check_mha_input_shapes(q, k, v);
  TORCH_CHECK(q.dtype() == at::kHalf, "q, k, v must be float16");
  TORCH_CHECK(q.size(3) % 16 == 0, "D must be multiple of 16 for WMMA");
  TORCH_CHECK(q.size(3) <= kMaxD, "D must be less than or equal to MAX_D(128)");
  HIPGuardMasqueradingAsCUDA guard(q.device());
  auto out = at::empty_like(q);
  launch_prefill(q, k, v, out, causal);
  return out;
}

// forward_prefill_gqa_fp16_warp (flash_attn_kernel.cu:3586-3637)
at::Tensor forward_prefill_gqa_fp16_warp(at::Tensor q, at::Tensor k, at::Tensor v, bool causal) {
  return forward_prefill_gqa_fp16(q, k, v, causal);
}

// ---------------------------------------------------------------------------
// Decode

void launch_decode(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, at::Tensor& out, bool causal,
                   int cache_len) {
  const int B = to_int(q.size(0), "B"), H_Q = to_int(q.size(1), "H_Q"), H_KV = to_int(k.size(1), "H_KV");
  const int N = to_int(k.size(2), "N"), D = to_int(q.size(3), "D");
  auto ws = decode_workspace(q, B, H_Q, H_KV, N, D);
  check_fa(fa_decode_fp16(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), B, H_Q, H_KV, N, D,
                          causal ? 1 : 0, cache_len, ws_ptr(ws), ws_bytes(ws),
                          cur_stream()));
}

// forward_decode_gqa_fp16 (flash_attn_kernel.cu:1800-1833)
at::Tensor forward_decode_gqa_fp16(at::Tensor q, at::Tensor k, at::Tensor v, bool causal, int cache_len) {
  CHECK_INPUT(q);
  CHECK_INPUT(k);
  CHECK_INPUT(v);
  check_decode_gqa_input_shapes(q, k, v);
  TORCH_CHECK(q.dtype() == at::kHalf, "q, k, v must be float16");
  TORCH_CHECK(q.size(2) == 1, "q sequence length must be 1 for decode mode");
  const auto H_Q = q.size(1), H_KV = k.size(1);
  TORCH_CHECK(H_KV == v.size(1), "k and v must have same number of heads");
  TORCH_CHECK(H_Q >= H_KV, "H_Q must be >= H_KV");
  TORCH_CHECK(H_Q % H_KV == 0, "H_Q must be divisible by H_KV");
  TORCH_CHECK(q.size(3) <= kMaxDLarge, "D must be less than or equal to MAX_D_LARGE(256)");
  check_cache_len(cache_len, k.size(2));
  HIPGuardMasqueradingAsCUDA guard(q.device());
  auto out = at::empty({q.size(0), H_Q, 1, q.size(3)}, q.options());
  launch_decode(q, k, v, out, causal, cache_len);
  return out;
}

// forward_decode_gqa_fp16_out (flash_attn_kernel.cu:1835-1861)
at::Tensor forward_decode_gqa_fp16_out(at::Tensor out, at::Tensor q, at::Tensor k, at::Tensor v, bool causal,
                                       int cache_len) {
  CHECK_INPUT(q);
  CHECK_INPUT(k);
  CHECK_INPUT(v);
  check_decode_gqa_input_shapes(q, k, v);
  check_decode_gqa_output_tensor(out, q);
  TORCH_CHECK(q.dtype() == at::kHalf, "q, k, v must be float16");
  TORCH_CHECK(q.size(2) == 1, "q sequence length must be 1 for decode mode");
  TORCH_CHECK(q.size(1) >= k.size(1), "H_Q must be >= H_KV");
  TORCH_CHECK(q.size(1) % k.size(1) == 0, "H_Q must be divisible by H_KV");
  TORCH_CHECK(q.size(3) <= kMaxDLarge, "D must be less than or equal to MAX_D_LARGE(256)");
  check_cache_len(cache_len, k.size(2));
  HIPGuardMasqueradingAsCUDA guard(q.device());
  launch_decode(q, k, v, out, causal, cache_len);
  return out;
}

// forward_decode_gqa_fp16_stream (flash_attn_kernel.cu:3639-3673)
at::Tensor forward_decode_gqa_fp16_stream(at::Tensor q, at::Tensor k, at::Tensor v, bool causal, int cache_len,
                                          int64_t stream_int) {
  HIPGuardMasqueradingAsCUDA guard(q.device());
  auto ext = c10::hip::getStreamFromExternalMasqueradingAsCUDA(reinterpret_cast<hipStream_t>(stream_int),
                                                               q.device().index());
  HIPStreamGuardMasqueradingAsCUDA sguard(ext);
  return forward_decode_gqa_fp16(q, k, v, causal, cache_len);
}

// forward_decode_fp16 (flash_attn_kernel.cu:1863-1913)
at::Tensor forward_decode_fp16(at::Tensor q, at::Tensor k, at::Tensor v, bool causal, int cache_len) {
  CHECK_INPUT(q);
  CHECK_INPUT(k);
  CHECK_INPUT(v);
  check_decode_mha_input_shapes(q, k, v);
  TORCH_CHECK(q.dtype() == at::kHalf, "q, k, v must be float16");
  TORCH_CHECK(q.size(2) == 1, "q sequence length must be 1 for decode mode");
  TORCH_CHECK(q.size(3) <= kMaxDLarge, "D must be less than or equal to MAX_D_LARGE(256)");
  check_cache_len(cache_len, k.size(2));
  HIPGuardMasqueradingAsCUDA guard(q.device());
  auto out = at::empty({q.size(0), q.size(1), 1, q.size(3)}, q.options());
  launch_decode(q, k, v, out, causal, cache_len);
  return out;
}

// forward_continuous_batching_fp16 (continuous_batching_kernel.cu:338-406)
at::Tensor forward_continuous_batching_fp16(at::Tensor q, at::Tensor k, at::Tensor v, at::Tensor cache_lens,
                                            bool causal) {
  CHECK_INPUT(q);
  CHECK_INPUT(k);
  CHECK_INPUT(v);
  CHECK_INPUT(cache_lens);
  TORCH_CHECK(q.dtype() == at::kHalf, "q must be float16");
  TORCH_CHECK(q.size(2) == 1, "q sequence length must be 1 for decode mode");
  TORCH_CHECK(cache_lens.dim() == 1, "cache_lens must be 1D tensor");
  TORCH_CHECK(cache_lens.size(0) == q.size(0), "cache_lens size must match batch size");
  const auto H_Q = q.size(1), H_KV = k.size(1), D = q.size(3);
  TORCH_CHECK(H_Q >= H_KV, "H_Q must be >= H_KV");
  TORCH_CHECK(H_Q % H_KV == 0, "H_Q must be divisible by H_KV");
  TORCH_CHECK(D <= kMaxDLarge, "D must be <= MAX_D_CB_LARGE(256)");
  // The reference reads these without checking (continuous_batching_kernel.cu:373-403);
  // a mismatch there reads out of bounds, here it is an error.
  TORCH_CHECK(cache_lens.dtype() == at::kInt, "cache_lens must be int32");
  check_decode_gqa_input_shapes(q, k, v);
  CHECK_SAME_DEVICE(q, cache_lens);
  HIPGuardMasqueradingAsCUDA guard(q.device());
  const int B = to_int(q.size(0), "B"), hq = to_int(H_Q, "H_Q"), hkv = to_int(H_KV, "H_KV");
  const int max_N = to_int(k.size(2), "max_N"), d = to_int(D, "D");
  auto out = at::empty({q.size(0), H_Q, 1, D}, q.options());
  auto ws = decode_workspace(q, B, hq, hkv, max_N, d);
  check_fa(fa_continuous_batching_fp16(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                       cache_lens.data_ptr<int32_t>(), B, hq, hkv, max_N, d, causal ? 1 : 0,
                                       ws_ptr(ws), ws_bytes(ws), cur_stream()));
  return out;
}

// forward_paged_decode_gqa_fp16 (flash_attn_kernel.cu:3516-3584)
at::Tensor forward_paged_decode_gqa_fp16(at::Tensor q, at::Tensor k_cache, at::Tensor v_cache,
                                         at::Tensor block_table, at::Tensor seq_lens, int max_num_blocks) {
  CHECK_INPUT(q);
  CHECK_INPUT(k_cache);
  CHECK_INPUT(v_cache);
  CHECK_INPUT(block_table);
  CHECK_INPUT(seq_lens);
  CHECK_DIM(q, 4);
  CHECK_DIM(k_cache, 4);
  CHECK_DIM(v_cache, 4);
  CHECK_DIM(block_table, 2);
  CHECK_DIM(seq_lens, 1);
  CHECK_SAME_DEVICE(q, k_cache);
  CHECK_SAME_DEVICE(q, v_cache);
  CHECK_SAME_DEVICE(q, block_table);
  CHECK_SAME_DEVICE(q, seq_lens);
  TORCH_CHECK(q.dtype() == at::kHalf, "q must be float16");
  TORCH_CHECK(k_cache.dtype() == at::kHalf, "k_cache must be float16");
  TORCH_CHECK(v_cache.dtype() == at::kHalf, "v_cache must be float16");
  TORCH_CHECK(block_table.dtype() == at::kInt, "block_table must be int32");
  TORCH_CHECK(seq_lens.dtype() == at::kInt, "seq_lens must be int32");
  TORCH_CHECK(q.size(2) == 1, "q sequence length must be 1 for decode mode");
  const auto B = q.size(0), H_Q = q.size(1), H_KV = k_cache.size(1), D = q.size(3);
  TORCH_CHECK(H_Q >= H_KV, "H_Q must be >= H_KV");
  TORCH_CHECK(H_Q % H_KV == 0, "H_Q must be divisible by H_KV");
  TORCH_CHECK(D <= kMaxDLarge, "D must be <= MAX_D_LARGE(256)");
  TORCH_CHECK(k_cache.size(2) == kPage, "k_cache block size mismatch");
  TORCH_CHECK(v_cache.size(2) == kPage, "v_cache block size mismatch");
  TORCH_CHECK(block_table.size(0) == B, "block_table batch size must match q");
  TORCH_CHECK(seq_lens.size(0) == B, "seq_lens batch size must match q");
  // Unchecked in the reference, which then addresses the caches with q's D.
  TORCH_CHECK(k_cache.sizes() == v_cache.sizes(), "k_cache and v_cache must have the same shape");
  TORCH_CHECK(k_cache.size(3) == D, "k_cache head dimension must match q");
  TORCH_CHECK(max_num_blocks >= 0, "max_num_blocks must be non-negative");
  HIPGuardMasqueradingAsCUDA guard(q.device());
  const int b = to_int(B, "B"), hq = to_int(H_Q, "H_Q"), hkv = to_int(H_KV, "H_KV"), d = to_int(D, "D");
  auto out = at::empty({B, H_Q, 1, D}, q.options());
  auto ws = decode_workspace(q, b, hq, hkv, max_num_blocks * static_cast<int>(kPage), d);
  check_fa(fa_paged_decode_gqa_fp16(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(),
                                    block_table.data_ptr<int32_t>(), block_table.numel(),
                                    seq_lens.data_ptr<int32_t>(), b, hq, hkv, d,
                                    to_int(k_cache.size(0), "num_pages"), max_num_blocks, ws_ptr(ws), ws_bytes(ws), cur_stream()));
  return out;
}

// forward_decode_int8_gqa (flash_attn_kernel.cu:2941-3003)
at::Tensor forward_decode_int8_gqa(at::Tensor q, at::Tensor k, at::Tensor v, at::Tensor q_scale,
                                   at::Tensor k_scale, int cache_len) {
  CHECK_INPUT(q);
  CHECK_INPUT(k);
  CHECK_INPUT(v);
  CHECK_INPUT(q_scale);
  CHECK_INPUT(k_scale);
  check_decode_gqa_input_shapes(q, k, v);
  TORCH_CHECK(q.dtype() == at::kHalf, "q, k, v must be float16");
  TORCH_CHECK(q_scale.dtype() == at::kFloat, "q_scale must be float32");
  TORCH_CHECK(k_scale.dtype() == at::kFloat, "k_scale must be float32");
  TORCH_CHECK(q.size(2) == 1, "q sequence length must be 1 for decode mode");
  const auto B = q.size(0), H_Q = q.size(1), H_KV = k.size(1), N = k.size(2), D = q.size(3);
  TORCH_CHECK(H_Q >= H_KV, "H_Q must be >= H_KV");
  TORCH_CHECK(H_Q % H_KV == 0, "H_Q must be divisible by H_KV");
  TORCH_CHECK(D <= kMaxDLarge, "D must be <= MAX_D_LARGE(256)");
  TORCH_CHECK(q_scale.dim() >= 2 && q_scale.size(0) == B && q_scale.size(1) == H_Q, "q_scale must be [B, H_Q]");
  TORCH_CHECK(k_scale.dim() >= 3 && k_scale.size(0) == B && k_scale.size(1) == H_KV && k_scale.size(2) == N,
              "k_scale must be [B, H_KV, N]");
  CHECK_SAME_DEVICE(q, q_scale);
  CHECK_SAME_DEVICE(q, k_scale);
  check_cache_len(cache_len, N);
  HIPGuardMasqueradingAsCUDA guard(q.device());
  const int b = to_int(B, "B"), hq = to_int(H_Q, "H_Q"), hkv = to_int(H_KV, "H_KV");
  const int n = to_int(N, "N"), d = to_int(D, "D");
  auto out = at::empty({B, H_Q, 1, D}, q.options());
  auto ws = decode_workspace(q, b, hq, hkv, n, d);
  check_fa(fa_decode_int8_gqa(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                              q_scale.data_ptr<float>(), k_scale.data_ptr<float>(), b, hq, hkv, n, d, cache_len,
                              ws_ptr(ws), ws_bytes(ws), cur_stream()));
  return out;
}

// ---------------------------------------------------------------------------
// Varlen prefill

// forward_varlen_prefill_fp16 (flash_attn_kernel.cu:3354-3387)
at::Tensor forward_varlen_prefill_fp16(at::Tensor q, at::Tensor k, at::Tensor v, at::Tensor cu_seqlens,
                                       int max_seqlen, bool causal) {
  CHECK_INPUT(q);
  CHECK_INPUT(k);
  CHECK_INPUT(v);
  CHECK_INPUT(cu_seqlens);
  check_varlen_prefill_input_shapes(q, k, v, cu_seqlens);
  TORCH_CHECK(q.dtype() == at::kHalf, "q, k, v must be float16");
  TORCH_CHECK(cu_seqlens.dtype() == at::kInt, "cu_seqlens must be int32");
  const auto total_q = q.size(0), H = q.size(1), D = q.size(2);
  const auto batch_size = cu_seqlens.size(0) - 1;
  TORCH_CHECK(D <= kMaxDLarge, "D must be <= MAX_D_LARGE(256)");
  TORCH_CHECK(k.size(0) == total_q, "k and q must have same total length");
  TORCH_CHECK(v.size(0) == total_q, "v and q must have same total length");
  TORCH_CHECK(max_seqlen > 0, "max_seqlen must be positive");
  TORCH_CHECK(batch_size > 0, "cu_seqlens must contain at least one sequence");
  HIPGuardMasqueradingAsCUDA guard(q.device());
  auto out = at::empty_like(q);  // the kernel zeroes every row it does not compute
  // Rows a sequence's reference grid reaches: tile*ceil(max_seqlen/tile), tile 32
  // for D <= 128 and 8 above (flash_attn_kernel.cu:3319-3320, :3336-3337).
  const int64_t tile = D <= kMaxD ? 32 : 8;
  const int64_t row_limit = ((static_cast<int64_t>(max_seqlen) + tile - 1) / tile) * tile;
  check_fa(fa_varlen_prefill_fp16(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                  cu_seqlens.data_ptr<int32_t>(), to_int(batch_size, "batch"),
                                  to_int(total_q, "total"), to_int(H, "H"), to_int(D, "D"), max_seqlen,
                                  to_int(std::min<int64_t>(row_limit, INT32_MAX), "row_limit"), causal ? 1 : 0,
                                  cur_stream()));
  return out;
}

// forward_varlen_prefill_fp16_stream (flash_attn_kernel.cu:3675-3712)
at::Tensor forward_varlen_prefill_fp16_stream(at::Tensor q, at::Tensor k, at::Tensor v, at::Tensor cu_seqlens,
                                              int max_seqlen, bool causal, int64_t stream_int) {
  HIPGuardMasqueradingAsCUDA guard(q.device());
  auto ext = c10::hip::getStreamFromExternalMasqueradingAsCUDA(reinterpret_cast<hipStream_t>(stream_int),
                                                               q.device().index());
  HIPStreamGuardMasqueradingAsCUDA sguard(ext);
  return forward_varlen_prefill_fp16(q, k, v, cu_seqlens, max_seqlen, causal);
}

// ---------------------------------------------------------------------------
// Training: log-sum-exp forwards and the backward.

void check_lse_forward(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, at::ScalarType dt,
                       const char* dtype_msg) {
  CHECK_INPUT(q);
  CHECK_INPUT(k);
  CHECK_INPUT(v);
  check_mha_input_shapes(q, k, v);
  TORCH_CHECK(q.dtype() == dt, dtype_msg);
  TORCH_CHECK(q.size(3) <= kMaxD, "D must be less than or equal to MAX_D(128)");
}

std::tuple<at::Tensor, at::Tensor> forward_fp32_impl(at::Tensor q, at::Tensor k, at::Tensor v, bool causal,
                                                     bool want_lse) {
  check_lse_forward(q, k, v, at::kFloat, "q, k, v must be float32");
  HIPGuardMasqueradingAsCUDA guard(q.device());
  auto out = at::empty_like(q);
  at::Tensor lse;
  if (want_lse) lse = at::empty({q.size(0), q.size(1), q.size(2)}, q.options().dtype(at::kFloat));
  check_fa(fa_prefill_fp32(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                           want_lse ? lse.data_ptr<float>() : nullptr, to_int(q.size(0), "B"),
                           to_int(q.size(1), "H"), to_int(q.size(2), "N"), to_int(q.size(3), "D"),
                           causal ? 1 : 0, cur_stream()));
  return std::make_tuple(out, lse);
}

// forward (flash_attn_kernel.cu:508-550): fp32 MHA forward.
at::Tensor forward_fp32(at::Tensor q, at::Tensor k, at::Tensor v, bool causal) {
  return std::get<0>(forward_fp32_impl(q, k, v, causal, false));
}

// forward_with_lse (flash_attn_kernel.cu:1964-2006): fp32 forward + LSE [B, H, N].
std::tuple<at::Tensor, at::Tensor> forward_with_lse(at::Tensor q, at::Tensor k, at::Tensor v, bool causal) {
  return forward_fp32_impl(q, k, v, causal, true);
}

// forward_fp16_with_lse (flash_attn_kernel.cu:2008-2050): fp16 forward + fp32 LSE [B, H, N].
std::tuple<at::Tensor, at::Tensor> forward_fp16_with_lse(at::Tensor q, at::Tensor k, at::Tensor v, bool causal) {
  check_lse_forward(q, k, v, at::kHalf, "q, k, v must be float16");
  HIPGuardMasqueradingAsCUDA guard(q.device());
  auto out = at::empty_like(q);
  auto lse = at::empty({q.size(0), q.size(1), q.size(2)}, q.options().dtype(at::kFloat));
  check_fa(fa_prefill_fp16_lse(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr<float>(),
                               to_int(q.size(0), "B"), to_int(q.size(1), "H"), to_int(q.size(2), "N"),
                               to_int(q.size(3), "D"), causal ? 1 : 0, cur_stream()));
  return std::make_tuple(out, lse);
}

// backward (flash_attn_kernel.cu:2173-2264): dq, dk, dv in q's dtype.
std::tuple<at::Tensor, at::Tensor, at::Tensor> backward(at::Tensor dout, at::Tensor q, at::Tensor k, at::Tensor v,
                                                        at::Tensor out, at::Tensor logsumexp, bool causal) {
  CHECK_INPUT(dout);
  CHECK_INPUT(q);
  CHECK_INPUT(k);
  CHECK_INPUT(v);
  CHECK_INPUT(out);
  CHECK_INPUT(logsumexp);
  check_mha_input_shapes(q, k, v);
  TORCH_CHECK(dout.sizes() == q.sizes(), "dout and q must have the same shape");
  TORCH_CHECK(out.sizes() == q.sizes(), "out and q must have the same shape");
  CHECK_SAME_DEVICE(dout, q);
  CHECK_SAME_DEVICE(out, q);
  CHECK_SAME_DEVICE(logsumexp, q);
  CHECK_SAME_DTYPE(dout, q);
  CHECK_SAME_DTYPE(out, q);
  TORCH_CHECK(q.dtype() == at::kFloat || q.dtype() == at::kHalf, "q, k, v must be float32 or float16");
  TORCH_CHECK(logsumexp.dtype() == at::kFloat, "logsumexp must be float32");
  const auto B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3);
  TORCH_CHECK(D <= kMaxD, "D must be less than or equal to MAX_D(128)");
  CHECK_DIM(logsumexp, 3);
  TORCH_CHECK(logsumexp.size(0) == B && logsumexp.size(1) == H && logsumexp.size(2) == N,
              "logsumexp shape must be [B, H, N]");
  HIPGuardMasqueradingAsCUDA guard(q.device());
  auto dq = at::empty_like(q);
  auto dk = at::empty_like(k);
  auto dv = at::empty_like(v);
  const int b = to_int(B, "B"), h = to_int(H, "H"), n = to_int(N, "N"), d = to_int(D, "D");
  const size_t ws_bytes = fa_backward_workspace_size(b, h, n);
  at::Tensor ws;
  if (ws_bytes > 0) ws = at::empty({static_cast<int64_t>(ws_bytes / sizeof(float))}, q.options().dtype(at::kFloat));
  auto fn = q.dtype() == at::kHalf ? fa_backward_fp16 : fa_backward_fp32;
  check_fa(fn(dout.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
              logsumexp.data_ptr<float>(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), b, h, n, d,
              causal ? 1 : 0, ws_ptr(ws), ws_bytes, cur_stream()));
  return std::make_tuple(dq, dk, dv);
}

// token_eviction (flash_attn_kernel.cu:4296-4344): (k_out, v_out, valid_mask).
std::tuple<at::Tensor, at::Tensor, at::Tensor> token_eviction(at::Tensor k, at::Tensor v, at::Tensor attn_scores,
                                                              int num_evict) {
  CHECK_INPUT(k);
  CHECK_INPUT(v);
  CHECK_INPUT(attn_scores);
  TORCH_CHECK(k.dtype() == at::kHalf, "k must be float16");
  TORCH_CHECK(v.dtype() == at::kHalf, "v must be float16");
  TORCH_CHECK(attn_scores.dtype() == at::kFloat, "attn_scores must be float32");
  CHECK_DIM(k, 4);
  TORCH_CHECK(v.sizes() == k.sizes(), "k and v must have the same shape");
  CHECK_SAME_DEVICE(k, v);
  CHECK_SAME_DEVICE(k, attn_scores);
  const auto B = k.size(0), H = k.size(1), N = k.size(2), D = k.size(3);
  CHECK_DIM(attn_scores, 2);
  TORCH_CHECK(attn_scores.size(0) == B, "attn_scores batch mismatch");
  TORCH_CHECK(attn_scores.size(1) == N, "attn_scores length mismatch");
  TORCH_CHECK(N <= 1024, "N must be <= 1024 for token eviction");
  HIPGuardMasqueradingAsCUDA guard(k.device());
  auto k_out = at::empty_like(k);
  auto v_out = at::empty_like(v);
  auto mask = at::empty({B, N}, k.options().dtype(at::kInt));
  check_fa(fa_token_eviction(k.data_ptr(), v.data_ptr(), attn_scores.data_ptr<float>(), k_out.data_ptr(),
                             v_out.data_ptr(), mask.data_ptr<int32_t>(), to_int(B, "B"), to_int(H, "H_KV"),
                             to_int(N, "N"), to_int(D, "D"), num_evict, cur_stream()));
  return std::make_tuple(k_out, v_out, mask);
}

// speculative_verify (flash_attn_kernel.cu:3972-4018): (accepted_count, output_tokens).
std::tuple<at::Tensor, at::Tensor> speculative_verify(at::Tensor target_probs, at::Tensor draft_probs,
                                                      at::Tensor draft_tokens, at::Tensor random_vals, int K) {
  CHECK_INPUT(target_probs);
  CHECK_INPUT(draft_probs);
  CHECK_INPUT(draft_tokens);
  CHECK_INPUT(random_vals);
  TORCH_CHECK(target_probs.dtype() == at::kFloat, "target_probs must be float32");
  TORCH_CHECK(draft_probs.dtype() == at::kFloat, "draft_probs must be float32");
  TORCH_CHECK(draft_tokens.dtype() == at::kLong, "draft_tokens must be int64");
  TORCH_CHECK(random_vals.dtype() == at::kFloat, "random_vals must be float32");
  CHECK_DIM(target_probs, 3);
  const auto B = target_probs.size(0), V = target_probs.size(2);
  TORCH_CHECK(K <= 8, "K must be <= SPEC_MAX_K(8)");
  TORCH_CHECK(K >= 1, "K must be >= 1");
  TORCH_CHECK(target_probs.size(1) == K + 1, "target_probs must have K+1 positions");
  CHECK_DIM(draft_probs, 3);
  TORCH_CHECK(draft_probs.size(0) == B && draft_probs.size(2) == V, "draft_probs must be [B, K, vocab_size]");
  TORCH_CHECK(draft_probs.size(1) == K, "draft_probs must have K positions");
  CHECK_DIM(draft_tokens, 2);
  TORCH_CHECK(draft_tokens.size(0) == B, "draft_tokens batch mismatch");
  TORCH_CHECK(draft_tokens.size(1) == K, "draft_tokens must have K tokens");
  TORCH_CHECK(random_vals.numel() >= B * K, "random_vals must hold B*K values");
  CHECK_SAME_DEVICE(target_probs, draft_probs);
  CHECK_SAME_DEVICE(target_probs, draft_tokens);
  CHECK_SAME_DEVICE(target_probs, random_vals);
  HIPGuardMasqueradingAsCUDA guard(target_probs.device());
  auto accepted = at::empty({B}, target_probs.options().dtype(at::kInt));
  auto tokens = at::empty({B, K + 1}, target_probs.options().dtype(at::kLong));
  check_fa(fa_speculative_verify(target_probs.data_ptr<float>(), draft_probs.data_ptr<float>(),
                                 draft_tokens.data_ptr<int64_t>(), random_vals.data_ptr<float>(),
                                 accepted.data_ptr<int32_t>(), tokens.data_ptr<int64_t>(), to_int(B, "B"), K,
                                 to_int(V, "vocab_size"), cur_stream()));
  return std::make_tuple(accepted, tokens);
}

// ---------------------------------------------------------------------------
// Tensor-parallel helpers: same-device head-range copies and the fp16 accumulate.

// cross_gpu_allreduce_fp16 (flash_attn_kernel.cu:597-620)
void cross_gpu_allreduce_fp16(at::Tensor dst_tensor, at::Tensor src_tensor) {
  CHECK_INPUT(dst_tensor);
  CHECK_INPUT(src_tensor);
  TORCH_CHECK(dst_tensor.dtype() == at::kHalf, "dst must be float16");
  TORCH_CHECK(src_tensor.dtype() == at::kHalf, "src must be float16");
  TORCH_CHECK(dst_tensor.numel() == src_tensor.numel(), "size mismatch");
  CHECK_SAME_DEVICE(dst_tensor, src_tensor);
  HIPGuardMasqueradingAsCUDA guard(dst_tensor.device());
  check_fa(fa_cross_gpu_allreduce_fp16(dst_tensor.data_ptr(), src_tensor.data_ptr(),
                                       static_cast<size_t>(dst_tensor.numel()), cur_stream()));
}

// Shared checks of scatter_heads_forward / gather_heads_forward
// (flash_attn_kernel.cu:685-701, :728-744).
void check_head_range(const at::Tensor& full_tensor, const at::Tensor& local_tensor, int total_heads,
                      int local_head_start, int local_head_count) {
  CHECK_INPUT(full_tensor);
  CHECK_INPUT(local_tensor);
  TORCH_CHECK(full_tensor.dtype() == at::kHalf, "full_tensor must be float16");
  TORCH_CHECK(local_tensor.dtype() == at::kHalf, "local_tensor must be float16");
  CHECK_DIM(full_tensor, 4);
  CHECK_DIM(local_tensor, 4);
  CHECK_SAME_DEVICE(full_tensor, local_tensor);
  const auto B = full_tensor.size(0), N = full_tensor.size(2), D = full_tensor.size(3);
  TORCH_CHECK(full_tensor.size(1) == total_heads, "full_tensor head count must match total_heads");
  TORCH_CHECK(local_tensor.size(1) == local_head_count, "local_tensor head count must match local_head_count");
  TORCH_CHECK(local_head_start >= 0 && local_head_count >= 0, "head range must be non-negative");
  TORCH_CHECK(local_head_start + local_head_count <= total_heads, "head range exceeds total_heads");
  TORCH_CHECK(local_tensor.size(0) == B && local_tensor.size(2) == N && local_tensor.size(3) == D,
              "local_tensor shape must match full_tensor except for head count");
}

// scatter_heads_forward (flash_attn_kernel.cu:678-719)
void scatter_heads(at::Tensor full_tensor, at::Tensor local_tensor, int total_heads, int local_head_start,
                   int local_head_count) {
  check_head_range(full_tensor, local_tensor, total_heads, local_head_start, local_head_count);
  HIPGuardMasqueradingAsCUDA guard(full_tensor.device());
  check_fa(fa_scatter_heads(full_tensor.data_ptr(), local_tensor.data_ptr(), to_int(full_tensor.size(0), "B"),
                            total_heads, local_head_start, local_head_count, to_int(full_tensor.size(2), "N"),
                            to_int(full_tensor.size(3), "D"), cur_stream()));
}

// gather_heads_forward (flash_attn_kernel.cu:721-762)
void gather_heads(at::Tensor full_tensor, at::Tensor local_tensor, int total_heads, int local_head_start,
                  int local_head_count) {
  check_head_range(full_tensor, local_tensor, total_heads, local_head_start, local_head_count);
  HIPGuardMasqueradingAsCUDA guard(full_tensor.device());
  check_fa(fa_gather_heads(full_tensor.data_ptr(), local_tensor.data_ptr(), to_int(full_tensor.size(0), "B"),
                           total_heads, local_head_start, local_head_count, to_int(full_tensor.size(2), "N"),
                           to_int(full_tensor.size(3), "D"), cur_stream()));
}

// forward_decode_int8_kv_cache_gqa (flash_attn_kernel.cu:4161-4221)
at::Tensor forward_decode_int8_kv_cache_gqa(at::Tensor q, at::Tensor k_int8, at::Tensor v_int8, at::Tensor k_scale,
                                            at::Tensor v_scale, int cache_len) {
  CHECK_INPUT(q);
  CHECK_INPUT(k_int8);
  CHECK_INPUT(v_int8);
  CHECK_INPUT(k_scale);
  CHECK_INPUT(v_scale);
  TORCH_CHECK(q.dtype() == at::kHalf, "q must be float16");
  TORCH_CHECK(k_int8.dtype() == at::kChar, "k_int8 must be int8");
  TORCH_CHECK(v_int8.dtype() == at::kChar, "v_int8 must be int8");
  TORCH_CHECK(k_scale.dtype() == at::kHalf, "k_scale must be float16");
  TORCH_CHECK(v_scale.dtype() == at::kHalf, "v_scale must be float16");
  TORCH_CHECK(q.size(2) == 1, "q sequence length must be 1 for decode mode");
  const auto B = q.size(0), H_Q = q.size(1), H_KV = k_int8.size(1), N = k_int8.size(2), D = q.size(3);
  TORCH_CHECK(H_Q >= H_KV, "H_Q must be >= H_KV");
  TORCH_CHECK(H_Q % H_KV == 0, "H_Q must be divisible by H_KV");
  TORCH_CHECK(D <= kMaxDLarge, "D must be <= MAX_D_LARGE(256)");
  TORCH_CHECK(k_int8.size(3) == D, "k_int8 last dim must match D");
  TORCH_CHECK(v_int8.size(3) == D, "v_int8 last dim must match D");
  TORCH_CHECK(k_scale.size(2) == N, "k_scale size mismatch");
  TORCH_CHECK(v_scale.size(2) == N, "v_scale size mismatch");
  // The reference reads these without checking them; here a mismatch is an error.
  TORCH_CHECK(q.dim() == 4 && k_int8.dim() == 4 && k_int8.sizes() == v_int8.sizes() && k_int8.size(0) == B,
              "k_int8 and v_int8 must be [B, H_KV, N, D]");
  TORCH_CHECK(k_scale.dim() == 3 && k_scale.size(0) == B && k_scale.size(1) == H_KV && k_scale.sizes() == v_scale.sizes(),
              "k_scale and v_scale must be [B, H_KV, N]");
  HIPGuardMasqueradingAsCUDA guard(q.device());
  auto out = at::empty({B, H_Q, 1, D}, q.options());
  const int b = to_int(B, "B"), hq = to_int(H_Q, "H_Q"), hkv = to_int(H_KV, "H_KV"), n = to_int(N, "N"),
            d = to_int(D, "D");
  auto ws = decode_workspace(q, b, hq, hkv, n, d);
  check_fa(fa_decode_int8_kv_cache_gqa(q.data_ptr(), k_int8.data_ptr(), v_int8.data_ptr(), k_scale.data_ptr(),
                                       v_scale.data_ptr(), out.data_ptr(), b, hq, hkv, n, d, cache_len,
                                       ws_ptr(ws), ws_bytes(ws), cur_stream()));
  return out;
}

// forward_decode_sliding_window_gqa (flash_attn_kernel.cu:4484-4535): keys k < sink_size
// plus the window [max(0, min(cache_len+1, N) - window_size), cache_len]; `causal` is unused.
at::Tensor forward_decode_sliding_window_gqa(at::Tensor q, at::Tensor k, at::Tensor v, bool causal, int cache_len,
                                             int window_size, int sink_size) {
  (void)causal;
  CHECK_INPUT(q);
  CHECK_INPUT(k);
  CHECK_INPUT(v);
  TORCH_CHECK(q.dtype() == at::kHalf, "q must be float16");
  TORCH_CHECK(q.size(2) == 1, "q sequence length must be 1 for decode mode");
  const auto H_Q = q.size(1), H_KV = k.size(1);
  TORCH_CHECK(H_Q >= H_KV, "H_Q must be >= H_KV");
  TORCH_CHECK(H_Q % H_KV == 0, "H_Q must be divisible by H_KV");
  TORCH_CHECK(q.size(3) <= kMaxDLarge, "D must be <= MAX_D_LARGE(256)");
  // The reference reads k/v without checking them; here a mismatch is an error.
  check_decode_gqa_input_shapes(q, k, v);
  TORCH_CHECK(k.dtype() == at::kHalf && v.dtype() == at::kHalf, "k, v must be float16");
  HIPGuardMasqueradingAsCUDA guard(q.device());
  auto out = at::empty({q.size(0), H_Q, 1, q.size(3)}, q.options());
  const int B = to_int(q.size(0), "B"), N = to_int(k.size(2), "N"), D = to_int(q.size(3), "D");
  auto ws = decode_workspace(q, B, to_int(H_Q, "H_Q"), to_int(H_KV, "H_KV"), N, D);
  check_fa(fa_decode_sliding_window_gqa(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), B,
                                        to_int(H_Q, "H_Q"), to_int(H_KV, "H_KV"), N, D, cache_len, window_size,
                                        sink_size, ws_ptr(ws), ws_bytes(ws), cur_stream()));
  return out;
}

// ---------------------------------------------------------------------------
// Host-to-device transfer helpers and the decode step that overlaps them

void check_hip(hipError_t err, const char* what) {
  TORCH_CHECK(err == hipSuccess, what, ": ", hipGetErrorString(err));
}

// async_h2d_transfer (flash_attn_kernel.cu:3714-3738)
void async_h2d_transfer(at::Tensor dst, at::Tensor src, int64_t stream_int) {
  TORCH_CHECK(dst.is_cuda(), "dst must be a CUDA tensor");
  TORCH_CHECK(!src.is_cuda(), "src must be a CPU tensor");
  TORCH_CHECK(dst.dtype() == src.dtype(), "dtype must match");
  TORCH_CHECK(dst.numel() == src.numel(), "size must match");
  TORCH_CHECK(src.is_pinned(), "src must be pinned memory for async transfer");
  TORCH_CHECK(dst.is_contiguous(), "dst must be contiguous");
  TORCH_CHECK(src.is_contiguous(), "src must be contiguous");
  HIPGuardMasqueradingAsCUDA guard(dst.device());
  const size_t nbytes = static_cast<size_t>(dst.numel()) * dst.element_size();
  check_hip(hipMemcpyAsync(dst.data_ptr(), src.data_ptr(), nbytes, hipMemcpyHostToDevice,
                           reinterpret_cast<hipStream_t>(stream_int)),
            "async_h2d_transfer");
}

// alloc_pinned_tensor (flash_attn_kernel.cu:3740-3750): page-locked host tensor.
at::Tensor alloc_pinned_tensor(std::vector<int64_t> sizes, int dtype_int) {
  auto options = at::TensorOptions().dtype(static_cast<at::ScalarType>(dtype_int)).device(at::kCPU).pinned_memory(true);
  return at::empty(sizes, options);
}

// pipeline_decode_step_out (flash_attn_kernel.cu:3786-3849): GQA decode on the
// compute stream, then the three host-to-device copies on the transfer stream.
std::tuple<at::Tensor, at::Tensor, at::Tensor> pipeline_decode_step_out(
    at::Tensor out, at::Tensor q_compute, at::Tensor k_compute, at::Tensor v_compute, at::Tensor q_transfer,
    at::Tensor k_transfer, at::Tensor v_transfer, at::Tensor q_h2d_dst, at::Tensor k_h2d_dst, at::Tensor v_h2d_dst,
    bool causal, int cache_len, int64_t compute_stream_int, int64_t transfer_stream_int) {
  CHECK_INPUT(q_compute);
  CHECK_INPUT(k_compute);
  CHECK_INPUT(v_compute);
  check_decode_gqa_input_shapes(q_compute, k_compute, v_compute);
  TORCH_CHECK(q_compute.dtype() == at::kHalf, "q_compute, k_compute, v_compute must be float16");
  TORCH_CHECK(q_compute.size(2) == 1, "q_compute sequence length must be 1 for decode mode");
  check_decode_gqa_output_tensor(out, q_compute);
  TORCH_CHECK(q_compute.size(3) <= kMaxDLarge, "D must be <= MAX_D_LARGE(256)");
  check_cache_len(cache_len, k_compute.size(2));
  TORCH_CHECK(!q_transfer.is_cuda() && !k_transfer.is_cuda() && !v_transfer.is_cuda(),
              "transfer source tensors must be CPU tensors");
  TORCH_CHECK(q_transfer.is_pinned() && k_transfer.is_pinned() && v_transfer.is_pinned(),
              "transfer source tensors must be pinned");
  TORCH_CHECK(q_h2d_dst.is_cuda() && k_h2d_dst.is_cuda() && v_h2d_dst.is_cuda(),
              "transfer destination tensors must be CUDA tensors");
  TORCH_CHECK(q_transfer.dtype() == q_h2d_dst.dtype() && k_transfer.dtype() == k_h2d_dst.dtype() &&
                  v_transfer.dtype() == v_h2d_dst.dtype(),
              "transfer tensor dtypes must match");
  TORCH_CHECK(q_transfer.numel() == q_h2d_dst.numel() && k_transfer.numel() == k_h2d_dst.numel() &&
                  v_transfer.numel() == v_h2d_dst.numel(),
              "transfer tensor sizes must match");
  TORCH_CHECK(q_h2d_dst.device() == q_compute.device() && k_h2d_dst.device() == q_compute.device() &&
                  v_h2d_dst.device() == q_compute.device(),
              "transfer destinations must be on compute device");
  TORCH_CHECK(q_compute.size(1) % k_compute.size(1) == 0, "H_Q must be divisible by H_KV");
  HIPGuardMasqueradingAsCUDA guard(q_compute.device());
  {
    auto cs = c10::hip::getStreamFromExternalMasqueradingAsCUDA(reinterpret_cast<hipStream_t>(compute_stream_int),
                                                                q_compute.device().index());
    HIPStreamGuardMasqueradingAsCUDA sguard(cs);
    launch_decode(q_compute, k_compute, v_compute, out, causal, cache_len);
  }
  if (q_transfer.numel() > 0 && q_h2d_dst.numel() > 0) {
    hipStream_t ts = reinterpret_cast<hipStream_t>(transfer_stream_int);
    const at::Tensor* pairs[3][2] = {{&q_h2d_dst, &q_transfer}, {&k_h2d_dst, &k_transfer}, {&v_h2d_dst, &v_transfer}};
    for (auto& pr : pairs)
      check_hip(hipMemcpyAsync(pr[0]->data_ptr(), pr[1]->data_ptr(),
                               static_cast<size_t>(pr[0]->numel()) * pr[0]->element_size(), hipMemcpyHostToDevice, ts),
                "pipeline_decode_step");
  }
  return std::make_tuple(out, q_h2d_dst, k_h2d_dst);
}

// pipeline_decode_step (flash_attn_kernel.cu:3752-3784)
std::tuple<at::Tensor, at::Tensor, at::Tensor> pipeline_decode_step(
    at::Tensor q_compute, at::Tensor k_compute, at::Tensor v_compute, at::Tensor q_transfer, at::Tensor k_transfer,
    at::Tensor v_transfer, at::Tensor q_h2d_dst, at::Tensor k_h2d_dst, at::Tensor v_h2d_dst, bool causal,
    int cache_len, int64_t compute_stream_int, int64_t transfer_stream_int) {
  auto out = at::empty({q_compute.size(0), q_compute.size(1), 1, q_compute.size(3)}, q_compute.options());
  return pipeline_decode_step_out(out, q_compute, k_compute, v_compute, q_transfer, k_transfer, v_transfer, q_h2d_dst,
                                  k_h2d_dst, v_h2d_dst, causal, cache_len, compute_stream_int, transfer_stream_int);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("forward_fp16", &forward_fp16, "Flash attention forward, fp16 (MI355X MFMA)");
  m.def("forward_fp16_warp", &forward_fp16_warp, "Flash attention forward, fp16 (MI355X MFMA)");
  m.def("forward_fp16_wmma", &forward_fp16_wmma, "Flash attention forward, fp16 (MI355X MFMA)");
  m.def("forward_prefill_gqa_fp16", &forward_prefill_gqa_fp16, "GQA/MQA prefill, fp16 (MI355X MFMA)");
  m.def("forward_prefill_gqa_fp16_out", &forward_prefill_gqa_fp16_out, "GQA/MQA prefill into out (MI355X)");
  m.def("forward_prefill_gqa_fp16_warp", &forward_prefill_gqa_fp16_warp, "GQA/MQA prefill, fp16 (MI355X MFMA)");
  m.def("forward_decode_fp16", &forward_decode_fp16, "MHA decode with KV cache (MI355X split-KV)");
  m.def("forward_decode_gqa_fp16", &forward_decode_gqa_fp16, "GQA/MQA decode with KV cache (MI355X split-KV)");
  m.def("forward_decode_gqa_fp16_out", &forward_decode_gqa_fp16_out, "GQA/MQA decode into out (MI355X)");
  m.def("forward_decode_gqa_fp16_stream", &forward_decode_gqa_fp16_stream, "GQA decode on a given stream");
  m.def("forward_continuous_batching_fp16", &forward_continuous_batching_fp16,
        "Continuous-batching GQA decode (MI355X split-KV)");
  m.def("forward_paged_decode_gqa_fp16", &forward_paged_decode_gqa_fp16, "Paged GQA decode (MI355X split-KV)");
  m.def("forward_decode_int8_gqa", &forward_decode_int8_gqa, "INT8 GQA decode (MI355X sdot4)");
  m.def("forward_varlen_prefill_fp16", &forward_varlen_prefill_fp16, "Packed varlen prefill (MI355X MFMA)");
  m.def("forward_varlen_prefill_fp16_stream", &forward_varlen_prefill_fp16_stream,
        "Packed varlen prefill on a given stream");
  m.def("forward_decode_int8_kv_cache_gqa", &forward_decode_int8_kv_cache_gqa,
        "GQA decode with an INT8 KV cache and per-token scales (MI355X split-KV)");
  m.def("forward_decode_sliding_window_gqa", &forward_decode_sliding_window_gqa,
        "Sliding-window + attention-sink GQA decode (MI355X split-KV)");
  m.def("async_h2d_transfer", &async_h2d_transfer, "Async host-to-device copy from pinned memory");
  m.def("alloc_pinned_tensor", &alloc_pinned_tensor, "Allocate a pinned (page-locked) host tensor");
  m.def("pipeline_decode_step", &pipeline_decode_step, "GQA decode on one stream, H2D copies on another");
  m.def("pipeline_decode_step_out", &pipeline_decode_step_out,
        "GQA decode into out on one stream, H2D copies on another");
  m.def("forward", &forward_fp32, "Flash attention forward, fp32 (MI355X fp32 MFMA)");
  m.def("forward_with_lse", &forward_with_lse, "fp32 forward with logsumexp (MI355X)");
  m.def("forward_fp16_with_lse", &forward_fp16_with_lse, "fp16 forward with logsumexp (MI355X MFMA)");
  m.def("backward", &backward, "Attention backward for MHA, fp32/fp16 (MI355X MFMA)");
  m.def("token_eviction", &token_eviction, "KV-cache token eviction by attention score (MI355X)");
  m.def("speculative_verify", &speculative_verify, "Speculative decoding verify (MI355X)");
  m.def("cross_gpu_allreduce_fp16", &cross_gpu_allreduce_fp16, "fp16 dst += src on one device (MI355X)");
  m.def("scatter_heads", &scatter_heads, "Copy a head range of full into local (MI355X)");
  m.def("gather_heads", &gather_heads, "Copy local into a head range of full (MI355X)");
  m.def("_fa_version", []() { return std::string(fa_version()); });
}
