// Training path: C ABI of the fp32 forward with log-sum-exp and of the
// attention backward, and the instantiations of the fp16 backward and fp32
// forward kernels (built with MFMA accumulators in VGPRs; the fp32 backward
// lives in train_fp32.hip).
#include <mutex>
#include <vector>

#include "capi_internal.h"
#include "train_kernels.h"

namespace fa {
namespace train {

hipStream_t backward_side_stream(hipStream_t caller, int which) {
  // Side streams per (device, caller stream): backward calls issued on
  // different caller streams (threads, serving loops) keep their concurrency
  // instead of queueing on one shared pair.  At most kMaxCallers pairs per
  // device are made; past that the oldest pair is handed to the new caller
  // (its work then queues behind the other caller's, which is still correct).
  // Streams are never destroyed, so a pair handed over can have work pending.
  constexpr int kMaxDevices = 64;
  constexpr size_t kMaxCallers = 16;
  struct Entry {
    hipStream_t caller;
    hipStream_t side[2];
  };
  static std::mutex mu;
  static std::vector<Entry> pairs[kMaxDevices];
  static size_t next_reuse[kMaxDevices] = {};
  int dev = 0;
  if (which < 0 || which > 1 || hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  std::vector<Entry>& list = pairs[dev];
  for (Entry& e : list)
    if (e.caller == caller) return e.side[which];
  if (list.size() >= kMaxCallers) {
    Entry& e = list[next_reuse[dev]++ % list.size()];
    e.caller = caller;
    return e.side[which];
  }
  Entry e = {caller, {nullptr, nullptr}};
  for (int i = 0; i < 2; ++i) {
    if (hipStreamCreateWithFlags(&e.side[i], hipStreamNonBlocking) != hipSuccess) {
      (void)hipGetLastError();  // leave no sticky error for check_launch
      if (i == 1) (void)hipStreamDestroy(e.side[0]);
      return nullptr;
    }
  }
  list.push_back(e);
  return e.side[which];
}

bool backward_events(hipEvent_t (&ev)[4]) {
  constexpr int kMaxDevices = 64;
  thread_local hipEvent_t events[kMaxDevices][4] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
  for (int e = 0; e < 4; ++e) {
    if (events[dev][e] == nullptr &&
        hipEventCreateWithFlags(&events[dev][e], hipEventDisableTiming) != hipSuccess) {
      events[dev][e] = nullptr;
      return false;
    }
    ev[e] = events[dev][e];
  }
  return true;
}

static int check_sizes(const char* fn, int B, int H, int N, int D) {
  if (B < 0 || H <= 0 || N < 0 || D <= 0)
    return set_error(FA_ERR_INVALID_ARG, "%s: bad sizes (B=%d H=%d N=%d D=%d)", fn, B, H, N, D);
  if (D > 128) return set_error(FA_ERR_UNSUPPORTED, "%s: D=%d exceeds 128", fn, D);
  if ((static_cast<long long>(B) * H + 8) * ceil_div(N, kBlockRows) > 0x7fffffffLL)
    return set_error(FA_ERR_UNSUPPORTED, "%s: problem too large for one launch", fn);
  return FA_OK;
}

}  // namespace train
}  // namespace fa

using namespace fa;
using namespace fa::train;

extern "C" int fa_prefill_fp32(const void* q, const void* k, const void* v, void* o, float* lse, int B, int H,
                               int N, int D, int causal, void* stream) {
  const char* fn = "fa_prefill_fp32";
  if (int rc = check_sizes(fn, B, H, N, D)) return rc;
  if (B == 0 || N == 0) return FA_OK;
  if (!q || !k || !v || !o) return set_error(FA_ERR_INVALID_ARG, "%s: null tensor pointer", fn);
  TrainParams p = {};
  p.q = q; p.k = k; p.v = v; p.out = o; p.lse = lse;
  p.BH = B * H; p.N = N; p.D = D; p.causal = causal ? 1 : 0;
  p.nblk = ceil_div(N, kBlockRows);
  p.scale = 1.0f / sqrtf(static_cast<float>(D));
  p.scale_log2 = p.scale * kLog2e;
  const bool vec = aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o);
  launch_forward_fp32(p, vec, static_cast<hipStream_t>(stream));
  return check_launch(fn);
}

extern "C" size_t fa_backward_workspace_size(int B, int H, int N) {
  if (B <= 0 || H <= 0 || N <= 0) return 0;
  return static_cast<size_t>(B) * H * N * sizeof(float);
}

static int backward_common(const char* fn, bool fp32, const void* dout, const void* q, const void* k,
                           const void* v, const void* out, const float* lse, void* dq, void* dk, void* dv,
                           int B, int H, int N, int D, int causal, void* workspace, size_t workspace_bytes,
                           void* stream) {
  if (int rc = check_sizes(fn, B, H, N, D)) return rc;
  if (B == 0 || N == 0) return FA_OK;
  if (!dout || !q || !k || !v || !out || !lse || !dq || !dk || !dv)
    return set_error(FA_ERR_INVALID_ARG, "%s: null tensor pointer", fn);
  const size_t need = fa_backward_workspace_size(B, H, N);
  if (!workspace || workspace_bytes < need)
    return set_error(FA_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given", fn, need,
                     workspace ? workspace_bytes : static_cast<size_t>(0));
  TrainParams p = {};
  p.q = q; p.k = k; p.v = v; p.o = out; p.dout = dout;
  p.out = dq; p.dk = dk; p.dv = dv;
  p.lse = const_cast<float*>(lse);
  p.delta = static_cast<float*>(workspace);
  p.BH = B * H; p.N = N; p.D = D; p.causal = causal ? 1 : 0;
  p.nblk = ceil_div(N, kBlockRows);
  p.scale = 1.0f / sqrtf(static_cast<float>(D));
  p.scale_log2 = p.scale * kLog2e;
  const bool vec = aligned16(dout) && aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out) &&
                   aligned16(dq) && aligned16(dk) && aligned16(dv);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (fp32) backward_fp32(p, vec, st);
  else launch_backward<half_t>(p, vec, st);
  return check_launch(fn);
}

extern "C" int fa_backward_fp16(const void* dout, const void* q, const void* k, const void* v, const void* out,
                                const float* lse, void* dq, void* dk, void* dv, int B, int H, int N, int D,
                                int causal, void* workspace, size_t workspace_bytes, void* stream) {
  return backward_common("fa_backward_fp16", false, dout, q, k, v, out, lse, dq, dk, dv, B, H, N, D, causal,
                         workspace, workspace_bytes, stream);
}

extern "C" int fa_backward_fp32(const void* dout, const void* q, const void* k, const void* v, const void* out,
                                const float* lse, void* dq, void* dk, void* dv, int B, int H, int N, int D,
                                int causal, void* workspace, size_t workspace_bytes, void* stream) {
  return backward_common("fa_backward_fp32", true, dout, q, k, v, out, lse, dq, dk, dv, B, H, N, D, causal,
                         workspace, workspace_bytes, stream);
}
