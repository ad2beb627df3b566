// Head-range copies and the fp16 accumulate of the tensor-parallel helpers,
// for gfx950.
//
// The reference's three helpers are same-device kernels (every wrapper checks
// CHECK_SAME_DEVICE, flash_attn_kernel.cu:597-762):
//   scatter_heads  local[b, h] = full[b, start + h]   for h < count
//   gather_heads   full[b, start + h] = local[b, h]
//   cross_gpu_allreduce_fp16   dst[i] = half(float(dst[i]) + float(src[i]))
// The reference runs one thread per fp16 element and recomputes (b, h, rest)
// with three integer divisions per element.  In [B, H, N, D] layout a head
// range of one batch row is ONE contiguous run of count*N*D elements, so both
// copies are B runs of equal length with different strides: `copy_runs_kernel`
// streams them with 16-byte loads and stores (four per lane in flight), no
// per-element index arithmetic.  The accumulate is an elementwise stream with
// the same vector width; each element is widened to fp32, added once (RNE) and
// narrowed once (RNE), exactly the reference's conversions.  All three are
// HBM-bound: algorithmic bytes = 2 x copied bytes (copies), 3 x dst bytes
// (accumulate: read dst and src, write dst).
#include "capi_internal.h"
#include "common.h"

namespace fa {
namespace tp {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;  // 16-byte vectors per lane per iteration
constexpr int kMaxGridY = 65535;

// Copies `rows` runs of `run` elements of type T: run r goes from
// src + r*src_stride to dst + r*dst_stride.  Grid x covers one run in chunks
// of kThreads*kUnroll elements; grid y walks the runs.
template <typename T>
__global__ __launch_bounds__(kThreads) void copy_runs_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                             int64_t rows, int64_t run, int64_t src_stride,
                                                             int64_t dst_stride) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kThreads * kUnroll) + threadIdx.x;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const T* s = src + r * src_stride;
    T* d = dst + r * dst_stride;
    T buf[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + u * kThreads;
      if (i < run) buf[u] = s[i];
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + u * kThreads;
      if (i < run) d[i] = buf[u];
    }
  }
}

__device__ __forceinline__ half8_t add_f16x8(half8_t a, half8_t b) {
  half8_t r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = static_cast<half_t>(static_cast<float>(a[j]) + static_cast<float>(b[j]));
  return r;
}

// dst[i] = half(float(dst[i]) + float(src[i])) over n8 vectors of 8 elements;
// grid-stride so any n fits one launch.  `src` may equal `dst` (then dst
// doubles, as in the reference), so neither pointer is __restrict__.
__global__ __launch_bounds__(kThreads) void add_vec_kernel(half8_t* dst, const half8_t* src, int64_t n8) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads * kUnroll;
  for (int64_t i0 = static_cast<int64_t>(blockIdx.x) * (kThreads * kUnroll) + threadIdx.x; i0 < n8; i0 += stride) {
    half8_t a[kUnroll], b[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = i0 + u * kThreads;
      if (i < n8) {
        a[u] = dst[i];
        b[u] = src[i];
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = i0 + u * kThreads;
      if (i < n8) dst[i] = add_f16x8(a[u], b[u]);
    }
  }
}

// Scalar form for tails and unaligned buffers.
__global__ __launch_bounds__(kThreads) void add_scalar_kernel(half_t* dst, const half_t* src, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride)
    dst[i] = static_cast<half_t>(static_cast<float>(dst[i]) + static_cast<float>(src[i]));
}

// Launches the run copy with 16-byte elements when every run start is 16-byte
// aligned and the run length is a whole number of 16-byte vectors, else with
// 2-byte elements.  Sizes are in fp16 elements.
int copy_runs(const half_t* src, half_t* dst, int64_t rows, int64_t run, int64_t src_stride, int64_t dst_stride,
              hipStream_t st, const char* fn) {
  if (rows == 0 || run == 0) return FA_OK;
  const int gy = static_cast<int>(rows < kMaxGridY ? rows : kMaxGridY);
  if (run % 8 == 0 && src_stride % 8 == 0 && dst_stride % 8 == 0 && aligned16(src) && aligned16(dst)) {
    const int64_t run8 = run / 8;
    const int64_t gx = (run8 + kThreads * kUnroll - 1) / (kThreads * kUnroll);
    if (gx > INT32_MAX) return set_error(FA_ERR_UNSUPPORTED, "%s: run of %lld elements too long", fn, (long long)run);
    hipLaunchKernelGGL(copy_runs_kernel<u32x4>, dim3(static_cast<unsigned>(gx), gy), dim3(kThreads), 0, st,
                       reinterpret_cast<const u32x4*>(src), reinterpret_cast<u32x4*>(dst), rows, run8,
                       src_stride / 8, dst_stride / 8);
  } else {
    const int64_t gx = (run + kThreads * kUnroll - 1) / (kThreads * kUnroll);
    if (gx > INT32_MAX) return set_error(FA_ERR_UNSUPPORTED, "%s: run of %lld elements too long", fn, (long long)run);
    hipLaunchKernelGGL(copy_runs_kernel<uint16_t>, dim3(static_cast<unsigned>(gx), gy), dim3(kThreads), 0, st,
                       reinterpret_cast<const uint16_t*>(src), reinterpret_cast<uint16_t*>(dst), rows, run,
                       src_stride, dst_stride);
  }
  return check_launch(fn);
}

// Common argument checks of the two head-range copies; on success sets the
// run geometry (elements per head, run length, full-tensor row stride).
int head_range_geometry(const void* full, const void* local, int B, int total_heads, int head_start, int head_count,
                        int N, int D, const char* fn, int64_t& head_elems, int64_t& run, int64_t& full_stride) {
  if (B < 0 || total_heads < 0 || N < 0 || D < 0)
    return set_error(FA_ERR_INVALID_ARG, "%s: bad sizes (B=%d total_heads=%d N=%d D=%d)", fn, B, total_heads, N, D);
  if (head_start < 0 || head_count < 0 || static_cast<int64_t>(head_start) + head_count > total_heads)
    return set_error(FA_ERR_INVALID_ARG, "%s: head range [%d, %d+%d) outside [0, %d)", fn, head_start, head_start,
                     head_count, total_heads);
  head_elems = static_cast<int64_t>(N) * D;
  run = head_elems * head_count;
  full_stride = head_elems * total_heads;
  if (B > 0 && run > 0 && (!full || !local)) return set_error(FA_ERR_INVALID_ARG, "%s: null pointer", fn);
  return FA_OK;
}

}  // namespace tp
}  // namespace fa

using namespace fa;

extern "C" int fa_scatter_heads(const void* full, void* local, int B, int total_heads, int head_start, int head_count,
                                int N, int D, void* stream) {
  const char* fn = "fa_scatter_heads";
  int64_t head_elems, run, full_stride;
  const int rc = tp::head_range_geometry(full, local, B, total_heads, head_start, head_count, N, D, fn, head_elems,
                                         run, full_stride);
  if (rc != FA_OK) return rc;
  const half_t* src = static_cast<const half_t*>(full) + head_elems * head_start;
  return tp::copy_runs(src, static_cast<half_t*>(local), B, run, full_stride, run, static_cast<hipStream_t>(stream),
                       fn);
}

extern "C" int fa_gather_heads(void* full, const void* local, int B, int total_heads, int head_start, int head_count,
                               int N, int D, void* stream) {
  const char* fn = "fa_gather_heads";
  int64_t head_elems, run, full_stride;
  const int rc = tp::head_range_geometry(full, local, B, total_heads, head_start, head_count, N, D, fn, head_elems,
                                         run, full_stride);
  if (rc != FA_OK) return rc;
  half_t* dst = static_cast<half_t*>(full) + head_elems * head_start;
  return tp::copy_runs(static_cast<const half_t*>(local), dst, B, run, run, full_stride,
                       static_cast<hipStream_t>(stream), fn);
}

extern "C" int fa_cross_gpu_allreduce_fp16(void* dst, const void* src, size_t n, void* stream) {
  const char* fn = "fa_cross_gpu_allreduce_fp16";
  if (n == 0) return FA_OK;
  if (!dst || !src) return set_error(FA_ERR_INVALID_ARG, "%s: null pointer", fn);
  if (n > static_cast<size_t>(INT64_MAX / 2)) return set_error(FA_ERR_INVALID_ARG, "%s: n too large", fn);
  hipStream_t st = static_cast<hipStream_t>(stream);
  half_t* d = static_cast<half_t*>(dst);
  const half_t* s = static_cast<const half_t*>(src);
  const int64_t total = static_cast<int64_t>(n);
  int64_t done = 0;
  // Enough workgroups for several resident rounds on 256 CUs; the kernels
  // grid-stride over the rest.
  constexpr int64_t kMaxBlocks = 256 * 16;
  if (aligned16(d) && aligned16(s) && total >= 8) {
    const int64_t n8 = total / 8;
    int64_t blocks = (n8 + tp::kThreads * tp::kUnroll - 1) / (tp::kThreads * tp::kUnroll);
    if (blocks > kMaxBlocks) blocks = kMaxBlocks;
    hipLaunchKernelGGL(tp::add_vec_kernel, dim3(static_cast<unsigned>(blocks)), dim3(tp::kThreads), 0, st,
                       reinterpret_cast<half8_t*>(d), reinterpret_cast<const half8_t*>(s), n8);
    const int rc = check_launch(fn);
    if (rc != FA_OK) return rc;
    done = n8 * 8;
  }
  const int64_t rest = total - done;
  if (rest > 0) {
    int64_t blocks = (rest + tp::kThreads - 1) / tp::kThreads;
    if (blocks > kMaxBlocks) blocks = kMaxBlocks;
    hipLaunchKernelGGL(tp::add_scalar_kernel, dim3(static_cast<unsigned>(blocks)), dim3(tp::kThreads), 0, st,
                       d + done, s + done, rest);
    return check_launch(fn);
  }
  return FA_OK;
}
