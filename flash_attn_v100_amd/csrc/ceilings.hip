// Measurement probes for the two rooflines the attention kernels are priced
// against (not part of the attention library; built into libfa_ceilings.so and
// called only by bench.py --ceilings):
//
//   fa_ceiling_stream_read   every byte of a buffer read once with 16-byte
//                            nontemporal loads by a full grid: the HBM read rate
//                            a streaming kernel can reach on this part.
//   fa_ceiling_mfma_chain    v_mfma_f32_32x32x16_f16 back to back from every
//                            SIMD, no memory traffic in the loop: the fp16 MFMA
//                            rate the part sustains for the operand data given
//                            (random N(0,1) fp16 toggles more bits, draws more
//                            power and runs at a lower clock than constant data).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;

// Each workgroup reads a contiguous slice of `words` 16-byte words; the XOR of
// everything read is stored per thread so the loads cannot be removed.
__global__ __launch_bounds__(kThreads) void stream_read_kernel(const u32x4* __restrict__ src, size_t words,
                                                               u32x4* __restrict__ sink) {
  const size_t per_block = (words + gridDim.x - 1) / gridDim.x;
  const size_t begin = static_cast<size_t>(blockIdx.x) * per_block;
  const size_t end = begin + per_block < words ? begin + per_block : words;
  u32x4 acc = {0u, 0u, 0u, 0u};
  size_t i = begin + threadIdx.x;
  // four independent loads in flight per thread per iteration
  for (; i + 3 * kThreads < end; i += 4 * kThreads) {
    const u32x4 a = __builtin_nontemporal_load(src + i);
    const u32x4 b = __builtin_nontemporal_load(src + i + kThreads);
    const u32x4 c = __builtin_nontemporal_load(src + i + 2 * kThreads);
    const u32x4 d = __builtin_nontemporal_load(src + i + 3 * kThreads);
    acc ^= a ^ b ^ c ^ d;
  }
  for (; i < end; i += kThreads) acc ^= __builtin_nontemporal_load(src + i);
  sink[static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x] = acc;
}

// Every wave loads 8 A and 8 B operand fragments (its own slice of `ops`) and
// then issues `iters` rounds of 8 MFMAs over 4 independent accumulators,
// cycling through the fragments so that every MFMA sees different data.
__global__ __launch_bounds__(kThreads) void mfma_chain_kernel(const half8* __restrict__ ops, int iters,
                                                              float* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  const size_t wave = static_cast<size_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
  const half8* w = ops + wave * 16 * 64;
  half8 a[8], b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = w[i * 64 + lane];
    b[i] = w[(8 + i) * 64 + lane];
  }
  float16v acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
  // iters is a multiple of 8: the rotation r of the B fragments is unrolled so
  // every fragment index is a compile-time constant (registers, not scratch)
  for (int it = 0; it < iters; it += 8) {
#pragma unroll
    for (int r = 0; r < 8; ++r)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        acc[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[(i + r) & 7], acc[i & 3], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[j][r];
  sink[wave * 64 + lane] = s;
}

}  // namespace

// Reads `bytes` (a multiple of 16) from `src` with `blocks` workgroups of 256
// threads; `sink` holds blocks * 256 * 16 bytes.  Returns a hipError_t.
extern "C" int fa_ceiling_stream_read(const void* src, size_t bytes, void* sink, int blocks, void* stream) {
  hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(src), bytes / 16, static_cast<u32x4*>(sink));
  return static_cast<int>(hipGetLastError());
}

// `ops` holds blocks * 4 waves * 16 fragments * 64 lanes * 8 fp16 values;
// `sink` blocks * 256 floats; iters a positive multiple of 8.  FLOPs per call:
// blocks * 4 * iters * 8 * 32768.
extern "C" int fa_ceiling_mfma_chain(const void* ops, int iters, void* sink, int blocks, void* stream) {
  if (iters <= 0 || iters % 8 != 0) return static_cast<int>(hipErrorInvalidValue);
  hipLaunchKernelGGL(mfma_chain_kernel, dim3(blocks), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const half8*>(ops), iters, static_cast<float*>(sink));
  return static_cast<int>(hipGetLastError());
}
