// KV-cache token eviction for gfx950.
//
// The reference (flash_attn_kernel.cu:4223-4344) bubble-sorts each batch
// row's attention scores ascending on one thread (swapping only when
// s[j] > s[j+1], i.e. a stable sort), evicts the `num_evict` lowest, and
// copies the kept K/V rows, in their original order, to the front of
// zero-filled outputs.  Here that is two launches:
//  1. rank_kernel: token i of row b is kept iff its stable ascending rank
//       #{j : s_j < s_i} + #{j < i : s_j == s_i}
//     is >= num_evict -- the position the stable sort gives it.  Scores of a
//     row sit in LDS; 16 lanes share each token's count.
//  2. compact_kernel: one workgroup per (batch, KV head, block of output rows)
//     turns the keep mask into the destination -> source row map (a
//     workgroup prefix count in LDS) and streams its output rows with 16-byte
//     loads and stores: kept rows copied, the tail zero-filled.  This is the
//     HBM-bound part: kept rows are read once, every output row written once.
// Scores containing NaN are outside the contract (the reference's bubble sort
// then depends on where the NaN sits; the rank order does not).
#include "capi_internal.h"
#include "common.h"

namespace fa {
namespace evict {

constexpr int kMaxN = 1024;  // the reference's limit (shared arrays of 1024)
constexpr int kThreads = 256;
constexpr int kRowsPerBlock = 128;  // output rows per compaction workgroup

// 16 lanes per token: lane g of token i's group counts j = g, g + 16, ...;
// the 16 partial ranks are summed with DPP moves inside the 16-lane row.
constexpr int kRankLanes = 16;
constexpr int kTokensPerBlock = kThreads / kRankLanes;
__global__ __launch_bounds__(kThreads) void rank_kernel(const float* __restrict__ scores, int32_t* __restrict__ keep,
                                                       int N, int num_evict) {
  __shared__ float s[kMaxN];
  const int b = blockIdx.y;
  const float* sb = scores + static_cast<size_t>(b) * N;
  for (int j = threadIdx.x; j < N; j += kThreads) s[j] = sb[j];
  __syncthreads();
  const int g = threadIdx.x % kRankLanes;
  const int i = blockIdx.x * kTokensPerBlock + threadIdx.x / kRankLanes;
  const int ii = min(i, N - 1);
  const float si = s[ii];
  int rank = 0;
  for (int j = g; j < N; j += kRankLanes) {
    const float sj = s[j];
    rank += (sj < si || (sj == si && j < ii)) ? 1 : 0;
  }
  rank = group_sum_i<kRankLanes>(rank);
  if (g == 0 && i < N) keep[static_cast<size_t>(b) * N + i] = rank >= num_evict ? 1 : 0;
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void compact_kernel(const half_t* __restrict__ k, const half_t* __restrict__ v,
                                                          const int32_t* __restrict__ keep, half_t* __restrict__ ko,
                                                          half_t* __restrict__ vo, int H, int N, int D) {
  __shared__ int src_of[kMaxN];  // output row -> source row (kept rows only)
  __shared__ int wave_total[kThreads / 64];
  const int bh = blockIdx.y;
  const int b = bh / H;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  // ---- prefix count of kept tokens: thread t owns tokens 4t .. 4t+3 ----
  const int32_t* kb = keep + static_cast<size_t>(b) * N;
  int flag[4];
  int cnt = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i = 4 * tid + q;
    flag[q] = (i < N && kb[i] != 0) ? 1 : 0;
    cnt += flag[q];
  }
  int incl = cnt;  // inclusive scan over the wave
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off, 64);
    if (lane >= off) incl += y;
  }
  if (lane == 63) wave_total[wave] = incl;
  __syncthreads();
  int before = 0, kept = 0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) {
    before += (w < wave) ? wave_total[w] : 0;
    kept += wave_total[w];
  }
  int dst = before + incl - cnt;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    if (flag[q]) src_of[dst++] = 4 * tid + q;
  __syncthreads();

  // ---- output rows [r0, r0 + kRowsPerBlock) of this (batch, head) ----
  const size_t base = static_cast<size_t>(bh) * N * D;
  const int r0 = blockIdx.x * kRowsPerBlock;
  const int rows = min(kRowsPerBlock, N - r0);
  if constexpr (VEC) {
    const int cpr = D / 8;  // 16-byte chunks per row
    const u32x4 zero = {0u, 0u, 0u, 0u};
    constexpr int U = 4;  // chunks in flight per thread: all loads, then all stores
    const int total = rows * cpr;
    for (int c0 = tid; c0 < total; c0 += U * kThreads) {
      u32x4 kx[U], vx[U];
      size_t dsto[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u * kThreads;
        const int w = r0 + c / cpr;
        const int col = (c % cpr) * 8;
        dsto[u] = base + static_cast<size_t>(w) * D + col;
        kx[u] = zero;
        vx[u] = zero;
        if (c < total && w < kept) {
          const size_t srco = base + static_cast<size_t>(src_of[w]) * D + col;
          kx[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(k + srco));
          vx[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(v + srco));
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (c0 + u * kThreads < total) {
          *reinterpret_cast<u32x4*>(ko + dsto[u]) = kx[u];
          *reinterpret_cast<u32x4*>(vo + dsto[u]) = vx[u];
        }
      }
    }
  } else {
    for (int e = tid; e < rows * D; e += kThreads) {
      const int w = r0 + e / D;
      const int col = e % D;
      const size_t dsto = base + static_cast<size_t>(w) * D + col;
      if (w < kept) {
        const size_t srco = base + static_cast<size_t>(src_of[w]) * D + col;
        ko[dsto] = k[srco];
        vo[dsto] = v[srco];
      } else {
        ko[dsto] = static_cast<half_t>(0.0f);
        vo[dsto] = static_cast<half_t>(0.0f);
      }
    }
  }
}

}  // namespace evict
}  // namespace fa

using namespace fa;
using namespace fa::evict;

extern "C" int fa_token_eviction(const void* k, const void* v, const float* attn_scores, void* k_out, void* v_out,
                                 int32_t* keep_mask, int B, int H_KV, int N, int D, int num_evict, void* stream) {
  const char* fn = "fa_token_eviction";
  if (B < 0 || H_KV <= 0 || N < 0 || D <= 0)
    return set_error(FA_ERR_INVALID_ARG, "%s: bad sizes (B=%d H_KV=%d N=%d D=%d)", fn, B, H_KV, N, D);
  if (N > kMaxN) return set_error(FA_ERR_UNSUPPORTED, "%s: N=%d exceeds %d", fn, N, kMaxN);
  if (static_cast<long long>(B) * H_KV > 65535) return set_error(FA_ERR_UNSUPPORTED, "%s: B*H_KV exceeds 65535", fn);
  if (B == 0 || N == 0) return FA_OK;
  if (!k || !v || !attn_scores || !k_out || !v_out || !keep_mask)
    return set_error(FA_ERR_INVALID_ARG, "%s: null pointer", fn);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(rank_kernel, dim3(ceil_div(N, kTokensPerBlock), B), dim3(kThreads), 0, st, attn_scores,
                     keep_mask, N, num_evict);
  const bool vec = D % 8 == 0 && aligned16(k) && aligned16(v) && aligned16(k_out) && aligned16(v_out);
  const dim3 grid(ceil_div(N, kRowsPerBlock), B * H_KV);
  const half_t* kh = static_cast<const half_t*>(k);
  const half_t* vh = static_cast<const half_t*>(v);
  if (vec)
    hipLaunchKernelGGL(compact_kernel<true>, grid, dim3(kThreads), 0, st, kh, vh, keep_mask,
                       static_cast<half_t*>(k_out), static_cast<half_t*>(v_out), H_KV, N, D);
  else
    hipLaunchKernelGGL(compact_kernel<false>, grid, dim3(kThreads), 0, st, kh, vh, keep_mask,
                       static_cast<half_t*>(k_out), static_cast<half_t*>(v_out), H_KV, N, D);
  return check_launch(fn);
}
