// KV-cache token eviction and speculative-decoding verification for gfx950.
//
// ---- token eviction ----
// The reference (flash_attn_kernel.cu:4223-4344) bubble-sorts each batch
// row's attention scores ascending on one thread (swapping only when
// s[j] > s[j+1], i.e. a stable sort), evicts the `num_evict` lowest, and
// copies the kept K/V rows, in their original order, to the front of
// zero-filled outputs.  Here that is one launch, one workgroup per (batch,
// KV head, block of output rows): each derives its batch row's keep mask --
// token i is kept iff its stable ascending rank
//     #{j : s_j < s_i} + #{j < i : s_j == s_i}
// is >= num_evict, the position the stable sort gives it -- from a radix
// select of the num_evict-th smallest score, turns it into the destination ->
// source row map (a workgroup prefix count in LDS) and streams its output
// rows with 16-byte loads and stores: kept rows copied, the tail zero-filled.
// This is the HBM-bound part: kept rows are read once, every output row
// written once.
// Scores containing NaN are outside the contract (the reference's bubble sort
// then depends on where the NaN sits; the rank order does not).
#include "capi_internal.h"
#include "common.h"

namespace fa {
namespace evict {

constexpr int kMaxN = 1024;  // the reference's limit (shared arrays of 1024)
constexpr int kThreads = 256;
constexpr int kRowsPerBlock = 128;  // output rows per compaction workgroup

// Block-wide exclusive prefix count of one flag per token (thread t owns
// tokens 4t .. 4t+3, in flag[0..3]); returns the count before thread t's first
// token and sets `total`.  `scratch` holds kThreads / 64 ints.
__device__ __forceinline__ int block_prefix(const int (&flag)[4], int* scratch, int& total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int cnt = flag[0] + flag[1] + flag[2] + flag[3];
  int incl = cnt;  // inclusive scan over the wave
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off, 64);
    if (lane >= off) incl += y;
  }
  __syncthreads();  // scratch may still be read by a previous call
  if (lane == 63) scratch[wave] = incl;
  __syncthreads();
  int before = 0;
  total = 0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) {
    before += (w < wave) ? scratch[w] : 0;
    total += scratch[w];
  }
  return before + incl - cnt;
}

// Order-preserving unsigned key of a (non-NaN) score: -0.0 and +0.0 compare
// equal as floats and so map to one key.
__device__ __forceinline__ uint32_t score_key(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x == 0.0f ? 0.0f : x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// One workgroup per (batch, KV head, block of output rows).  Every workgroup
// of batch row b derives row b's keep mask itself (1024 scores at most):
// a radix select (four 8-bit passes over LDS histograms) finds the key T of
// the num_evict-th smallest score and the count c of smaller ones; a token is
// evicted iff its key is below T, or equals T and fewer than num_evict - c
// equal keys precede it -- exactly the tokens whose stable ascending rank
// #{j : s_j < s_i} + #{j < i : s_j == s_i} is below num_evict, i.e. the first
// num_evict of the reference's stable sort.  A prefix count of the keep mask
// then gives the output -> source row map, and the workgroup streams its
// output rows: kept rows copied, the tail zero-filled.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void evict_kernel(const half_t* __restrict__ k, const half_t* __restrict__ v,
                                                        const float* __restrict__ scores, int32_t* __restrict__ keep,
                                                        half_t* __restrict__ ko, half_t* __restrict__ vo, int H,
                                                        int N, int D, int num_evict) {
  static_assert(kThreads == 256 && 4 * kThreads == kMaxN, "one histogram bin and four tokens per thread");
  __shared__ int src_of[kMaxN];  // output row -> source row (kept rows only)
  __shared__ int hist[256];
  __shared__ int scratch[kThreads / 64];
  __shared__ int pick[2];
  const int bh = blockIdx.y;
  const int b = bh / H;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  // ---- keys of this thread's tokens 4t .. 4t+3 ----
  const float* sb = scores + static_cast<size_t>(b) * N;
  uint32_t key[4];
  bool valid[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i = 4 * tid + q;
    valid[q] = i < N;
    key[q] = valid[q] ? score_key(sb[i]) : 0u;
  }
  const int E = num_evict;
  int keepf[4];
  if (E <= 0 || E >= N) {
#pragma unroll
    for (int q = 0; q < 4; ++q) keepf[q] = (valid[q] && E <= 0) ? 1 : 0;
  } else {
    // ---- radix select of the E-th smallest key (1-based) ----
    uint32_t prefix = 0u, himask = 0u;
    int need = E, below = 0;
#pragma unroll 1
    for (int shift = 24; shift >= 0; shift -= 8) {
      hist[tid] = 0;  // kThreads == 256 bins
      __syncthreads();
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (valid[q] && (key[q] & himask) == prefix) atomicAdd(&hist[(key[q] >> shift) & 255u], 1);
      __syncthreads();
      if (wave == 0) {
        int c[4], sum = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          c[j] = hist[4 * lane + j];
          sum += c[j];
        }
        int incl = sum;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const int y = __shfl_up(incl, off, 64);
          if (lane >= off) incl += y;
        }
        int run = incl - sum;  // keys in the bins before this lane's first bin
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // the bin where the running count first reaches `need` (one lane, one j)
          if (run < need && run + c[j] >= need) {
            pick[0] = 4 * lane + j;
            pick[1] = run;
          }
          run += c[j];
        }
      }
      __syncthreads();
      const int digit = pick[0];
      need -= pick[1];
      below += pick[1];
      prefix |= static_cast<uint32_t>(digit) << shift;
      himask |= 0xFFu << shift;
      __syncthreads();  // every thread has read pick before the next pass
    }
    // prefix = T; below = #{key < T}; the first E - below keys equal to T are evicted
    int eq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) eq[q] = (valid[q] && key[q] == prefix) ? 1 : 0;
    int eq_total;
    int eq_before = block_prefix(eq, scratch, eq_total);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      keepf[q] = valid[q] && (key[q] > prefix || (eq[q] && eq_before >= E - below)) ? 1 : 0;
      eq_before += eq[q];
    }
  }
  // the mask output: written once per batch row
  if (bh % H == 0 && blockIdx.x == 0) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (valid[q]) keep[static_cast<size_t>(b) * N + 4 * tid + q] = keepf[q];
  }

  // ---- prefix count of kept tokens -> output row map ----
  int kept;
  int dst = block_prefix(keepf, scratch, kept);
#pragma unroll
  for (int q = 0; q < 4; ++q)
    if (keepf[q]) src_of[dst++] = 4 * tid + q;
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

// ---- speculative verification ----
// The reference (flash_attn_kernel.cu:3853-4018) accepts draft token t at
// step i when r_i < min(1, p_t / (q_t + 1e-10)); at the first rejection it
// samples from max(target - draft, 0) / Z and draws a bonus token from the
// next target row, each by a running fp32 sum over the vocabulary compared
// against r (with its "tok == 0" update rule: a hit at index 0 is replaced by
// the next hit).  The sampled indices depend on the exact fp32 value of every
// partial sum, so each sum is accumulated serially in index order, as there.
// One workgroup of two waves per batch row: wave 0 computes Z and then the
// residual sample, wave 1 the bonus token, concurrently.  Within a wave the 64
// lanes load kChunk consecutive elements and compute their terms (differences,
// the division by Z) in parallel into LDS, with the next chunk already
// loading -- for Z and the residual only the terms that change the sum,
// compacted in index order with their indices (config 9: 327 -> 240 us);
// lane 0 then runs only the dependent adds, 64 terms per batch read
// from LDS, and tests the running sum once per batch: sums only grow, so the
// first hit lies in the batch where the test first passes, and lane 0 replays
// that batch's adds one by one (the same adds in the same order, so the same
// sums) to find it.  The sample and bonus scans stop at their first decisive
// hit.
namespace spec {

constexpr int kMaxK = 8;     // SPEC_MAX_K (flash_attn_kernel.cu:3851)
constexpr int kChunk = 2048;  // elements per wave step (32 per lane)
constexpr int kPerLane = kChunk / 64;

enum ChainMode { kZ = 0, kResidual = 1, kPrefix = 2, kBonus = 3 };

// Serial scan of row a (minus row b for kZ / kResidual) over [0, V).
//  kZ:        *sum = the sum of the positive (a - b) in index order.
//  kResidual: cs += (a - b) / Z where a - b > 0; hit at such v when r < cs.
//  kPrefix:   cs += a; hit when r < cs.
//  kBonus:    cs += a; hit when cs >= r.
// Returns the reference's token: the first hit, or the next hit if the first
// is index 0 (0 without hits).  A term that does not contribute (a - b <= 0
// for kZ / kResidual, or past V) is -0.0, which leaves a non-negative running
// sum unchanged; a contributing term has its sign bit clear (+0.0 if the
// division underflows), so the replay reads "contributed" off the sign.  For
// kResidual the first v with r < cs always contributed (cs only grows where
// a term is added); a later hit must contribute too.
//
// kZ and kResidual stage only the contributing terms, compacted in index
// order with their indices: a non-contributing term is -0.0 and adding it to
// the non-negative running sum changes nothing, so lane 0 runs the same adds
// in the same order over the contributing terms alone (about half of them for
// unrelated target and draft rows).
template <int MODE>
__device__ int chain(const float* __restrict__ a, const float* __restrict__ b, int V, float Z, float r, float* sum,
                     float* lds, int* lds_idx) {
  constexpr bool kCompact = MODE == kZ || MODE == kResidual;
  const int lane = threadIdx.x & 63;
  float cs = 0.0f;        // lane 0's running sum
  int tok = 0;            // lane 0: the token found so far
  bool zero_hit = false;  // lane 0: a hit at index 0 was seen, the next hit decides
  // lane l holds elements c0 + 256 q + 4 l + e (q < kPerLane / 4, e < 4): 16-byte loads
  // 16-byte loads where the row allows them (V % 4 == 0 and 16-byte aligned
  // rows), element loads otherwise
  const bool vec = (V & 3) == 0 && (reinterpret_cast<uintptr_t>(a) & 15) == 0 &&
                   (MODE == kPrefix || MODE == kBonus || (reinterpret_cast<uintptr_t>(b) & 15) == 0);
  auto load = [&](int c0, float4_t (&x)[kPerLane / 4], float4_t (&y)[kPerLane / 4]) {
#pragma unroll
    for (int q = 0; q < kPerLane / 4; ++q) {
      const int v0 = c0 + 256 * q + 4 * lane;
      if (vec) {
        const bool in = v0 < V;
        x[q] = in ? *reinterpret_cast<const float4_t*>(a + v0) : float4_t{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (MODE == kZ || MODE == kResidual)
          y[q] = in ? *reinterpret_cast<const float4_t*>(b + v0) : float4_t{0.0f, 0.0f, 0.0f, 0.0f};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[q][e] = v0 + e < V ? a[v0 + e] : 0.0f;
          if constexpr (MODE == kZ || MODE == kResidual) y[q][e] = v0 + e < V ? b[v0 + e] : 0.0f;
        }
      }
    }
  };
  // xa / ya hold the current chunk: loaded during the previous chunk's
  // serial adds, consumed by this chunk's term computation, then reloaded
  // with the next chunk just before this chunk's adds (so no wait for
  // memory ever falls between a chunk's terms and its adds)
  float4_t xa[kPerLane / 4], ya[kPerLane / 4];
  load(0, xa, ya);
  for (int c0 = 0; c0 < V; c0 += kChunk) {
    int staged = min(kChunk, V - c0);  // terms lane 0 walks in this chunk
    if constexpr (kCompact) {
      int base = 0;
#pragma unroll
      for (int q = 0; q < kPerLane / 4; ++q) {
        float t[4];
        bool f[4];
        uint64_t bal[4];
        int below = 0, total = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float d = xa[q][e] - ya[q][e];
          f[e] = d > 0.0f && c0 + 256 * q + 4 * lane + e < V;
          t[e] = MODE == kZ ? d : d / Z;
          bal[e] = __builtin_amdgcn_ballot_w64(f[e]);
          below += __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal[e] >> 32),
                                             __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal[e]), 0u));
          total += __builtin_popcountll(bal[e]);
        }
        // element order c0 + 256 q + 4 lane + e: lanes below first, then e
        int pos = base + below;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (f[e]) {
            lds[pos] = t[e];
            lds_idx[pos] = c0 + 256 * q + 4 * lane + e;
            ++pos;
          }
        base += total;
      }
      lds[base + lane] = -0.0f;  // pad the last batch of 64: no change, never a hit
      staged = base;
    } else {
#pragma unroll
      for (int q = 0; q < kPerLane / 4; ++q) {
        float4_t t4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float t = xa[q][e];
          if (c0 + 256 * q + 4 * lane + e >= V) t = -0.0f;  // past V: no change, never a hit
          t4[e] = t;
        }
        *reinterpret_cast<float4_t*>(lds + 256 * q + 4 * lane) = t4;
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave's LDS writes are done
    if (c0 + kChunk < V) load(c0 + kChunk, xa, ya);
    bool done = false;
    if (lane == 0) {
      const int n = staged;
      for (int h = 0; h < n; h += 64) {
        float4_t q[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) q[j] = *reinterpret_cast<const float4_t*>(lds + h + 4 * j);
        const float cs0 = cs;
#pragma unroll
        for (int j = 0; j < 16; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) cs += q[j][e];
        if constexpr (MODE != kZ) {
          const bool crossed = (MODE == kBonus) ? (cs >= r) : (r < cs);
          if (crossed || zero_hit) {
            // replay the batch: the first hit, or the next one after a hit at 0
            float x = cs0;
            for (int k = 0; k < 64 && !done; ++k) {
              if (h + k >= n) break;
              const float t = lds[h + k];  // the batch's terms are still staged there
              x += t;
              const bool contrib = MODE != kResidual || !__builtin_signbit(t);
              const bool hit = (MODE == kBonus) ? (x >= r) : (r < x) && contrib;
              if (!hit) continue;
              const int v = kCompact ? lds_idx[h + k] : c0 + h + k;
              if (v == 0 && !zero_hit) {
                zero_hit = true;
              } else {
                tok = v;
                done = true;
              }
            }
            if (done) break;
          }
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lane 0's LDS reads are done before the next chunk's writes
    if (__builtin_amdgcn_readfirstlane(static_cast<int>(done))) break;
  }
  if (sum) *sum = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, cs)));
  return __builtin_amdgcn_readfirstlane(tok);
}

__global__ __launch_bounds__(128) void verify_kernel(const float* __restrict__ target, const float* __restrict__ draft,
                                                     const int64_t* __restrict__ draft_tokens,
                                                     const float* __restrict__ rand, int32_t* __restrict__ accepted,
                                                     int64_t* __restrict__ out, int K, int V) {
  // per-wave term staging, plus one batch of padding past the last staged term
  __shared__ __attribute__((aligned(16))) float lds[2][kChunk + 64];
  __shared__ int lds_idx[2][kChunk];                                  // their indices (compacted chains)
  const int b = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const float* tb = target + static_cast<size_t>(b) * (K + 1) * V;
  const float* db = draft + static_cast<size_t>(b) * K * V;
  const int64_t* tok_b = draft_tokens + static_cast<size_t>(b) * K;
  const float* rb = rand + static_cast<size_t>(b) * K;
  int64_t* ob = out + static_cast<size_t>(b) * (K + 1);

  // acceptance steps (wave-uniform: every lane reads the same values)
  int acc = 0;
  int rej = -1;
  for (int i = 0; i < K; ++i) {
    const int64_t t = tok_b[i];
    const bool in_range = t >= 0 && t < V;
    const float p = in_range ? tb[static_cast<size_t>(i) * V + t] : 0.0f;
    const float q = in_range ? db[static_cast<size_t>(i) * V + t] : 0.0f;
    const float accept_prob = fminf(1.0f, p / (q + 1e-10f));
    if (rb[i] < accept_prob) {
      ++acc;
    } else {
      rej = i;
      break;
    }
  }
  if (wave == 0) {
    if (lane == 0) {
      // every position is written: accepted tokens, then (after a rejection at
      // rej) the sample at rej, the bonus at rej + 1 (wave 1) and -1 beyond
      for (int i = 0; i < acc; ++i) ob[i] = tok_b[i];
      if (rej >= 0)
        for (int j = rej + 2; j <= K; ++j) ob[j] = -1;
      accepted[b] = acc;
    }
    if (rej >= 0) {
      const float* ti = tb + static_cast<size_t>(rej) * V;
      const float* di = db + static_cast<size_t>(rej) * V;
      float Z;
      chain<kZ>(ti, di, V, 0.0f, 0.0f, &Z, lds[0], lds_idx[0]);
      const int s = Z > 0.0f ? chain<kResidual>(ti, di, V, Z, rb[rej], nullptr, lds[0], lds_idx[0])
                             : chain<kPrefix>(ti, nullptr, V, 0.0f, rb[rej], nullptr, lds[0], lds_idx[0]);
      if (lane == 0) ob[rej] = s;
    }
  } else {
    const int row = rej >= 0 ? rej + 1 : K;
    const float r = rb[rej >= 0 ? min(rej, K - 1) : K - 1];
    const int bonus = chain<kBonus>(tb + static_cast<size_t>(row) * V, nullptr, V, 0.0f, r, nullptr, lds[1], lds_idx[1]);
    if (lane == 0) ob[row] = bonus;
  }
}

}  // namespace spec
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
  const bool vec = D % 8 == 0 && aligned16(k) && aligned16(v) && aligned16(k_out) && aligned16(v_out);
  const dim3 grid(ceil_div(N, kRowsPerBlock), B * H_KV);
  const half_t* kh = static_cast<const half_t*>(k);
  const half_t* vh = static_cast<const half_t*>(v);
  if (vec)
    hipLaunchKernelGGL(evict_kernel<true>, grid, dim3(kThreads), 0, st, kh, vh, attn_scores, keep_mask,
                       static_cast<half_t*>(k_out), static_cast<half_t*>(v_out), H_KV, N, D, num_evict);
  else
    hipLaunchKernelGGL(evict_kernel<false>, grid, dim3(kThreads), 0, st, kh, vh, attn_scores, keep_mask,
                       static_cast<half_t*>(k_out), static_cast<half_t*>(v_out), H_KV, N, D, num_evict);
  return check_launch(fn);
}

extern "C" int fa_speculative_verify(const float* target_probs, const float* draft_probs, const int64_t* draft_tokens,
                                     const float* random_vals, int32_t* accepted_count, int64_t* output_tokens, int B,
                                     int K, int vocab_size, void* stream) {
  const char* fn = "fa_speculative_verify";
  if (B < 0 || vocab_size <= 0)
    return set_error(FA_ERR_INVALID_ARG, "%s: bad sizes (B=%d vocab=%d)", fn, B, vocab_size);
  if (K < 1 || K > spec::kMaxK) return set_error(FA_ERR_INVALID_ARG, "%s: K=%d outside [1, %d]", fn, K, spec::kMaxK);
  if (B == 0) return FA_OK;
  if (!target_probs || !draft_probs || !draft_tokens || !random_vals || !accepted_count || !output_tokens)
    return set_error(FA_ERR_INVALID_ARG, "%s: null pointer", fn);
  hipLaunchKernelGGL(spec::verify_kernel, dim3(B), dim3(128), 0, static_cast<hipStream_t>(stream), target_probs,
                     draft_probs, draft_tokens, random_vals, accepted_count, output_tokens, K, vocab_size);
  return check_launch(fn);
}
