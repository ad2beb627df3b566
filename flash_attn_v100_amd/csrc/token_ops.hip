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
// Output rows per compaction workgroup: the largest of 128, 256 and 512
// that still gives every CU a workgroup (evict_rows_per_block).  Each
// workgroup runs the selection once for its rows, so fewer, longer
// workgroups spend less of the call selecting (config 8, B = 16, 8 heads,
// N = 1024: 128 rows 28.6 us, 256 rows 26.9, 512 rows 26.0, 1024 rows 32).
constexpr int kMinRowsPerBlock = 128;
constexpr int kMaxRowsPerBlock = 512;
constexpr long long kFillWorkgroups = 256;

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
                                                        int N, int D, int num_evict, int rows_per_block) {
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

  // ---- output rows [r0, r0 + rows_per_block) of this (batch, head) ----
  const size_t base = static_cast<size_t>(bh) * N * D;
  const int r0 = blockIdx.x * rows_per_block;
  const int rows = min(rows_per_block, N - r0);
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
// Two workgroups of two waves per batch row: one computes Z and then the
// residual sample, the other the bonus token, concurrently.  In each, wave 1
// loads kChunk consecutive elements and stages their terms (differences, the
// division by Z) into LDS -- for Z and the residual only the terms that change
// the sum, compacted in index order with their indices -- while lane 0 of
// wave 0 runs only the dependent adds of the previous chunk, 64 terms per
// batch, and tests the running sum once per batch: sums only grow, so the
// first hit lies in the batch where the test first passes, and lane 0 replays
// that batch's adds one by one (the same adds in the same order, so the same
// sums) to find it.  The sample and bonus scans stop at their first decisive
// hit.  (Config 9: 327 us with one workgroup per row staging and adding in
// turn, 240 with the compaction, 130 with staging and adds on separate waves.)
namespace spec {

constexpr int kMaxK = 8;     // SPEC_MAX_K (flash_attn_kernel.cu:3851)
constexpr int kChunk = 2048;  // elements per staged chunk (32 per lane)
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
// Two waves: wave 1 stages the terms of chunk c + 1 into one LDS buffer
// while lane 0 of wave 0 adds chunk c from the other; one workgroup barrier
// per chunk hands the buffers over.  kZ and kResidual stage only the
// contributing terms, compacted in index order with their indices: adding a
// non-contributing -0.0 to the non-negative running sum changes nothing, so
// lane 0 runs the same adds in the same order over about half the terms for
// unrelated target and draft rows.  Every wave runs the same number of
// barriers: the loop is bounded by the chunk count and its early exit is read
// from LDS after a barrier.
struct Stage {
  float t[2][kChunk + 64];  // terms (+ one batch of -0.0 padding)
  int idx[2][kChunk];       // their indices (compacted modes)
  int n[2];                 // terms staged
  int done, tok;
  float sum;
};

template <int MODE>
__device__ int chain(const float* __restrict__ a, const float* __restrict__ b, int V, float Z, float r, float* sum,
                     Stage& st) {
  constexpr bool kCompact = MODE == kZ || MODE == kResidual;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nchunks = (V + kChunk - 1) / kChunk;
  // lane l holds elements c0 + 256 q + 4 l + e (q < kPerLane / 4, e < 4):
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
  // wave 1: stage chunk c into buffer c & 1
  auto stage = [&](int c) {
    const int c0 = c * kChunk;
    const int buf = c & 1;
    float4_t x[kPerLane / 4], y[kPerLane / 4];
    load(c0, x, y);
    float* t_out = st.t[buf];
    if constexpr (kCompact) {
      int base = 0;
#pragma unroll
      for (int q = 0; q < kPerLane / 4; ++q) {
        float t[4];
        bool f[4];
        int below = 0, total = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float d = x[q][e] - y[q][e];
          f[e] = d > 0.0f && c0 + 256 * q + 4 * lane + e < V;
          t[e] = MODE == kZ ? d : d / Z;
          const uint64_t bal = __builtin_amdgcn_ballot_w64(f[e]);
          below += __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal >> 32),
                                             __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0u));
          total += __builtin_popcountll(bal);
        }
        // element order c0 + 256 q + 4 lane + e: lanes below first, then e
        int pos = base + below;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (f[e]) {
            t_out[pos] = t[e];
            st.idx[buf][pos] = c0 + 256 * q + 4 * lane + e;
            ++pos;
          }
        base += total;
      }
      t_out[base + lane] = -0.0f;  // pad the last batch of 64: no change, never a hit
      if (lane == 0) st.n[buf] = base;
    } else {
#pragma unroll
      for (int q = 0; q < kPerLane / 4; ++q) {
        float4_t t4;
#pragma unroll
        for (int e = 0; e < 4; ++e) t4[e] = c0 + 256 * q + 4 * lane + e < V ? x[q][e] : -0.0f;  // past V: never a hit
        *reinterpret_cast<float4_t*>(t_out + 256 * q + 4 * lane) = t4;
      }
      if (lane == 0) st.n[buf] = min(kChunk, V - c0);
    }
  };

  if (threadIdx.x == 0) st.done = 0;
  if (wave == 1) stage(0);
  __syncthreads();
  float cs = 0.0f;        // lane 0 of wave 0: the running sum
  int tok = 0;            // lane 0 of wave 0: the token found so far
  bool zero_hit = false;  // lane 0 of wave 0: a hit at index 0 was seen, the next hit decides
  for (int c = 0; c < nchunks; ++c) {
    const int buf = c & 1;
    if (wave == 1) {
      if (c + 1 < nchunks) stage(c + 1);
    } else if (lane == 0) {
      const float* tb = st.t[buf];
      const int n = st.n[buf];
      bool done = false;
      for (int h = 0; h < n && !done; h += 64) {
        float4_t q[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) q[j] = *reinterpret_cast<const float4_t*>(tb + h + 4 * j);
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
              const float t = tb[h + k];
              x += t;
              const bool contrib = MODE != kResidual || !__builtin_signbit(t);
              const bool hit = (MODE == kBonus) ? (x >= r) : (r < x) && contrib;
              if (!hit) continue;
              const int v = kCompact ? st.idx[buf][h + k] : c * kChunk + h + k;
              if (v == 0 && !zero_hit) {
                zero_hit = true;
              } else {
                tok = v;
                done = true;
              }
            }
          }
        }
      }
      if (done) st.done = 1;
    }
    __syncthreads();  // chunk c consumed, chunk c + 1 staged
    if (st.done) break;
  }
  if (threadIdx.x == 0) {
    st.tok = tok;
    st.sum = cs;
  }
  __syncthreads();
  const int result = st.tok;
  if (sum) *sum = st.sum;
  __syncthreads();  // every thread has read tok / sum before the next chain resets them
  return result;
}

// Grid (B, 2): workgroup (b, 0) settles the acceptance steps of row b and,
// after a rejection, samples the residual (Z, then the residual scan);
// workgroup (b, 1) draws the bonus token.  Both run the (cheap) acceptance
// steps themselves.
__global__ __launch_bounds__(128) void verify_kernel(const float* __restrict__ target, const float* __restrict__ draft,
                                                     const int64_t* __restrict__ draft_tokens,
                                                     const float* __restrict__ rand, int32_t* __restrict__ accepted,
                                                     int64_t* __restrict__ out, int K, int V) {
  __shared__ __attribute__((aligned(16))) Stage st;
  const int b = blockIdx.x;
  const int role = blockIdx.y;
  const float* tb = target + static_cast<size_t>(b) * (K + 1) * V;
  const float* db = draft + static_cast<size_t>(b) * K * V;
  const int64_t* tok_b = draft_tokens + static_cast<size_t>(b) * K;
  const float* rb = rand + static_cast<size_t>(b) * K;
  int64_t* ob = out + static_cast<size_t>(b) * (K + 1);

  // acceptance steps (uniform: every thread reads the same values)
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
  if (role == 0) {
    if (threadIdx.x == 0) {
      // every position is written: accepted tokens, then (after a rejection at
      // rej) the sample at rej, the bonus at rej + 1 (workgroup (b, 1)) and -1 beyond
      for (int i = 0; i < acc; ++i) ob[i] = tok_b[i];
      if (rej >= 0)
        for (int j = rej + 2; j <= K; ++j) ob[j] = -1;
      accepted[b] = acc;
    }
    if (rej >= 0) {
      const float* ti = tb + static_cast<size_t>(rej) * V;
      const float* di = db + static_cast<size_t>(rej) * V;
      float Z;
      chain<kZ>(ti, di, V, 0.0f, 0.0f, &Z, st);
      const int s = Z > 0.0f ? chain<kResidual>(ti, di, V, Z, rb[rej], nullptr, st)
                             : chain<kPrefix>(ti, nullptr, V, 0.0f, rb[rej], nullptr, st);
      if (threadIdx.x == 0) ob[rej] = s;
    }
  } else {
    const int row = rej >= 0 ? rej + 1 : K;
    const float r = rb[rej >= 0 ? min(rej, K - 1) : K - 1];
    const int bonus = chain<kBonus>(tb + static_cast<size_t>(row) * V, nullptr, V, 0.0f, r, nullptr, st);
    if (threadIdx.x == 0) ob[row] = bonus;
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
  int rpb = kMaxRowsPerBlock;
  while (rpb > kMinRowsPerBlock && static_cast<long long>(B) * H_KV * ceil_div(N, rpb) < kFillWorkgroups) rpb /= 2;
  const dim3 grid(ceil_div(N, rpb), B * H_KV);
  const half_t* kh = static_cast<const half_t*>(k);
  const half_t* vh = static_cast<const half_t*>(v);
  if (vec)
    hipLaunchKernelGGL(evict_kernel<true>, grid, dim3(kThreads), 0, st, kh, vh, attn_scores, keep_mask,
                       static_cast<half_t*>(k_out), static_cast<half_t*>(v_out), H_KV, N, D, num_evict, rpb);
  else
    hipLaunchKernelGGL(evict_kernel<false>, grid, dim3(kThreads), 0, st, kh, vh, attn_scores, keep_mask,
                       static_cast<half_t*>(k_out), static_cast<half_t*>(v_out), H_KV, N, D, num_evict, rpb);
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
  hipLaunchKernelGGL(spec::verify_kernel, dim3(B, 2), dim3(128), 0, static_cast<hipStream_t>(stream), target_probs,
                     draft_probs, draft_tokens, random_vals, accepted_count, output_tokens, K, vocab_size);
  return check_launch(fn);
}
