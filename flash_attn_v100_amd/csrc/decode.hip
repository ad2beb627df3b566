// Split-KV ("flash-decoding") single-token attention for gfx950.
//
// One kernel family serves every decode entry point (contiguous MHA/GQA and
// sliding-window decode, continuous batching, paged decode, INT8 decode, INT8
// KV cache):
//
//   grid  = B * H_KV * head_groups * splits workgroups of 256 threads (4 waves)
//   block = one KV head's key range [split*chunk, min(len_b, (split+1)*chunk))
//           for GB query heads of that KV head's group, so each K/V byte is read
//           from HBM once per group instead of once per query head.
//
// Each wave walks 32-key tiles (16 at D = 256).  QK^T runs on MFMA
// (v_mfma_f32_16x16x32_f16, or the int8 MFMA for INT8 decode) with the query
// heads as the 16 M rows and 16 keys as N; K comes straight from HBM in the
// B-operand layout, or (continuous batching, paged, contiguous and INT8
// decode launches of 512+ workgroups) through a per-wave LDS buffer filled by
// row-coalesced HBM->LDS copies.  P V runs on the VALU in a
// row layout: a key row of D fp16 over LPR = DP/8 lanes, 16 contiguous bytes
// each (every dwordx4 load reads 64/LPR whole rows), two keys per
// v_dot2_f32_f16.  Every lane of a wave shares the online-softmax max, so the
// waves' (m, l, O) merge once, at the end of the split, through LDS.  A
// sequence covered by one split writes the fp16 output directly; otherwise
// each split writes a (log2-sum-exp, normalised output) partial, takes an
// arrival rank on its unit's counter, and the last split to arrive merges the
// partials -- one kernel per call, no separate combine launch.  The last split
// also resets the counter, so a zero-filled workspace stays zero-filled
// between calls (and across graph replays) without any memset.
#include <math.h>

#include <algorithm>
#include <mutex>

#include "capi_internal.h"
#include "common.h"

namespace fa {

enum DecodeMode : int { kModeDecode = 0, kModeCB = 1, kModePaged = 2, kModeInt8 = 3, kModeInt8KV = 4 };

constexpr int kDecWaves = 4;
constexpr int kDecThreads = kDecWaves * 64;
constexpr int kPage = 16;             // PAGE_BLOCK_SIZE of the paged cache
// Split sizing.  The FA_DEC_* macros exist only to let a tuning sweep build
// variants; the defaults are the shipped configuration.
#ifndef FA_DEC_TARGET_BLOCKS
#define FA_DEC_TARGET_BLOCKS 4096
#endif
#ifndef FA_DEC_CHUNK_QUANTUM
#define FA_DEC_CHUNK_QUANTUM 256
#endif
constexpr unsigned kCounterSlotsDev = 65536;  // arrival counters in the workspace
constexpr int kMaxChunk = 8192;                        // keys per split, upper bound
constexpr int kChunkQuantum = FA_DEC_CHUNK_QUANTUM;    // split boundaries are multiples of this
constexpr int kTargetBlocks = FA_DEC_TARGET_BLOCKS;    // aim for this many split workgroups
// The paged kernel stages each split's page ids in LDS before its first load,
// one extra memory round trip per split, so it prefers fewer, longer splits.
#ifndef FA_DEC_PAGED_DIV
#define FA_DEC_PAGED_DIV 4
#endif
constexpr int kTargetBlocksPaged = FA_DEC_TARGET_BLOCKS / FA_DEC_PAGED_DIV;
// Every sequence of a fixed-length call (contiguous / INT8 / sliding-window
// decode) has the same key count, so its splits are all full: about 2.5
// workgroups per CU balance the per-split merge cost against HBM parallelism.
#ifndef FA_DEC_TARGET_BLOCKS_FIXED
#define FA_DEC_TARGET_BLOCKS_FIXED 640
#endif
constexpr int kTargetBlocksFixed = FA_DEC_TARGET_BLOCKS_FIXED;
#ifndef FA_DEC_FIXED_QUANTUM
#define FA_DEC_FIXED_QUANTUM 256
#endif
constexpr int kFixedQuantum = FA_DEC_FIXED_QUANTUM;  // fixed-length split boundaries (kSmallGridQuantum below)
// The INT8 KV cache reads half the bytes per key and dequantizes them with a
// few packed fp16 ops, so its splits are cheaper than the fp16 modes': finer
// ones (128-key quantum, about three workgroups per CU) balance better there
// (6a 18.8 -> 18.2 us; the same plan made 5b and 6b slower, 29.0 -> 29.6-30.1
// and 26.5 -> 27.1 us).
constexpr int kTargetBlocksInt8KV = 768;
constexpr int kInt8KVQuantum = 128;
constexpr int kMaxSplits = 128;         // splits per sequence, upper bound
constexpr int kSplitMajorUnits = 64;  // fixed-length launches of at least this many units run split-major
// Switches for the measured kernel variants (the same rule: defaults shipped).
#ifndef FA_DEC_PEEK
#define FA_DEC_PEEK 1
#endif
#ifndef FA_DEC_PIPE
#define FA_DEC_PIPE 1
#endif
#ifndef FA_DEC_TAIL_FIRST
#define FA_DEC_TAIL_FIRST 1
#endif
#ifndef FA_DEC_PRIO
#define FA_DEC_PRIO 1
#endif
#ifndef FA_DEC_PREFETCH2
#define FA_DEC_PREFETCH2 1
#endif

constexpr int kLptMaxSeqs = 512;      // longest-first ordering up to this many sequences

struct DecodeParams {
  const half_t* q;
  const half_t* k;
  const half_t* v;
  const int8_t* k8;            // INT8 KV cache: codes [B, H_KV, N, D]
  const int8_t* v8;
  const half_t* k_sc;          // INT8 KV cache: per-token scales [B, H_KV, N]
  const half_t* v_sc;
  half_t* o;
  const int32_t* lens;         // CB: cache_lens; paged: seq_lens
  const int32_t* block_table;  // paged
  long long bt_numel;
  const float* q_scale;        // INT8
  const float* k_scale;        // INT8
  float* ws_o;                 // [B*H_Q, S, DP] normalised partial outputs
  float* ws_lse;               // [B*H_Q, S] log2-sum-exp of each partial
  unsigned* counters;          // [kCounterSlots] arrival counters, one per unit; zero between calls
  int unit_base;               // first unit of this launch
  int B, H_Q, H_KV, N, D, G;
  int fixed_len;               // decode / INT8: number of attended keys
  int chunk, num_splits, num_hg;
  int max_num_blocks, num_pages;
  int lpt;                     // paged: serve sequences longest first
  int absorb_tail;             // fixed-length: split 0 also takes the keys past S * chunk
  int seg1, seg_shift;         // contiguous modes: key v < seg1 is row v, later keys row v + seg_shift
                               // (seg_shift = 0: identity; sliding window: sink run, then window run)
  float scale_log2;            // (1/sqrt(D)) * log2(e)
  float scale;                 // 1/sqrt(D) (INT8 score formula)
};

// Fetch the kernel arguments a mode uses at once: left to itself the compiler
// loads them in dependent rounds behind the early exits, a memory round trip
// each before the first key load can issue.
template <int MODE>
__device__ __forceinline__ void preload_args(const DecodeParams& p) {
  // gridDim.x (a hidden kernel argument) too: the split-major test needs it,
  // and fetched on its own it was a second dependent round trip
  asm volatile("" ::"s"(p.q), "s"(p.o), "s"(p.ws_o), "s"(p.ws_lse), "s"(p.counters), "s"(gridDim.x));
  asm volatile("" ::"s"(p.unit_base), "s"(p.B), "s"(p.H_Q), "s"(p.H_KV),
               "s"(p.N), "s"(p.D), "s"(p.G));
  asm volatile("" ::"s"(p.chunk), "s"(p.num_splits), "s"(p.num_hg), "s"(p.absorb_tail), "s"(p.scale_log2));
  if constexpr (MODE == kModeInt8KV) {
    asm volatile("" ::"s"(p.k8), "s"(p.v8), "s"(p.k_sc), "s"(p.v_sc), "s"(p.fixed_len), "s"(p.seg1),
                 "s"(p.seg_shift));
  } else {
    asm volatile("" ::"s"(p.k), "s"(p.v));
  }
  if constexpr (MODE == kModeInt8) asm volatile("" ::"s"(p.q_scale), "s"(p.k_scale), "s"(p.fixed_len), "s"(p.scale));
  if constexpr (MODE == kModeDecode) asm volatile("" ::"s"(p.fixed_len), "s"(p.seg1), "s"(p.seg_shift));
  if constexpr (MODE == kModeCB) asm volatile("" ::"s"(p.lens), "s"(p.seg1), "s"(p.seg_shift));
  if constexpr (MODE == kModePaged)
    asm volatile("" ::"s"(p.lens), "s"(p.lpt), "s"(p.block_table), "s"(p.bt_numel), "s"(p.max_num_blocks),
                 "s"(p.num_pages));
}

template <int MODE>
__device__ __forceinline__ int seq_len_of(const DecodeParams& p, int b) {
  if constexpr (MODE == kModeCB) {
    long long n = static_cast<long long>(p.lens[b]) + 1;  // cache_len + current token
    return n > p.N ? p.N : static_cast<int>(n);
  } else if constexpr (MODE == kModePaged) {
    return p.lens[b];
  } else {
    return p.fixed_len;
  }
}

// Eight fp16 values -> eight int8 codes clamp(roundf(h * inv), -127, 127),
// packed little-endian into two dwords.  Per value: clamp first (the bounds
// are integers, so clamp-then-round equals round-then-clamp; fminf maps NaN to
// +127), then round half away from zero as the truncating conversion of
// c + copysign(0.5 - 2^-25, c) (exact for |c| <= 127, ties included); two
// byte permutes and an OR pack four codes.
__device__ __forceinline__ int quant_rh(float x) {
  const float c = fmaxf(-127.0f, fminf(127.0f, x));
  return static_cast<int>(c + __builtin_copysignf(0.49999997f, c));
}

__device__ __forceinline__ int pack4_i8(int a, int b, int c, int d) {
  // perm(hi, lo, sel): selector byte k picks byte k' of lo (0-3) or of hi (4-7); 0x0c gives 0.
  return static_cast<int>(__builtin_amdgcn_perm(b, a, 0x0c0c0400u) | __builtin_amdgcn_perm(d, c, 0x04000c0cu));
}

__device__ __forceinline__ void quant8(u32x4 raw, float inv, int& lo, int& hi) {
  half8_t h = __builtin_bit_cast(half8_t, raw);
  int r[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = quant_rh(__builtin_fmaf(static_cast<float>(h[j]), inv, 0.0f));
  lo = pack4_i8(r[0], r[1], r[2], r[3]);
  hi = pack4_i8(r[4], r[5], r[6], r[7]);
}

// Eight int8 codes starting at column `col` of a row of length `d` (zero past d);
// VEC: one unconditional 8-byte load (col + 8 <= d, 8-byte aligned address).
template <bool VEC>
__device__ __forceinline__ u32x2 load_i8x8(const int8_t* row, int col, int d) {
  if constexpr (VEC) {
    (void)d;
    return *reinterpret_cast<const u32x2*>(row + col);
  } else {
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (col + j < d) w[j >> 2] |= static_cast<uint32_t>(static_cast<uint8_t>(row[col + j])) << (8 * (j & 3));
    return u32x2{w[0], w[1]};
  }
}

// Eight int8 codes c -> eight fp16 half(c * s), as the reference's
// __float2half((float)c * scale): c * s is exact in fp32 (8-bit by 11-bit
// significands), so the result is the exact product rounded once to fp16.
// Here: flip each code's top bit (u = c + 128), byte-permute u under 0x64 to
// get the fp16 value 1024 + u, subtract 1152 (exact: c), and multiply by s in
// packed fp16 -- an IEEE fp16 multiply is that same single rounding of the
// exact product.  Four permutes, four packed adds, four packed multiplies.
__device__ __forceinline__ u32x4 dequant_i8x8(u32x2 raw, half_t s) {
  const u32x2 x = raw ^ u32x2{0x80808080u, 0x80808080u};
  const half2_t bias = {static_cast<half_t>(-1152.0f), static_cast<half_t>(-1152.0f)};
  const half2_t sc = {s, s};
  u32x4 out;
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    // perm(hi, lo, sel): selector byte k picks byte k' of lo (0-3) or of hi (4-7)
    const uint32_t lo2 = __builtin_amdgcn_perm(0x64646464u, x[w], 0x05010400u);  // u0, u1 -> 1024 + u
    const uint32_t hi2 = __builtin_amdgcn_perm(0x64646464u, x[w], 0x05030402u);  // u2, u3
    out[2 * w] = as_u32((as_h2(lo2) + bias) * sc);
    out[2 * w + 1] = as_u32((as_h2(hi2) + bias) * sc);
  }
  return out;
}

// Per-wave LDS scratch used to hand probabilities from the MFMA layout (lane =
// key) to the row layout (lanes = one key's columns).
template <int GB>
struct PExchange {
  static constexpr int kPad = GB < 4 ? 4 : GB;
};

// Issue priority (s_setprio) from the iterations a wave has left: 3 with
// three or more, then 2, 1, and 0 once its walk is done.  Workgroups that
// share a CU then progress together instead of the older one (which the
// arbiter favours) finishing first and the younger one walking alone at the
// end.  Measured, same box: INT8 KV cache 18.2 -> 16.7 us, INT8 decode 28.3
// -> 28.0, continuous batching 181 -> 180.6, paged 176.6 -> 175.7; the
// contiguous fp16 modes (config 2, sliding window) measured no gain or a
// loss and keep the default priority.
template <int MODE>
__device__ __forceinline__ void prio_by_remaining(int left) {
  if constexpr (!FA_DEC_PRIO || MODE == kModeDecode) return;
  if (left >= 3) __builtin_amdgcn_s_setprio(3);
  else if (left == 2) __builtin_amdgcn_s_setprio(2);
  else __builtin_amdgcn_s_setprio(1);
}
template <int MODE>
__device__ __forceinline__ void prio_after_walk() {
  if constexpr (!FA_DEC_PRIO || MODE == kModeDecode) return;
  __builtin_amdgcn_s_setprio(0);
}

// Arrival counter of a launch's unit slot.  Consecutive slots sit in
// different 128-byte lines (32 counters apart), since atomics on one line
// are serialised: with the splits of eight units counting on one line, 256
// arrivals took up to 3 us; on separate lines about 1 us.
__device__ __forceinline__ int counter_index(int slot) {
  constexpr int kLines = static_cast<int>(kCounterSlotsDev / 32);
  return (slot % kLines) * 32 + slot / kLines;
}

template <int DP, int GB, int MODE, bool VEC, bool LDSK>
// Registers are the compiler's choice under the 256-thread bound (94-256
// VGPRs across the instantiations, none spilling); asking for four waves per
// SIMD made the INT8 KV cache spill (128 registers) and run 14 % slower.
__global__ __launch_bounds__(kDecThreads) void decode_splitkv_kernel(
    DecodeParams p) {
  constexpr int NC = DP / 32;                 // 32-column slices of the QK^T product
  constexpr int LPR = DP / 8;                 // lanes per key row in the row layout
  constexpr int RPW = 64 / LPR;               // rows covered by one row-layout load
  constexpr int T16 = DP == 256 ? 1 : 2;      // 16-key MFMA tiles per iteration
  constexpr int TK = 16 * T16;                // keys per wave per iteration
  constexpr int UV = TK / RPW;                // row-layout V loads per lane per iteration
  constexpr int GP = PExchange<GB>::kPad;     // padded heads per key in the exchange
  constexpr float kRescaleSlack = 8.0f;       // log2 headroom before the max is refreshed
  static_assert(TK % RPW == 0, "tile");
  preload_args<MODE>(p);

  const int S = p.num_splits;
  // Workgroup -> (unit slot, split).  Fixed-length launches of many units
  // deal the splits split-major (workgroup j: split j / units, unit j % units),
  // so the workgroups resident at any time spread over every unit's first
  // keys instead of one unit's whole range (sliding-window decode at
  // B = 16: 28.6 -> 27.7 us); small launches (config 2: 8 units, 9.3 us
  // split-major against 8.8) keep a unit's splits consecutive.
  constexpr bool kFixedLen = MODE == kModeDecode || MODE == kModeInt8 || MODE == kModeInt8KV;
  const int nslots = static_cast<int>(gridDim.x) / S;
  const bool split_major = kFixedLen && nslots >= kSplitMajorUnits;
  const int split = split_major ? static_cast<int>(blockIdx.x) / nslots : blockIdx.x % S;
  const int slot = split_major ? static_cast<int>(blockIdx.x) % nslots : blockIdx.x / S;  // this launch's counter slot
  const int rest = p.unit_base + slot;  // (b, h_kv, head group) unit
  const int hg = rest % p.num_hg;
  const int pair = rest / p.num_hg;
  const int hkv = pair % p.H_KV;
  const int D = p.D;
  const int G = p.G;
  const int g_base = hg * GB;
  const int g_valid = min(GB, G - g_base);  // heads of this group that exist

  const int tid = threadIdx.x;
  // Sequence served.  Paged decode with lpt set: unit rank r serves
  // the sequence of rank r in descending length order (ties by index), so the
  // longest sequences are dispatched first and the short ones fill the tail.
  int b = pair / p.H_KV;
  if constexpr (MODE == kModePaged) {
    if (p.lpt) {
      __shared__ int s_len[kLptMaxSeqs];
      __shared__ int s_seq;
      for (int i = tid; i < p.B; i += kDecThreads) s_len[i] = seq_len_of<MODE>(p, i);
      __syncthreads();
      const int r = b;
      for (int i = tid; i < p.B; i += kDecThreads) {
        const int li = s_len[i];
        int rank = 0;
        for (int j = 0; j < p.B; ++j) {
          const int lj = s_len[j];
          rank += (lj > li) || (lj == li && j < i);
        }
        if (rank == r) s_seq = i;
      }
      __syncthreads();
      b = s_seq;
    }
  }
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // MFMA layout: lane = (key l16 of a 16-key tile, quarter q)
  const int l16 = lane & 15;
  const int q4 = lane >> 4;
  // row layout: lane = (row group rg, 8 columns at col)
  const int rg = lane / LPR;
  const int col = (lane % LPR) * 8;

  const int L = seq_len_of<MODE>(p, b);
  // With absorb_tail (fixed-length calls only) the short remainder past
  // S * chunk (at most a quarter chunk) goes to split 0: [0, chunk + extra),
  // then split s takes [extra + s * chunk, +chunk).  Split 0 is dispatched
  // first, and on a CU shared with a later split's workgroup its waves are the
  // older ones and win the arbitration: 5b's splits 0-3 finished at 21.8,
  // 21.7, 24.1 and 26.5 us on average with the remainder on split 3, whose
  // one-key tile cost its waves a whole extra iteration.
  // Paged: the splits are planned over the table row (16 * max_num_blocks
  // tokens); a longer sequence keeps reading the flat table past its row, as
  // the reference does, and the last split takes all of those keys.
  int k0 = split * p.chunk;
  int k1;
  if (FA_DEC_TAIL_FIRST && p.absorb_tail) {
    const int extra = max(0, L - S * p.chunk);
    k0 = split == 0 ? 0 : extra + split * p.chunk;
    k1 = min(L, extra + (split + 1) * p.chunk);
  } else {
    const bool last_takes_rest = (p.absorb_tail || MODE == kModePaged) && split == S - 1;
    k1 = last_takes_rest ? L : min(L, k0 + p.chunk);
  }

  if (k0 >= k1) {
    // No key at all (L <= 0): the reference's acc/l_i is 0/0 there.  Split 0
    // writes the NaN; other empty splits just leave.
    if (L <= 0 && split == 0) {
      for (int i = tid; i < GB * D; i += kDecThreads) {
        const int g = i / D, d = i % D;
        if (g < g_valid) {
          const int h = hkv * G + g_base + g;
          p.o[(static_cast<size_t>(b) * p.H_Q + h) * D + d] = static_cast<half_t>(__builtin_nanf(""));
        }
      }
    }
    return;
  }

  // Splits that hold keys of this sequence (>= 1 here, since k0 < k1).
  const int sb = min(S, (L + p.chunk - 1) / p.chunk);

  // Paged: the page ids of the keys [r0, r1) being walked are staged in LDS,
  // kMaxChunk keys per round (one round unless the sequence overruns its
  // table row).  Token t's page id is block_table.flat[b * max_num_blocks +
  // t / 16] (flash_attn_kernel.cu:3438); a flat index past the table or a page
  // id outside [0, num_pages) would be an out-of-bounds read in the reference
  // and makes this sequence NaN instead.
  __shared__ int s_pages[MODE == kModePaged ? kMaxChunk / kPage : 1];
  __shared__ int s_bad;
  int r0 = k0, npages = 1;
  auto stage_pages = [&](int from, int to) {
    const int np = (to - from + kPage - 1) / kPage;
    for (int i = tid; i < np; i += kDecThreads) {
      const long long idx = static_cast<long long>(b) * p.max_num_blocks + from / kPage + i;
      int id = (idx >= 0 && idx < p.bt_numel) ? p.block_table[idx] : -1;
      if (id < 0 || id >= p.num_pages) {
        s_bad = 1;
        id = 0;
      }
      s_pages[i] = id;
    }
    __syncthreads();
    r0 = from;
    npages = np;
  };
  if constexpr (MODE == kModePaged) {
    if (tid == 0) s_bad = 0;
    __syncthreads();
  }

  // Row addressing.  Contiguous caches: one base per (b, h_kv) plus a 32-bit row
  // offset.  Paged cache: a 16-key MFMA tile and each row-layout load both lie
  // inside one page, so the page base is wave-uniform; rows past k1 inside the
  // last page are real page memory (their scores are masked), and page slots
  // past the round's last page are clamped to it.
  const size_t kv_head_base = (static_cast<size_t>(b) * p.H_KV + hkv) * static_cast<size_t>(p.N) * D;
  auto page_base = [&](int t) -> size_t {  // t: any key of the page, t >= r0
    const int slot = min((t - r0) >> 4, npages - 1);
    const int pg = __builtin_amdgcn_readfirstlane(s_pages[slot]);
    return (static_cast<size_t>(pg) * p.H_KV + hkv) * kPage * D;
  };

  // ---- query fragments: MFMA A operand, lane holds head l16, columns
  //      k_col(c) .. +8 of slice c (the K fragments use the same columns) ----
  // The score sums over every column once whatever the order, so the INT8 KV
  // cache pairs slices (c, c + 1) at 16 contiguous columns 16*q4 + 64*(c/2)
  // (+8 for c + 1): one 16-byte load of int8 codes per pair.  Other modes:
  // columns 32c + 8*q4.
  auto k_col = [&](int c) {
    if constexpr (MODE == kModeInt8KV && NC % 2 == 0) return 16 * q4 + 64 * (c / 2) + 8 * (c % 2);
    else return 32 * c + 8 * q4;
  };
  const int hq_lane = hkv * G + g_base + l16;  // head of this lane's A row
  const bool row_ok = l16 < g_valid;
  half8_t qa[NC];
  int qi8[NC][2];
  float qsc[4];  // INT8: q scale of the heads whose scores this lane holds (g = 4*q4 + r)
  float ks = 0.0f, inv_ks = 0.0f;
  if constexpr (MODE == kModeInt8) {
    ks = p.k_scale[static_cast<size_t>(b) * p.H_KV + hkv];
    inv_ks = 1.0f / ks;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int g = 4 * q4 + r;
      qsc[r] = g < g_valid ? p.q_scale[static_cast<size_t>(b) * p.H_Q + hkv * G + g_base + g] : 1.0f;
    }
  }
  {
    const half_t* qrow = p.q + (static_cast<size_t>(b) * p.H_Q + (row_ok ? hq_lane : 0)) * D;
    const float inv_qs = (MODE == kModeInt8 && row_ok)
                             ? 1.0f / p.q_scale[static_cast<size_t>(b) * p.H_Q + hq_lane] : 1.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      u32x4 x = u32x4{0u, 0u, 0u, 0u};
      if (row_ok) x = load_row8<VEC>(qrow, k_col(c), D);
      qa[c] = __builtin_bit_cast(half8_t, x);
      if constexpr (MODE == kModeInt8) quant8(x, inv_qs, qi8[c][0], qi8[c][1]);
    }
  }

  // Running state.  mu[r]: max (log2 domain) used for head g = 4*q4 + r, uniform
  // across the 16 key lanes of quarter q4.  lpart[r]: this lane's partial sum.
  float mu[4], lpart[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    mu[r] = kNegBig;
    lpart[r] = 0.0f;
  }
  float acc[GB][8];
#pragma unroll
  for (int g = 0; g < GB; ++g)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[g][j] = 0.0f;

  __shared__ __attribute__((aligned(16))) float s_p[kDecWaves][TK][GP];
  __shared__ float s_alpha[kDecWaves][GP];
  const int klast = k1 - 1;

  // Continuous batching and paged decode stage each wave's K tile in LDS:
  // HBM -> LDS copies (global_load_lds_dwordx4) read whole key rows, 16 lanes
  // per 256-byte row (a 32-key tile at D = 128 is 8 copies of 4 rows), where
  // loading K straight into the MFMA operand layout reads 64 bytes from each
  // of 16 rows per instruction.  The rows' 16-byte chunks are XOR-swizzled
  // (physical chunk = logical ^ (row % 16)) by the choice of source chunk per
  // lane, so the MFMA-layout reads (16 lanes = 16 rows at one chunk) hit 16
  // distinct bank groups.  Each wave owns its tile: no barriers.
  constexpr bool kLdsK = (MODE == kModeCB || MODE == kModePaged || LDSK) && VEC;
  // Every fp16 cache is read once per call: nontemporal loads (measured 11 %
  // faster on the paged cache, 2-3 % on contiguous and INT8 decode; the int8
  // cache's 8-byte V loads measured 8 % slower with them).
  constexpr bool kStreamKV = MODE != kModeInt8KV;
  constexpr int CPR = DP / 8;                   // 16-byte chunks per key row
  constexpr int KCOPIES = TK * CPR / 64;        // copies per lane per tile
  constexpr int RPC = 64 / CPR;                 // key rows per copy instruction
  static_assert(!kLdsK || (KCOPIES * 64 == TK * CPR && kPage % RPC == 0), "K copy shape");
  __shared__ __attribute__((aligned(16))) half_t s_k[kLdsK ? kDecWaves * TK * DP : 1];
  const unsigned k_lds = static_cast<unsigned>(reinterpret_cast<uintptr_t>(
                             (__attribute__((address_space(3))) half_t*)s_k)) + wave * (TK * DP * 2);
  // D = 64 rows are 128 bytes, two to a 256-byte bank window: rows 2j, 2j + 1
  // share a swizzle and differ in the window half
  auto kswz = [&](int r) { return CPR >= 16 ? (r & 15) : ((r >> 1) & 7); };
  auto k_copy = [&](int t0) {
    if constexpr (kLdsK) {
#pragma unroll
      for (int i = 0; i < KCOPIES; ++i) {
        const int slot = i * 64 + lane;
        const int r = slot / CPR;                       // key row of the tile
        const int lc = (slot % CPR) ^ kswz(r);          // logical chunk this lane fetches
        const unsigned dst = k_lds + i * 1024;
        if constexpr (MODE == kModePaged) {
          // all RPC rows of a copy lie in one page; rows past the split's last
          // page read that page again (masked)
          const half_t* pg = p.k + page_base(t0 + (i * RPC / kPage) * kPage);
          const unsigned off = static_cast<unsigned>((((t0 + r) & (kPage - 1)) * D + lc * 8) * 2);
          if constexpr (kStreamKV) copy16_to_lds_nt(pg, off, dst); else copy16_to_lds(pg, off, dst);
        } else {
          const half_t* kh = p.k + kv_head_base;
          const int t = min(t0 + r, klast);
          const int row = t < p.seg1 ? t : t + p.seg_shift;
          const unsigned off = static_cast<unsigned>((row * D + lc * 8) * 2);
          if constexpr (kStreamKV) copy16_to_lds_nt(kh, off, dst); else copy16_to_lds(kh, off, dst);
        }
      }
    }
  };
  // Pipelined walk (continuous batching, and contiguous fp16 decode launches
  // that stage K in LDS): V is staged in a second per-wave LDS buffer by the
  // same kind of copies, lane i of copy u landing its 16 bytes (its own
  // row-layout chunk) at u * 1024 + 16 i.  A tile's K fragments and V chunks
  // are read into registers as soon as its copies have landed, and the next
  // tile's copies are issued at once, so they travel while this tile's
  // scores, softmax and P V are computed.
  // (Config 3 186 -> 182 us, sliding-window B = 16 26.5 -> 26.1 us.  Paged
  // decode measured slower with it, 179 -> 180.5 us: its 78 KB workgroups
  // fit two per CU where three fit without; INT8 decode, 29.4 -> 30.6 us.)
  constexpr bool kPipe = FA_DEC_PIPE && kLdsK && (MODE == kModeCB || MODE == kModeDecode);
  __shared__ __attribute__((aligned(16))) half_t s_v[kPipe ? kDecWaves * TK * DP : 1];
  const unsigned v_lds = static_cast<unsigned>(reinterpret_cast<uintptr_t>(
                             (__attribute__((address_space(3))) half_t*)s_v)) + wave * (TK * DP * 2);
  static_assert(!kPipe || UV * 1024 == TK * DP * 2, "V copy shape");
  auto v_copy = [&](int t0) {
    if constexpr (kPipe) {
      const half_t* vh = p.v + kv_head_base;
#pragma unroll
      for (int u = 0; u < UV; ++u) {
        const int t = min(t0 + u * RPW + rg, klast);
        const int row = t < p.seg1 ? t : t + p.seg_shift;
        const unsigned off = static_cast<unsigned>((row * D + col) * 2);
        if constexpr (kStreamKV) copy16_to_lds_nt(vh, off, v_lds + u * 1024);
        else copy16_to_lds(vh, off, v_lds + u * 1024);
      }
    }
  };
  // K fragment (MFMA B operand) of 16-key tile tt, 32-column slice c
  auto k_frag = [&](int tt, int c) -> half8_t {
    const int r = 16 * tt + l16;
    return *lds_at<half8_t>(k_lds + (r * CPR + ((4 * c + q4) ^ kswz(r))) * 16);
  };

  // Continuous batching streams K/V with nontemporal loads (measured faster
  // there; slower for the paged gathers and the INT8 path).
  // One iteration's K (MFMA layout) and V (row layout) registers.
  struct Tile {
    u32x4 k[T16][NC];
    u32x4 v[UV];
  };
  // INT8 KV cache: one iteration's raw codes (K in the MFMA layout, V in the row
  // layout, eight codes per 8-byte load) and the scales of their token rows.
  struct Tile8 {
    u32x2 k[T16][NC];
    u32x2 v[UV];
    half_t ks[T16];
    half_t vs[UV];
  };
  auto load_tile8 = [&](Tile8& T, int t0) {
    const int8_t* kh = p.k8 + kv_head_base;
    const int8_t* vh = p.v8 + kv_head_base;
    const size_t sbase = (static_cast<size_t>(b) * p.H_KV + hkv) * static_cast<size_t>(p.N);
#pragma unroll
    for (int tt = 0; tt < T16; ++tt) {
      const int t = min(t0 + 16 * tt + l16, klast);
      T.ks[tt] = p.k_sc[sbase + t];
      if constexpr (VEC) {
        // slices c, c + 1 in one 16-byte load (columns k_col(c) .. +16)
#pragma unroll
        for (int c = 0; c < NC; c += 2) {
          const u32x4 x = *reinterpret_cast<const u32x4*>(kh + static_cast<size_t>(t) * D + k_col(c));
          T.k[tt][c] = u32x2{x[0], x[1]};
          T.k[tt][c + 1] = u32x2{x[2], x[3]};
        }
      } else {
#pragma unroll
        for (int c = 0; c < NC; ++c) T.k[tt][c] = load_i8x8<VEC>(kh + static_cast<size_t>(t) * D, k_col(c), D);
      }
    }
#pragma unroll
    for (int u = 0; u < UV; ++u) {
      const int t = min(t0 + u * RPW + rg, klast);
      T.vs[u] = p.v_sc[sbase + t];
      T.v[u] = load_i8x8<VEC>(vh + static_cast<size_t>(t) * D, col, D);
    }
  };
  // -- loads: rows past k1 are clamped to k1-1 (always valid memory) and their
  //    scores are masked in compute_tile.
  auto load_tile = [&](Tile& T, int t0) {
    if constexpr (kLdsK) k_copy(t0);  // K to LDS first: the V loads below complete after it
    if constexpr (MODE == kModePaged) {
      if constexpr (!kLdsK) {
#pragma unroll
        for (int tt = 0; tt < T16; ++tt) {
          const half_t* kr = p.k + page_base(t0 + 16 * tt) + l16 * D;
#pragma unroll
          for (int c = 0; c < NC; ++c) T.k[tt][c] = load_row8<VEC>(kr, 32 * c + 8 * q4, D);
        }
      }
#pragma unroll
      for (int u = 0; u < UV; ++u) {
        const int t = t0 + u * RPW;  // RPW divides 16: all rows of this load share a page
        T.v[u] = load_row8<VEC, kStreamKV>(p.v + page_base(t) + ((t + rg) & (kPage - 1)) * D, col, D);
      }
    } else {
      const half_t* kh = p.k + kv_head_base;
      const half_t* vh = p.v + kv_head_base;
      auto row_of = [&](int t) { return t < p.seg1 ? t : t + p.seg_shift; };
      if constexpr (!kLdsK) {
#pragma unroll
        for (int tt = 0; tt < T16; ++tt) {
          const int t = row_of(min(t0 + 16 * tt + l16, klast));
#pragma unroll
          for (int c = 0; c < NC; ++c) T.k[tt][c] = load_row8<VEC, kStreamKV>(kh + t * D, 32 * c + 8 * q4, D);
        }
      }
#pragma unroll
      for (int u = 0; u < UV; ++u) {
        const int t = row_of(min(t0 + u * RPW + rg, klast));
        T.v[u] = load_row8<VEC, kStreamKV>(vh + t * D, col, D);
      }
    }
  };

  auto compute_tile = [&](const Tile& T, int t0) {
    // -- scores S[g = 4*q4 + r][key = l16] for each 16-key tile
    float s[T16][4];
#pragma unroll
    for (int tt = 0; tt < T16; ++tt) {
      float4_t sc;
      if constexpr (MODE == kModeInt8) {
        typedef int int4v __attribute__((ext_vector_type(4)));
        int4v ci = {0, 0, 0, 0};
        if constexpr (kLdsK && !kPipe) {
          if (tt == 0) wait_vm<UV>();
        }
#pragma unroll
        for (int c = 0; c < NC; c += 2) {
          int k0lo, k0hi, k1lo, k1hi;
          if constexpr (kLdsK && !kPipe) {
            quant8(__builtin_bit_cast(u32x4, k_frag(tt, c)), inv_ks, k0lo, k0hi);
            quant8(__builtin_bit_cast(u32x4, k_frag(tt, c + 1)), inv_ks, k1lo, k1hi);
          } else {
            quant8(T.k[tt][c], inv_ks, k0lo, k0hi);
            quant8(T.k[tt][c + 1], inv_ks, k1lo, k1hi);
          }
          const int4v av = {qi8[c][0], qi8[c][1], qi8[c + 1][0], qi8[c + 1][1]};
          const int4v bv = {k0lo, k0hi, k1lo, k1hi};
          ci = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, ci, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
          sc[r] = static_cast<float>(ci[r]) * qsc[r] * ks * p.scale * kLog2e;
      } else {
        sc = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (kLdsK && !kPipe) {
          // this wave's K copies have landed once at most the UV later V loads are outstanding
          if (tt == 0) wait_vm<UV>();
#pragma unroll
          for (int c = 0; c < NC; ++c) sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[c], k_frag(tt, c), sc, 0, 0, 0);
        } else {
#pragma unroll
          for (int c = 0; c < NC; ++c)
            sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[c], __builtin_bit_cast(half8_t, T.k[tt][c]), sc, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[r] *= p.scale_log2;
      }
      const bool key_ok = t0 + 16 * tt + l16 < k1;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool ok = key_ok && (4 * q4 + r < g_valid);
        s[tt][r] = ok ? sc[r] : -INFINITY;
      }
    }

    // -- lazy max refresh: only when a score exceeds the max in use by 2^8
    bool grow = false;
#pragma unroll
    for (int tt = 0; tt < T16; ++tt)
#pragma unroll
      for (int r = 0; r < 4; ++r) grow |= s[tt][r] > mu[r] + kRescaleSlack;
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
      float alpha[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float mx = s[0][r];
#pragma unroll
        for (int tt = 1; tt < T16; ++tt) mx = fmaxf(mx, s[tt][r]);
        mx = fmaxf(mx, dpp_mov<kDppQuadXor1>(mx));
        mx = fmaxf(mx, dpp_mov<kDppQuadXor2>(mx));
        mx = fmaxf(mx, dpp_mov<kDppRowHalfMirror>(mx));
        mx = fmaxf(mx, dpp_mov<kDppRowMirror>(mx));
        const float mn = fmaxf(mu[r], mx);
        alpha[r] = fast_exp2(mu[r] - mn);
        mu[r] = mn;
        lpart[r] *= alpha[r];
      }
      // hand alpha to the row layout
      if (l16 == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (4 * q4 + r < GP) s_alpha[wave][4 * q4 + r] = alpha[r];
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int g = 0; g < GB; ++g) {
        const float a = s_alpha[wave][g];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[g][j] *= a;
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }

    // -- probabilities: exp, partial sums, and hand-off to the row layout
#pragma unroll
    for (int tt = 0; tt < T16; ++tt) {
      float pr[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pr[r] = fast_exp2(s[tt][r] - mu[r]);
        lpart[r] += pr[r];
      }
      if (4 * q4 < GP) {
        float* dst = &s_p[wave][16 * tt + l16][4 * q4];
        if constexpr (GP >= 4) {
          *reinterpret_cast<float4_t*>(dst) = float4_t{pr[0], pr[1], pr[2], pr[3]};
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();

    // -- O += P V in the row layout, two keys (loads u and u + 1: keys kl and
    //    kl + RPW) per v_dot2_f32_f16: P rounded to fp16 (as in the prefill's
    //    P V product), products exact, fp32 accumulation.
    static_assert(UV % 2 == 0, "V loads pair up");
#pragma unroll
    for (int u = 0; u < UV; u += 2) {
      const int kl = u * RPW + rg;  // key of load u inside this iteration's tile
      half2_t pp[GP];
#pragma unroll
      for (int g4 = 0; g4 < GP; g4 += 4) {
        const float4_t x0 = *reinterpret_cast<const float4_t*>(&s_p[wave][kl][g4]);
        const float4_t x1 = *reinterpret_cast<const float4_t*>(&s_p[wave][kl + RPW][g4]);
#pragma unroll
        for (int e = 0; e < 4; ++e) pp[g4 + e] = half2_t{static_cast<half_t>(x0[e]), static_cast<half_t>(x1[e])};
      }
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        // columns 2w, 2w+1 of both keys: {v_u[2w], v_u+1[2w]} and {v_u[2w+1], v_u+1[2w+1]}
        const uint32_t a = T.v[u][w], b = T.v[u + 1][w];
        const half2_t ve = as_h2(__builtin_amdgcn_perm(b, a, 0x05040100u));
        const half2_t vo = as_h2(__builtin_amdgcn_perm(b, a, 0x07060302u));
#pragma unroll
        for (int g = 0; g < GB; ++g) {
          acc[g][2 * w] = __builtin_amdgcn_fdot2(pp[g], ve, acc[g][2 * w], false);
          acc[g][2 * w + 1] = __builtin_amdgcn_fdot2(pp[g], vo, acc[g][2 * w + 1], false);
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
  };

  const int stride = kDecWaves * TK;
  // The waves walk the keys [from, to) in strides of kDecWaves * TK.  (The
  // tiles are locals of the loop body: kept in registers, not behind a
  // reference, or the compiler moves the INT8 scales to scratch memory.)
  auto walk = [&](int from, int to) {
    if constexpr (kPipe) {
      int t0 = from + wave * TK;
      if (t0 >= to) return;
      k_copy(t0);
      v_copy(t0);
      for (;;) {
        prio_by_remaining<MODE>((to - t0 + stride - 1) / stride);
        // this wave's copies of tile t0 have landed (no other vector-memory
        // operation is outstanding inside the walk)
        wait_vm<0>();
        Tile A;
#pragma unroll
        for (int tt = 0; tt < T16; ++tt)
#pragma unroll
          for (int c = 0; c < NC; ++c) A.k[tt][c] = __builtin_bit_cast(u32x4, k_frag(tt, c));
#pragma unroll
        for (int u = 0; u < UV; ++u) A.v[u] = *lds_at<u32x4>(v_lds + u * 1024 + lane * 16);
        const int tn = t0 + stride;
        const bool more = tn < to;
        if (more) {
          // the reads above have returned before the buffers are overwritten
          __builtin_amdgcn_sched_barrier(0);
          wait_vm_lgkm0<63>();
          k_copy(tn);
          v_copy(tn);
          __builtin_amdgcn_sched_barrier(0);
        }
        compute_tile(A, t0);
        if (!more) break;
        t0 = tn;
      }
      return;
    }
#if FA_DEC_PREFETCH2
    if constexpr (MODE == kModeDecode && !kLdsK) {
      // A wave with exactly two iterations (a split that took a short
      // remainder) issues both tiles' loads before computing either: the
      // second tile then costs its arithmetic, not another memory round trip
      // (config 2, where the absorbed remainder gives split 0 two tiles:
      // 9.3 -> 9.0 us).  Only the small grids that do not stage K in LDS take
      // this path, so the extra registers cost no occupancy that matters.
      const int t0 = from + wave * TK;
      if (t0 + stride < to && t0 + 2 * stride >= to) {
        Tile A, B;
        load_tile(A, t0);
        load_tile(B, t0 + stride);
        __builtin_amdgcn_sched_barrier(0);
        compute_tile(A, t0);
        compute_tile(B, t0 + stride);
        return;
      }
    }
#endif
    for (int t0 = from + wave * TK; t0 < to; t0 += stride) {
      prio_by_remaining<MODE>((to - t0 + stride - 1) / stride);
      Tile A;
      if constexpr (MODE == kModeInt8KV) {
        Tile8 R;
        load_tile8(R, t0);
#pragma unroll
        for (int tt = 0; tt < T16; ++tt)
#pragma unroll
          for (int c = 0; c < NC; ++c) A.k[tt][c] = dequant_i8x8(R.k[tt][c], R.ks[tt]);
#pragma unroll
        for (int u = 0; u < UV; ++u) A.v[u] = dequant_i8x8(R.v[u], R.vs[u]);
      } else {
        load_tile(A, t0);
      }
      // Contiguous decode: every load of the tile is issued before any of its
      // arithmetic (left to itself the scheduler put the first QK^T MFMA, and
      // its wait for Q and the first K rows, ahead of the V loads; config 2
      // 9.2 -> 9.05 us).  The INT8 modes measured slower with it (5b +4 %).
      // With K staged in LDS the barrier is also what the copies' wait relies
      // on: compute_tile's vmcnt(UV) counts exactly the UV V loads issued after
      // the K copies, so no other vector-memory load may be scheduled between
      // the copies and that wait.
      if constexpr (MODE == kModeDecode || kLdsK) __builtin_amdgcn_sched_barrier(0);
      compute_tile(A, t0);
    }
  };
  if constexpr (MODE == kModePaged) {
    static_assert(kMaxChunk % (kDecWaves * 32) == 0, "page rounds hold whole wave iterations");
    for (int rb = k0; rb < k1; rb += kMaxChunk) {
      const int re = k1 - rb > kMaxChunk ? rb + kMaxChunk : k1;
      if (rb != k0) __syncthreads();  // every wave is done with the previous round's ids
      stage_pages(rb, re);
      walk(rb, re);
    }
  } else {
    walk(k0, k1);
  }
  prio_after_walk<MODE>();

  // ---- wave-level reduction: all lanes of a wave share mu, so plain sums ----
#pragma unroll
  for (int r = 0; r < 4; ++r) lpart[r] = group_sum<16>(lpart[r]);

  // ---- merge the waves through LDS ----
  __shared__ float s_m[kDecWaves][GP];
  __shared__ float s_l[kDecWaves][GP];
  // The pipelined walk keeps its V buffers for the wave partials once every
  // wave is done with them (two 80 KB workgroups per CU instead of one).
  constexpr bool kAccInV = kPipe && GB * DP * 4 <= TK * DP * 2;
  __shared__ __attribute__((aligned(16))) float s_acc_own[kAccInV ? 1 : kDecWaves * GB * DP];
  typedef float AccBuf[kDecWaves][GB][DP];
  AccBuf& s_acc = *reinterpret_cast<AccBuf*>(kAccInV ? reinterpret_cast<float*>(s_v) : s_acc_own);
  if constexpr (kAccInV) __syncthreads();
  if (l16 == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int g = 4 * q4 + r;
      if (g < GP) {
        s_m[wave][g] = mu[r];
        s_l[wave][g] = lpart[r];
      }
    }
  }
  if constexpr (LPR == 16 && GB % 4 == 0) {
    // The four row groups (lanes l, l^16, l^32, l^48) hold partial sums of
    // the same columns.  Two lane-swap steps reduce four heads at once: the
    // 32-lane swap adds rows (0,2) and (1,3) of a head pair, the 16-lane swap
    // then adds rows (0,1) and (2,3) of two such pairs, leaving head 4hq + r
    // fully reduced in row r.  Each lane then writes its 8 columns of one head.
    const int r_row = lane >> 4;
#pragma unroll
    for (int hq = 0; hq < GB / 4; ++hq) {
      float u[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float x0 = acc[4 * hq + 0][j], x1 = acc[4 * hq + 2][j];
        float y0 = acc[4 * hq + 1][j], y1 = acc[4 * hq + 3][j];
        permlane32_swap(x0, x1);
        permlane32_swap(y0, y1);
        float z0 = x0 + x1, z1 = y0 + y1;
        permlane16_swap(z0, z1);
        u[j] = z0 + z1;
      }
      float* dst = &s_acc[wave][4 * hq + r_row][col];
      *reinterpret_cast<float4_t*>(dst) = float4_t{u[0], u[1], u[2], u[3]};
      *reinterpret_cast<float4_t*>(dst + 4) = float4_t{u[4], u[5], u[6], u[7]};
    }
  } else {
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1)
#pragma unroll
      for (int g = 0; g < GB; ++g)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[g][j] += __shfl_xor(acc[g][j], off, 64);
    if (rg == 0) {
#pragma unroll
      for (int g = 0; g < GB; ++g)
#pragma unroll
        for (int j = 0; j < 8; ++j) s_acc[wave][g][col + j] = acc[g][j];
    }
  }
  __syncthreads();

  bool bad = false;
  if constexpr (MODE == kModePaged) bad = s_bad != 0;
  // Peek (fixed-length launches that stage K in LDS, split-major): a split
  // that finds every other split of its unit already arrived is the merger;
  // it keeps its own partial in LDS (the K staging buffer, free after the
  // walk) instead of writing it out, waiting for the writes and taking an
  // arrival rank, i.e. one device round trip less on the path of the split
  // that finishes last.  Others publish as usual after the peek.
  constexpr bool kPeek = FA_DEC_PEEK && kLdsK && kFixedLen;
  __shared__ int s_peek;
  bool merger_now = false;
  float* own = reinterpret_cast<float*>(s_k);  // [GB][DP] partial, then [GB] log2-sum-exp
  static_assert(!kPeek || sizeof(s_k) >= (GB * DP + GB) * sizeof(float), "own partial fits the K buffer");
  if constexpr (kPeek) {
    if (split_major && sb > 1) {
      if (tid == 0)
        s_peek = __hip_atomic_load(&p.counters[counter_index(slot)], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 static_cast<unsigned>(sb - 1);
      __syncthreads();
      merger_now = s_peek != 0;
    }
  }
  // One thread per (head, 4 columns): every LDS read of the wave merge is
  // issued at once, then one 16-byte store of the split's partial.
  constexpr int NC4 = DP / 4;
  for (int i = tid; i < GB * NC4; i += kDecThreads) {
    const int g = i / NC4, d4 = (i % NC4) * 4;
    if (g >= g_valid || d4 >= D) continue;
    float mw[kDecWaves], lw[kDecWaves];
    float4_t aw[kDecWaves];
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) {
      mw[w] = s_m[w][g];
      lw[w] = s_l[w][g];
      aw[w] = *reinterpret_cast<const float4_t*>(&s_acc[w][g][d4]);
    }
    float mx = mw[0];
#pragma unroll
    for (int w = 1; w < kDecWaves; ++w) mx = fmaxf(mx, mw[w]);
    float lsum = 0.0f;
    float4_t a = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) {
      const float e = fast_exp2(mw[w] - mx);
      lsum += lw[w] * e;
      a += aw[w] * e;
    }
    float4_t outv = a / lsum;
    float lse = mx + __log2f(lsum);
    if (bad) {
      outv = float4_t{__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf("")};
      lse = __builtin_nanf("");
    }
    const int h = hkv * G + g_base + g;
    const size_t bh = static_cast<size_t>(b) * p.H_Q + h;
    if (sb == 1) {
      half_t* op = p.o + bh * D + d4;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (d4 + j < D) op[j] = static_cast<half_t>(outv[j]);
    } else if (kPeek && merger_now) {
      *reinterpret_cast<float4_t*>(&own[g * DP + d4]) = outv;
      if (d4 == 0) own[GB * DP + g] = lse;
    } else {
      const size_t e = bh * S + split;
      store_coherent4(&p.ws_o[e * DP + d4], outv);
      if (d4 == 0) store_coherent(&p.ws_lse[e], lse);
    }
  }
  if (sb == 1) return;

  // ---- publish this split's partial; the last-arriving split merges ----
  // Partials travel through device-coherent (L2-bypassing, sc1) stores and
  // loads, so no whole-L2 writeback/invalidate fence is needed.  Once all of
  // a split's partial stores are complete it takes its arrival rank on the
  // unit's counter; the split with the last rank finds every other partial
  // complete and merges at once.
  __shared__ int s_last;
  if (kPeek && merger_now) {
    __syncthreads();  // the own partial is in LDS
  } else {
    wait_vmem_stores();
    __syncthreads();
    if (tid == 0) {
      const unsigned arrival = atomicAdd(&p.counters[counter_index(slot)], 1u);
      s_last = (arrival == static_cast<unsigned>(sb - 1));
    }
    __syncthreads();
    if (!s_last) return;
  }
  // Every split of the unit has taken its arrival rank: the counter can go
  // back to zero for the next call on this workspace.
  if (tid == 0) __hip_atomic_store(&p.counters[counter_index(slot)], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // ---- merge ----
  // Thread (column group c, phase ph) merges 4 output columns over the splits
  // ph, ph + NPH, ..., in batches of NB loads, in split order (the result
  // does not depend on the arrival order).  Partials are read with
  // device-coherent (sc1) buffer loads.
  constexpr int NP = GB * DP / 4;                                  // float4 columns
  constexpr int NPH = NP >= kDecThreads ? 1 : kDecThreads / NP;    // split phases
  constexpr int NB = 16;                                           // splits per load batch
  constexpr int NCOL = (NP + kDecThreads - 1) / kDecThreads;       // columns per thread
  __shared__ float4_t s_num[NPH][NPH > 1 ? NP : 1];
  __shared__ float s_mx[NPH][NPH > 1 ? NP : 1];
  __shared__ float s_den[NPH][NPH > 1 ? NP : 1];
  const size_t unit_bh = static_cast<size_t>(b) * p.H_Q + hkv * G + g_base;
  const __amdgpu_buffer_rsrc_t ws_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(p.ws_o + unit_bh * S * DP, 0, 0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t lse_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(p.ws_lse + unit_bh * S, 0, 0x7fffffff, 0x00020000);
  struct Part {
    float4_t num;
    float mx, den;
  };
  auto column_ok = [&](int c) { return c < NP && c / (DP / 4) < g_valid && (c % (DP / 4)) * 4 < D; };
  // loads split sp of column c into (v, l)
  auto load_split = [&](int c, int sp, float4_t& v, float& l) {
    const int g = c / (DP / 4), d4 = (c % (DP / 4)) * 4;
    if (kPeek && merger_now && sp == split) {
      v = *reinterpret_cast<const float4_t*>(&own[g * DP + d4]);
      l = own[GB * DP + g];
      return;
    }
    v = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                         ws_rsrc, ((g * S + sp) * DP + d4) * static_cast<int>(sizeof(float)), 0, 16));
    l = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                      lse_rsrc, (g * S + sp) * static_cast<int>(sizeof(float)), 0, 16));
  };
  // online combine of one batch in split order
  auto combine = [&](Part& r, const float4_t (&v)[NB], const float (&lv)[NB]) {
    float m = r.mx;
#pragma unroll
    for (int j = 0; j < NB; ++j) m = fmaxf(m, lv[j]);
    const float a = fast_exp2(r.mx - m);
    r.num *= a;
    r.den *= a;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const float w = fast_exp2(lv[j] - m);
      r.den += w;
      r.num += w * v[j];
    }
    r.mx = m;
  };
  const int c_mine = NPH > 1 ? tid % NP : tid;
  const int ph = NPH > 1 ? tid / NP : 0;
  Part parts[NCOL];
#pragma unroll
  for (int q = 0; q < NCOL; ++q) parts[q] = Part{float4_t{0.0f, 0.0f, 0.0f, 0.0f}, -INFINITY, 0.0f};
  if (ph < NPH) {
#pragma unroll
    for (int q = 0; q < NCOL; ++q) {
      const int c = c_mine + q * kDecThreads;
      if (!column_ok(c)) continue;
      for (int k0 = ph; k0 < sb; k0 += NB * NPH) {
        float4_t v[NB];
        float lv[NB];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          v[j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
          lv[j] = -INFINITY;
          const int sp = k0 + j * NPH;
          if (sp < sb) load_split(c, sp, v[j], lv[j]);
        }
        combine(parts[q], v, lv);
      }
    }
  }

  auto store_out = [&](int c, float4_t o) {
    const int g = c / (DP / 4), d4 = (c % (DP / 4)) * 4;
    half_t* op = p.o + (unit_bh + g) * D + d4;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (d4 + j < D) op[j] = static_cast<half_t>(o[j]);
  };
  if constexpr (NPH == 1) {
#pragma unroll
    for (int q = 0; q < NCOL; ++q) {
      const int c = c_mine + q * kDecThreads;
      if (column_ok(c)) store_out(c, parts[q].num / parts[q].den);
    }
  } else {
    if (ph < NPH) {
      s_num[ph][c_mine] = parts[0].num;
      s_mx[ph][c_mine] = parts[0].mx;
      s_den[ph][c_mine] = parts[0].den;
    }
    __syncthreads();
    if (tid < NP && column_ok(tid)) {
      float m = s_mx[0][tid];
#pragma unroll
      for (int q = 1; q < NPH; ++q) m = fmaxf(m, s_mx[q][tid]);
      float4_t num = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
      float den = 0.0f;
#pragma unroll
      for (int q = 0; q < NPH; ++q) {
        const float w = s_mx[q][tid] == -INFINITY ? 0.0f : fast_exp2(s_mx[q][tid] - m);
        num += w * s_num[q][tid];
        den += w * s_den[q][tid];
      }
      store_out(tid, num / den);
    }
  }
}

// ---------------------------------------------------------------------------
// Host side: split planning and dispatch.

struct DecodePlan {
  int dp, gb, num_hg, chunk, splits;
};

static int pick_dp(int d) { return d <= 64 ? 64 : (d <= 128 ? 128 : 256); }
// Query heads per workgroup: one 16-row MFMA tile holds up to 16 heads of a group.
static int pick_gb(int g) { return g <= 1 ? 1 : (g <= 2 ? 2 : (g <= 4 ? 4 : (g <= 8 ? 8 : 16))); }

// absorb_tail (fixed-length calls): when the keys past the last full chunk
// are at most a quarter chunk, a full split (split 0, in the kernel) takes
// them too instead of a split of their own (e.g. 4097 keys in 256-key
// splits: 16 splits, not 17 -- one workgroup and one merge round trip less).
static DecodePlan make_plan(int B, int H_Q, int H_KV, int max_len, int D, int target_blocks,
                            bool absorb_tail = false, int quantum = kChunkQuantum) {
  DecodePlan pl;
  const int G = H_Q / H_KV;
  pl.dp = pick_dp(D);
  pl.gb = pick_gb(G);
  pl.num_hg = ceil_div(G, pl.gb);
  const long long units = static_cast<long long>(B) * H_KV * pl.num_hg;
  long long want = (static_cast<long long>(max_len > 0 ? max_len : 1) * units + target_blocks - 1) / target_blocks;
  long long chunk = ((want + quantum - 1) / quantum) * quantum;
  // at most kMaxSplits splits per sequence
  const long long min_chunk = (static_cast<long long>(max_len) + kMaxSplits - 1) / kMaxSplits;
  if (chunk < min_chunk) chunk = ((min_chunk + quantum - 1) / quantum) * quantum;
  if (chunk < quantum) chunk = quantum;
  if (chunk > kMaxChunk) chunk = kMaxChunk;
  pl.chunk = static_cast<int>(chunk);
  pl.splits = max_len > 0 ? ceil_div(max_len, chunk) : 1;
  if (absorb_tail && pl.splits > 1) {
    const long long tail = max_len - (pl.splits - 1) * chunk;
    if (tail <= chunk / 4 && chunk + tail <= kMaxChunk) --pl.splits;
  }
  return pl;
}

static size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// Workspace layout: [arrival counters: kCounterSlots u32][lse: B*H_Q*S f32]
// [partials: B*H_Q*S*DP f32], each region 256-byte aligned.  Needed only when
// a sequence can span several splits.  The counter region has the same size
// and place for every call, so one workspace can serve calls of any shape: no
// call's partials ever land on another call's counters.  A launch covers at
// most kCounterSlots units; larger problems are issued as several launches
// over unit ranges.
constexpr size_t kCounterSlots = kCounterSlotsDev;
constexpr size_t kCounterWords = kCounterSlots;

struct WorkspaceLayout {
  size_t counters, lse, o, total;
};

static WorkspaceLayout plan_layout(const DecodePlan& pl, int B, int H_Q, int H_KV) {
  (void)H_KV;
  WorkspaceLayout w = {0, 0, 0, 0};
  if (pl.splits <= 1) return w;
  const size_t entries = static_cast<size_t>(B) * H_Q * pl.splits;
  w.counters = 0;
  w.lse = align256(kCounterWords * sizeof(unsigned));
  w.o = w.lse + align256(entries * sizeof(float));
  w.total = w.o + entries * pl.dp * sizeof(float);
  return w;
}

// Contiguous and INT8 decode stage K in LDS (as continuous batching and
// paged decode do) when the launch has at least this many workgroups:
// row-coalesced copies pay off once the call is bandwidth-bound (sliding
// window at B = 16, 512 workgroups: 27.9 -> 26.7 us; INT8 at B = 16:
// 29.25 -> 29.0 us, its K quantized from the LDS fragments) but not for
// latency-bound small grids (config 2, 256 workgroups: 9.0 -> 9.2 us).
constexpr int kLdsKMinBlocks = 512;

template <int DP, int GB, int MODE, bool VEC>
static void launch_split(const DecodeParams& p, int blocks, hipStream_t st) {
  if constexpr ((MODE == kModeDecode || MODE == kModeInt8) && VEC) {
    if (blocks >= kLdsKMinBlocks) {
      hipLaunchKernelGGL((decode_splitkv_kernel<DP, GB, MODE, VEC, true>), dim3(blocks), dim3(kDecThreads), 0, st, p);
      return;
    }
  }
  hipLaunchKernelGGL((decode_splitkv_kernel<DP, GB, MODE, VEC, false>), dim3(blocks), dim3(kDecThreads), 0, st, p);
}

template <int DP, int MODE, bool VEC>
static void dispatch_gb(int gb, const DecodeParams& p, int blocks, hipStream_t st) {
  switch (gb) {
    case 1: launch_split<DP, 1, MODE, VEC>(p, blocks, st); break;
    case 2: launch_split<DP, 2, MODE, VEC>(p, blocks, st); break;
    case 4: launch_split<DP, 4, MODE, VEC>(p, blocks, st); break;
    case 8: launch_split<DP, 8, MODE, VEC>(p, blocks, st); break;
    default: launch_split<DP, 16, MODE, VEC>(p, blocks, st); break;
  }
}

template <int MODE>
static void dispatch(const DecodePlan& pl, bool vec, const DecodeParams& p, int blocks, hipStream_t st) {
  if (vec) {
    if (pl.dp == 64) dispatch_gb<64, MODE, true>(pl.gb, p, blocks, st);
    else if (pl.dp == 128) dispatch_gb<128, MODE, true>(pl.gb, p, blocks, st);
    else dispatch_gb<256, MODE, true>(pl.gb, p, blocks, st);
  } else {
    if (pl.dp == 64) dispatch_gb<64, MODE, false>(pl.gb, p, blocks, st);
    else if (pl.dp == 128) dispatch_gb<128, MODE, false>(pl.gb, p, blocks, st);
    else dispatch_gb<256, MODE, false>(pl.gb, p, blocks, st);
  }
}

static int check_common(const char* fn, int B, int H_Q, int H_KV, int D) {
  if (B < 0 || H_Q <= 0 || H_KV <= 0 || D <= 0)
    return set_error(FA_ERR_INVALID_ARG, "%s: sizes must be positive (B=%d H_Q=%d H_KV=%d D=%d)", fn, B, H_Q, H_KV, D);
  if (H_Q < H_KV || H_Q % H_KV != 0)
    return set_error(FA_ERR_INVALID_ARG, "%s: H_Q (%d) must be a multiple of H_KV (%d)", fn, H_Q, H_KV);
  if (D > 256) return set_error(FA_ERR_UNSUPPORTED, "%s: D=%d exceeds 256", fn, D);
  return FA_OK;
}

template <int MODE>
static int target_blocks() {
  if constexpr (MODE == kModeInt8KV) return kTargetBlocksInt8KV;
  return MODE == kModePaged ? kTargetBlocksPaged : (MODE == kModeCB ? kTargetBlocks : kTargetBlocksFixed);
}
// Split quantum of a fixed-length mode.
template <int MODE>
static int fixed_quantum() {
  return MODE == kModeInt8KV ? kInt8KVQuantum : kFixedQuantum;
}

// The split plan of a call.  Fixed-length calls split at multiples of
// kFixedQuantum keys; when that leaves CUs idle (fewer split workgroups than
// kSmallGridBlocks) they split at kSmallGridQuantum instead: one 32-key tile
// per wave, every load of the call issued at once (config 2: 16 -> 32 splits
// per head, 128 -> 256 workgroups; 64-key splits or none measured slower).
constexpr int kSmallGridQuantum = kDecWaves * 32;
constexpr long long kSmallGridBlocks = 256;

template <int MODE>
static DecodePlan plan_for(int B, int H_Q, int H_KV, int max_len, int D) {
  constexpr bool kFixed = MODE == kModeDecode || MODE == kModeInt8 || MODE == kModeInt8KV;
  if (!kFixed) return make_plan(B, H_Q, H_KV, max_len, D, target_blocks<MODE>(), false, kChunkQuantum);
  DecodePlan pl = make_plan(B, H_Q, H_KV, max_len, D, target_blocks<MODE>(), true, fixed_quantum<MODE>());
  const long long blocks = static_cast<long long>(B) * H_KV * pl.num_hg * pl.splits;
  if (blocks < kSmallGridBlocks) pl = make_plan(B, H_Q, H_KV, max_len, D, target_blocks<MODE>(), true, kSmallGridQuantum);
  return pl;
}

// max_len: keys of the longest sequence the call attends (fixed-length modes:
// exactly the attended count, which is at most N).
template <int MODE>
static int run_decode(const char* fn, DecodeParams p, int max_len, void* ws, size_t ws_bytes, void* stream) {
  constexpr bool kFixed = MODE == kModeDecode || MODE == kModeInt8 || MODE == kModeInt8KV;
  const DecodePlan pl = plan_for<MODE>(p.B, p.H_Q, p.H_KV, max_len, p.D);
  p.absorb_tail = kFixed ? 1 : 0;
  const WorkspaceLayout wl = plan_layout(pl, p.B, p.H_Q, p.H_KV);
  const size_t need = wl.total;
  if (need > 0 && (ws == nullptr || ws_bytes < need))
    return set_error(FA_ERR_WORKSPACE, "%s: workspace of %zu bytes required, %zu given", fn, need, ws_bytes);
  if (p.B == 0) return FA_OK;
  if (pl.splits > kMaxSplits)
    return set_error(FA_ERR_UNSUPPORTED, "%s: %d keys per sequence exceed %d", fn, max_len, kMaxSplits * kMaxChunk);
  p.G = p.H_Q / p.H_KV;
  // Longest first for paged decode only: its splits are long (a quarter of
  // the continuous-batching target), so a long sequence dispatched late
  // would trail the grid (config 4: 178 us with the order, 194 without).
  // Continuous batching splits finely enough that no workgroup trails by
  // much, and skipping the order's per-workgroup length ranking is faster
  // there (config 3: 184.7 us without, 187.4 with).
  p.lpt = MODE == kModePaged && p.B > 1 && p.B <= kLptMaxSeqs;
  p.chunk = pl.chunk;
  p.num_splits = pl.splits;
  p.num_hg = pl.num_hg;
  p.scale = 1.0f / sqrtf(static_cast<float>(p.D));
  p.scale_log2 = p.scale * kLog2e;
  if (need > 0) {
    char* base = static_cast<char*>(ws);
    p.counters = reinterpret_cast<unsigned*>(base + wl.counters);
    p.ws_lse = reinterpret_cast<float*>(base + wl.lse);
    p.ws_o = reinterpret_cast<float*>(base + wl.o);
  }
  // Vector path: D fills the padded width exactly and every row starts 16-byte aligned.
  const bool vec = (p.D == pl.dp) && aligned16(p.q) &&
                   (MODE == kModeInt8KV ? aligned16(p.k8) && aligned8(p.v8) : aligned16(p.k) && aligned16(p.v));
  const long long units = static_cast<long long>(p.B) * p.H_KV * pl.num_hg;
  hipStream_t st = static_cast<hipStream_t>(stream);
  for (long long u0 = 0; u0 < units; u0 += static_cast<long long>(kCounterSlots)) {
    const long long nu = units - u0 < static_cast<long long>(kCounterSlots) ? units - u0 : kCounterSlots;
    p.unit_base = static_cast<int>(u0);
    dispatch<MODE>(pl, vec, p, static_cast<int>(nu * pl.splits), st);
    const int rc = check_launch(fn);
    if (rc != FA_OK) return rc;
  }
  return FA_OK;
}

}  // namespace fa

using namespace fa;

extern "C" size_t fa_decode_workspace_size(int B, int H_Q, int H_KV, int max_len, int D) {
  if (B <= 0 || H_Q <= 0 || H_KV <= 0 || D <= 0 || D > 256 || H_Q % H_KV != 0) return 0;
  // Large enough for the plan of every mode at every key count up to max_len.
  // The split count is not monotonic in the key count (the chunk rounds up to
  // a quantum: 128 units of 1280 keys split 5 ways, of 1281 keys 3 ways), so
  // this bounds it instead of planning max_len: a plan with target T over u
  // units has chunk >= L u / T, hence at most ceil(T / u) splits (or
  // ceil(L / kMaxChunk) once the chunk is capped), and never more than
  // ceil(L / quantum) with the smallest quantum, nor more than kMaxSplits.
  DecodePlan pl = make_plan(B, H_Q, H_KV, max_len, D, kTargetBlocks);
  const long long units = static_cast<long long>(B) * H_KV * pl.num_hg;
  const long long tmax = std::max(kTargetBlocks, kTargetBlocksFixed);
  const long long L = std::max(max_len, 1);
  long long s = std::max((tmax + units - 1) / units, (L + kMaxChunk - 1) / kMaxChunk);
  s = std::min(s, (L + kSmallGridQuantum - 1) / kSmallGridQuantum);
  s = std::min(s, static_cast<long long>(kMaxSplits));
  pl.splits = static_cast<int>(s);
  return plan_layout(pl, B, H_Q, H_KV).total;
}

extern "C" int fa_decode_fp16(const void* q, const void* k, const void* v, void* o, int B, int H_Q,
                              int H_KV, int N, int D, int causal, int cache_len, void* workspace,
                              size_t workspace_bytes, void* stream) {
  const char* fn = "fa_decode_fp16";
  int rc = check_common(fn, B, H_Q, H_KV, D);
  if (rc != FA_OK) return rc;
  if (N <= 0) return set_error(FA_ERR_INVALID_ARG, "%s: N must be positive", fn);
  if (cache_len < 0 || cache_len >= N)
    return set_error(FA_ERR_INVALID_ARG, "%s: cache_len=%d must lie in [0, N=%d)", fn, cache_len, N);
  if (B > 0 && (!q || !k || !v || !o)) return set_error(FA_ERR_INVALID_ARG, "%s: null tensor pointer", fn);
  DecodeParams p = {};
  p.q = static_cast<const half_t*>(q);
  p.k = static_cast<const half_t*>(k);
  p.v = static_cast<const half_t*>(v);
  p.o = static_cast<half_t*>(o);
  p.B = B; p.H_Q = H_Q; p.H_KV = H_KV; p.N = N; p.D = D;
  p.fixed_len = causal ? cache_len + 1 : N;
  return run_decode<kModeDecode>(fn, p, p.fixed_len, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free decode: the split workspace lives in a static device array.
//
// `scratch` is one array per GPU (each device that loads this library holds
// its own copy until the process ends).  Host code never uses its name as an
// address: the device address comes from hipGetSymbolAddress, once per device
// with that device current, and only that pointer is passed to kernels or
// memory calls.  The region the kernels expect at zero (the arrival
// counters) starts at zero (static storage, and a
// synchronous clear at set-up when the first call is not being captured),
// and every call leaves them at zero.  Calls that overlap on one GPU share
// the array and race.
constexpr size_t kStaticScratchBytes = 16u << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {
constexpr int kMaxScratchDevices = 64;
struct ScratchSlot {
  std::once_flag once;
  void* ptr = nullptr;
  hipError_t err = hipSuccess;
};
ScratchSlot g_scratch[kMaxScratchDevices];

// Device address of this device's `scratch`, resolved on the first call.
int static_scratch(const char* fn, void* stream, void** out) {
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(FA_ERR_HIP, "%s: hipGetDevice: %s", fn, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return set_error(FA_ERR_UNSUPPORTED, "%s: device %d beyond %d", fn, dev, kMaxScratchDevices);
  ScratchSlot& slot = g_scratch[dev];
  std::call_once(slot.once, [&]() {
    void* ptr = nullptr;
    slot.err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (slot.err != hipSuccess) return;
    slot.ptr = ptr;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cap) == hipSuccess &&
        cap == hipStreamCaptureStatusNone) {
      const size_t zero_bytes = align256(kCounterWords * sizeof(unsigned));
      slot.err = hipMemset(ptr, 0, zero_bytes);
    }
  });
  if (slot.err != hipSuccess)
    return set_error(FA_ERR_HIP, "%s: static scratch set-up: %s", fn, hipGetErrorString(slot.err));
  *out = slot.ptr;
  return FA_OK;
}
}  // namespace

extern "C" int fa_decode_fp16_noalloc(const void* q, const void* k, const void* v, void* o, int B, int H_Q,
                                      int H_KV, int N, int D, int causal, int cache_len, void* stream) {
  const char* fn = "fa_decode_fp16_noalloc";
  int rc = check_common(fn, B, H_Q, H_KV, D);
  if (rc != FA_OK) return rc;
  if (N <= 0) return set_error(FA_ERR_INVALID_ARG, "%s: N must be positive", fn);
  if (cache_len < 0 || cache_len >= N)
    return set_error(FA_ERR_INVALID_ARG, "%s: cache_len=%d must lie in [0, N=%d)", fn, cache_len, N);
  const int attended = causal ? cache_len + 1 : N;
  const size_t need = plan_layout(plan_for<kModeDecode>(B, H_Q, H_KV, attended, D), B, H_Q, H_KV).total;
  if (need > kStaticScratchBytes)
    return set_error(FA_ERR_UNSUPPORTED,
                     "%s: this call needs a %zu-byte split workspace; the static scratch holds %zu bytes "
                     "(use fa_decode_fp16 with a caller workspace)", fn, need, kStaticScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    rc = static_scratch(fn, stream, &ws);
    if (rc != FA_OK) return rc;
  }
  return fa_decode_fp16(q, k, v, o, B, H_Q, H_KV, N, D, causal, cache_len, ws, need, stream);
}

extern "C" int fa_decode_sliding_window_gqa(const void* q, const void* k, const void* v, void* o, int B,
                                           int H_Q, int H_KV, int N, int D, int cache_len, int window_size,
                                           int sink_size, void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "fa_decode_sliding_window_gqa";
  int rc = check_common(fn, B, H_Q, H_KV, D);
  if (rc != FA_OK) return rc;
  if (N <= 0) return set_error(FA_ERR_INVALID_ARG, "%s: N must be positive", fn);
  if (B > 0 && (!q || !k || !v || !o)) return set_error(FA_ERR_INVALID_ARG, "%s: null tensor pointer", fn);
  // Attended keys: k < sink_size (whatever cache_len is), and
  // window_start <= k <= cache_len with window_start = max(0, min(cache_len+1, N) - window_size).
  // As one key sequence: the sink run [0, L1), then the window run from max(window_start, L1).
  const long long eff_end = std::min<long long>(static_cast<long long>(cache_len) + 1, N);
  const long long wstart = std::max<long long>(0, eff_end - window_size);
  const int L1 = static_cast<int>(std::min<long long>(std::max(sink_size, 0), N));
  const long long lo = std::max<long long>(wstart, L1);
  const long long hi = std::min<long long>(cache_len, static_cast<long long>(N) - 1);
  const int L2 = hi >= lo ? static_cast<int>(hi - lo + 1) : 0;
  DecodeParams p = {};
  p.q = static_cast<const half_t*>(q);
  p.k = static_cast<const half_t*>(k);
  p.v = static_cast<const half_t*>(v);
  p.o = static_cast<half_t*>(o);
  p.B = B; p.H_Q = H_Q; p.H_KV = H_KV; p.N = N; p.D = D;
  p.fixed_len = L1 + L2;
  p.seg1 = L1;
  p.seg_shift = static_cast<int>(lo - L1);
  return run_decode<kModeDecode>(fn, p, p.fixed_len, workspace, workspace_bytes, stream);
}

extern "C" int fa_continuous_batching_fp16(const void* q, const void* k, const void* v, void* o,
                                           const int32_t* cache_lens, int B, int H_Q, int H_KV,
                                           int max_N, int D, int causal, void* workspace,
                                           size_t workspace_bytes, void* stream) {
  (void)causal;  // keys past cache_len are never read, so causal masks nothing more
  const char* fn = "fa_continuous_batching_fp16";
  int rc = check_common(fn, B, H_Q, H_KV, D);
  if (rc != FA_OK) return rc;
  if (max_N <= 0) return set_error(FA_ERR_INVALID_ARG, "%s: max_N must be positive", fn);
  if (B > 0 && (!q || !k || !v || !o || !cache_lens))
    return set_error(FA_ERR_INVALID_ARG, "%s: null pointer", fn);
  DecodeParams p = {};
  p.q = static_cast<const half_t*>(q);
  p.k = static_cast<const half_t*>(k);
  p.v = static_cast<const half_t*>(v);
  p.o = static_cast<half_t*>(o);
  p.lens = cache_lens;
  p.B = B; p.H_Q = H_Q; p.H_KV = H_KV; p.N = max_N; p.D = D;
  return run_decode<kModeCB>(fn, p, max_N, workspace, workspace_bytes, stream);
}

extern "C" int fa_paged_decode_gqa_fp16(const void* q, const void* k_cache, const void* v_cache,
                                        void* o, const int32_t* block_table,
                                        int64_t block_table_numel, const int32_t* seq_lens, int B,
                                        int H_Q, int H_KV, int D, int num_pages,
                                        int max_num_blocks, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  const char* fn = "fa_paged_decode_gqa_fp16";
  int rc = check_common(fn, B, H_Q, H_KV, D);
  if (rc != FA_OK) return rc;
  if (num_pages < 0 || max_num_blocks < 0 || block_table_numel < 0)
    return set_error(FA_ERR_INVALID_ARG, "%s: negative page count / table size", fn);
  if (B > 0 && (!q || !o || !seq_lens || ((!k_cache || !v_cache || !block_table) && num_pages > 0)))
    return set_error(FA_ERR_INVALID_ARG, "%s: null pointer", fn);
  const long long max_len_ll = static_cast<long long>(max_num_blocks) * kPage;
  if (max_len_ll > 0x3fffffffLL) return set_error(FA_ERR_UNSUPPORTED, "%s: max_num_blocks too large", fn);
  DecodeParams p = {};
  p.q = static_cast<const half_t*>(q);
  p.k = static_cast<const half_t*>(k_cache);
  p.v = static_cast<const half_t*>(v_cache);
  p.o = static_cast<half_t*>(o);
  p.lens = seq_lens;
  p.block_table = block_table;
  p.bt_numel = block_table_numel;
  p.B = B; p.H_Q = H_Q; p.H_KV = H_KV; p.N = 0; p.D = D;
  p.max_num_blocks = max_num_blocks;
  p.num_pages = num_pages;
  // Splits are planned over tokens [0, 16*max_num_blocks); the last split also
  // takes the tokens of a sequence that overruns its table row.
  const int plan_len = max_len_ll > 0 ? static_cast<int>(max_len_ll) : 1;
  return run_decode<kModePaged>(fn, p, plan_len, workspace, workspace_bytes, stream);
}

extern "C" int fa_decode_int8_gqa(const void* q, const void* k, const void* v, void* o,
                                  const float* q_scale, const float* k_scale, int B, int H_Q,
                                  int H_KV, int N, int D, int cache_len, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  const char* fn = "fa_decode_int8_gqa";
  int rc = check_common(fn, B, H_Q, H_KV, D);
  if (rc != FA_OK) return rc;
  if (N <= 0) return set_error(FA_ERR_INVALID_ARG, "%s: N must be positive", fn);
  if (cache_len < 0 || cache_len >= N)
    return set_error(FA_ERR_INVALID_ARG, "%s: cache_len=%d must lie in [0, N=%d)", fn, cache_len, N);
  if (B > 0 && (!q || !k || !v || !o || !q_scale || !k_scale))
    return set_error(FA_ERR_INVALID_ARG, "%s: null pointer", fn);
  DecodeParams p = {};
  p.q = static_cast<const half_t*>(q);
  p.k = static_cast<const half_t*>(k);
  p.v = static_cast<const half_t*>(v);
  p.o = static_cast<half_t*>(o);
  p.q_scale = q_scale;
  p.k_scale = k_scale;
  p.B = B; p.H_Q = H_Q; p.H_KV = H_KV; p.N = N; p.D = D;
  p.fixed_len = cache_len + 1;
  return run_decode<kModeInt8>(fn, p, p.fixed_len, workspace, workspace_bytes, stream);
}

extern "C" int fa_decode_int8_kv_cache_gqa(const void* q, const void* k_int8, const void* v_int8,
                                          const void* k_scale, const void* v_scale, void* o, int B, int H_Q,
                                          int H_KV, int N, int D, int cache_len, void* workspace,
                                          size_t workspace_bytes, void* stream) {
  const char* fn = "fa_decode_int8_kv_cache_gqa";
  int rc = check_common(fn, B, H_Q, H_KV, D);
  if (rc != FA_OK) return rc;
  if (N <= 0) return set_error(FA_ERR_INVALID_ARG, "%s: N must be positive", fn);
  if (B > 0 && (!q || !k_int8 || !v_int8 || !k_scale || !v_scale || !o))
    return set_error(FA_ERR_INVALID_ARG, "%s: null pointer", fn);
  DecodeParams p = {};
  p.q = static_cast<const half_t*>(q);
  p.k8 = static_cast<const int8_t*>(k_int8);
  p.v8 = static_cast<const int8_t*>(v_int8);
  p.k_sc = static_cast<const half_t*>(k_scale);
  p.v_sc = static_cast<const half_t*>(v_scale);
  p.o = static_cast<half_t*>(o);
  p.B = B; p.H_Q = H_Q; p.H_KV = H_KV; p.N = N; p.D = D;
  // keys k <= cache_len always (cache_len unchecked: past N every key, below 0 none -> NaN)
  p.fixed_len = static_cast<int>(std::min<long long>(std::max<long long>(static_cast<long long>(cache_len) + 1, 0), N));
  return run_decode<kModeInt8KV>(fn, p, p.fixed_len, workspace, workspace_bytes, stream);
}
