// MFMA-tiled online-softmax prefill for gfx950 (dense MHA/GQA and packed varlen).
//
// Workgroup = 4 waves; each wave owns RW = 32 query rows of one (batch, head),
// so a workgroup covers 128 rows.  The KV sequence is walked in 32-key tiles
// that stream through a ring of NS LDS stages (3 for D <= 64, 2 above; on
// N(0,1) data two stages ran 5a 2 % faster than three at D = 128).  Each
// stage holds one K and one V tile, unpadded, with the 16-byte chunks of row r
// XOR-swizzled by chunk_swizzle(r) so that both LDS read patterns below are
// free of bank conflicts:
//   K   read 16 B per lane as the A operand of S^T = K Q^T
//   V   read with ds_read_b64_tr_b16 as the A operand of O^T = V^T P^T
// Tiles are copied HBM -> LDS by global_load_lds_dwordx4 (no VGPR staging), NS-1
// tiles ahead of the one being computed, with one barrier per tile; every
// wave waits (vmcnt) only for its own copies of the current tile.  Shapes the
// DMA cannot serve (D not 64/128/256 or unaligned rows) stage through registers
// into the same layout.
//
// S^T = K Q^T puts one query row per lane (lane l owns query l%32 of each block
// and 16 keys of each 32-key block): the row max needs one exchange (lanes l,
// l^32) and the row sum stays lane-partial until the end.  The fp32 S^T
// accumulator, converted to fp16, is directly the B operand of the PV product:
// inside each 16-key slice lane half h holds keys {4h..4h+3, 8+4h..8+4h+3}, and
// the transposing LDS read delivers V in exactly that key order (one read per
// 4-key run: 16 source lanes read a 4-key x 16-column block of row-major V and
// lane i receives the 4 keys of column i).
//
// Online softmax with lazy rescaling: the exponentials use the running max,
// which is only refreshed (and O, l rescaled) when some p of a tile would
// exceed 2^8, detected from the lane's partial sum (wave-uniform test), so the
// row max is rarely computed and the O accumulators rarely touched outside the
// MFMAs.  Only tiles that cross the causal diagonal or the sequence end apply
// the mask (a wave-uniform branch around the mask step alone); each wave stops
// computing at its own diagonal but keeps copying its share of later tiles.
// Work items are dealt XCD by XCD (the dispatcher sends workgroup j to XCD
// j % 8): each XCD owns a set of KV heads and runs them in groups of about
// 128 workgroups (under two resident rounds), heaviest query tile first
// within a group, so the query tiles that share K/V tiles run together
// behind one L2 and the hardware dispatcher packs the lighter ones into the
// tail.
#include <math.h>

#include <algorithm>

#include "capi_internal.h"
#include "common.h"

namespace fa {

constexpr int kPreWaves = 4;
constexpr int kXcds = 8;  // XCDs per MI355X; workgroups are dealt to them round-robin
#ifndef FA_PRE_ORDER
#define FA_PRE_ORDER 1
#endif
#ifndef FA_PRE_GROUP_WGS
#define FA_PRE_GROUP_WGS 128
#endif
// Workgroups per XCD scheduling group: 128 measured 2 % faster than 384 on 5a
// (and 1-5 % on dense causal N = 1024-4096); 96 and 192 made dense N = 4096
// 6-12 % slower (groups of unequal unit counts).
constexpr long long kGroupWorkgroups = FA_PRE_GROUP_WGS;
constexpr int kPreThreads = kPreWaves * 64;

struct PrefillParams {
  const half_t* q;
  const half_t* k;
  const half_t* v;
  half_t* o;
  float* lse;                 // dense only: natural-log log-sum-exp [B, H_Q, N], written if non-null
  const int32_t* cu_seqlens;  // varlen only
  int B, H_Q, H_KV, N, D, G;
  int total, row_limit;       // varlen only
  int causal;
  int qtiles;                 // query tiles per (batch, head) in the grid
  int zero_base;              // varlen only: first workgroup of the zero-fill tail
  int group_units;            // KV heads per XCD scheduling group
  float scale_log2;           // (1/sqrt(D)) * log2(e)
};

// Tile shape per padded head dim.  The FA_PRE_* macros are tuning hooks for
// building variants; the defaults are the shipped configuration.
//
// Ablation hooks (FA_ABL_*, off by default) remove one part of the tile loop
// so that a timed run shows what that part costs; such a build computes wrong
// results and is only ever timed:
//   FA_ABL_NOCOPY   no tile copies after the first NS - 1 (the waits return at once)
//   FA_ABL_HOTCOPY  every copy reads the sequence's first tile (always cache-resident)
//   FA_ABL_NOQK     no QK^T MFMAs (and no K fragment reads)
//   FA_ABL_NOPV     no P V MFMAs
#ifndef FA_PRE_RB64
#define FA_PRE_RB64 1
#endif
#ifndef FA_PRE_BK64
#define FA_PRE_BK64 32
#endif
#ifndef FA_PRE_W64
#define FA_PRE_W64 4
#endif
#ifndef FA_PRE_NSW
#define FA_PRE_NSW 4
#endif
#ifndef FA_PRE_NS128
#define FA_PRE_NS128 2
#endif
#ifndef FA_PRE_W128
#define FA_PRE_W128 3
#endif
// WIDE (D <= 64 only): 64-key tiles for launches of at most about one
// residency round of workgroups, where fewer, longer tiles per barrier win
// (measured 5-12 % on N <= 1024); larger launches keep 32-key tiles.  Their
// ring has 4 stages, so three tiles are in flight from the start (short
// sequences: most of the keys).
//
// KSPLIT (D <= 128, launches far smaller than the chip): the four waves share
// one 32-row query block and split every 128-key tile, wave w taking keys
// 32w .. 32w + 31; their partial (max, sum, O) merge through LDS at the end.
// Each wave's serial chain is then a quarter of the keys, which is what bounds
// short prefills that occupy only a few dozen CUs.
template <int DP, bool WIDE = false, bool KSPLIT = false>
struct PrefillShape {
  static constexpr int RB = KSPLIT ? 1 : (DP <= 64 ? FA_PRE_RB64 : 1);  // 32-row query blocks per wave
  static constexpr int RW = 32 * RB;                                    // query rows per wave
  static constexpr int BQ = KSPLIT ? RW : kPreWaves * RW;               // query rows per workgroup
  static constexpr int BK = KSPLIT ? 32 * kPreWaves : (DP <= 64 ? (WIDE ? 64 : FA_PRE_BK64) : 32);  // keys per tile
  static constexpr int NS = KSPLIT ? (DP <= 64 ? 3 : 2)
                                   : (DP <= 64 ? (WIDE ? FA_PRE_NSW : 3) : (DP <= 128 ? FA_PRE_NS128 : 2));  // LDS ring stages
  static constexpr int TILE = BK * DP;                                  // halves per K (or V) tile
  static constexpr int WAVES_PER_SIMD =
      KSPLIT ? 2 : (DP <= 64 ? (WIDE ? 3 : FA_PRE_W64) : (DP <= 128 ? FA_PRE_W128 : 2));  // register budget target
};

// Varlen output rows that no sequence's attention writes are set to zero by
// batch + 1 extra workgroups: workgroup b < batch clears rows
// [cu[b] + min(len_b, row_limit), cu[b+1]) of sequence b, workgroup batch
// clears [0, cu[0]) and [cu[batch], total).  Any row outside every
// [cu[b], cu[b+1]) lies before cu[0] or at/after cu[batch] (the boundaries
// are a path from cu[0] to cu[batch]), so every unwritten row is cleared; for
// valid (non-decreasing) cu_seqlens the cleared rows are exactly the unwritten
// ones and the ranges are usually empty.
__device__ void zero_unwritten_rows(const PrefillParams& p, int z) {
  const size_t row_halves = static_cast<size_t>(p.H_Q) * p.D;
  auto clamp_row = [&](int r) { return max(0, min(r, p.total)); };
  auto clear = [&](int r0, int r1) {
    if (r0 >= r1) return;
    half_t* base = p.o + static_cast<size_t>(r0) * row_halves;
    const size_t n = static_cast<size_t>(r1 - r0) * row_halves;
    if ((reinterpret_cast<uintptr_t>(base) & 15) == 0 && (n & 7) == 0) {
      for (size_t i = threadIdx.x; i < n / 8; i += kPreThreads)
        reinterpret_cast<u32x4*>(base)[i] = u32x4{0u, 0u, 0u, 0u};
    } else {
      for (size_t i = threadIdx.x; i < n; i += kPreThreads) base[i] = static_cast<half_t>(0.0f);
    }
  };
  if (z < p.B) {
    const int s = clamp_row(p.cu_seqlens[z]);
    const int e = clamp_row(p.cu_seqlens[z + 1]);
    const int len = e - s;
    clear(s + max(0, min(len, p.row_limit)), e);
  } else {
    clear(0, clamp_row(p.cu_seqlens[0]));
    clear(clamp_row(p.cu_seqlens[p.B]), p.total);
  }
}

__device__ __forceinline__ void preload_args(const PrefillParams& p) {
  asm volatile("" ::"s"(p.q), "s"(p.k), "s"(p.v), "s"(p.o), "s"(p.lse), "s"(p.cu_seqlens));
  asm volatile("" ::"s"(p.B), "s"(p.H_Q), "s"(p.H_KV), "s"(p.N), "s"(p.D), "s"(p.G), "s"(p.total), "s"(p.row_limit));
  asm volatile("" ::"s"(p.causal), "s"(p.qtiles), "s"(p.zero_base), "s"(p.group_units), "s"(p.scale_log2));
}

template <int DP, bool VARLEN, bool VEC, bool WIDE = false, bool KSPLIT = false>
__global__ __launch_bounds__(kPreThreads)
__attribute__((amdgpu_waves_per_eu(PrefillShape<DP, WIDE, KSPLIT>::WAVES_PER_SIMD))) void prefill_kernel(PrefillParams p) {
  using Shape = PrefillShape<DP, WIDE, KSPLIT>;
  constexpr int RB = Shape::RB;
  constexpr int RW = Shape::RW;
  constexpr int BQ = Shape::BQ;
  constexpr int kBK = Shape::BK;
  constexpr int NS = Shape::NS;
  constexpr int TILE = Shape::TILE;
  constexpr int NBLK = KSPLIT ? 1 : kBK / 32;  // 32-key blocks per tile computed by one wave
  constexpr int KK = DP / 16;                 // 16-wide d slices of QK^T
  constexpr int DB = DP / 32;                 // 32-row d blocks of PV
  constexpr int CPR = DP / 8;                 // 16-byte chunks per row
  constexpr int IPW = TILE / 8 / 64 / kPreWaves;  // 16-byte copies per lane per tensor per tile
  constexpr float kRescaleLimit = 256.0f;  // 2^8: largest p before the max is refreshed
  static_assert(IPW * 8 * 64 * kPreWaves == TILE, "tile must split evenly over the waves");

  __shared__ __attribute__((aligned(1024))) half_t smem[NS * 2 * Shape::TILE];

  // Fetch every kernel argument at once: left to itself the compiler loads
  // them in several dependent rounds behind the early exits, each a memory
  // round trip before the first tile copy can issue.
  preload_args(p);
  const int D = p.D;
  if constexpr (VARLEN) {
    if (static_cast<int>(blockIdx.x) >= p.zero_base) {
      zero_unwritten_rows(p, static_cast<int>(blockIdx.x) - p.zero_base);
      return;
    }
  }
#if FA_PRE_ORDER == 0
  // Heaviest work first: all (batch, head) pairs of the last query tile, then the next.
  const int pairs = p.H_Q * p.B;
  const int qt = p.qtiles - 1 - static_cast<int>(blockIdx.x / pairs);
  const int rem = blockIdx.x % pairs;
  const int h = rem % p.H_Q;
  const int b = rem / p.H_Q;
  const int hk = h / p.G;
#else
  // XCD-grouped order: workgroup j runs on XCD j % 8 (the dispatcher deals
  // workgroups round-robin over the 8 XCDs), so XCD x owns the KV heads
  // (batch, KV head) units u = x, x + 8, ...  Its stream j / 8 takes them in
  // groups of p.group_units units and, inside a group, heaviest query tile
  // first over all the group's (unit, query head) pairs.  A group's
  // workgroups run together on one XCD and walk the same K/V tiles through
  // its L2; the heaviest-first order inside the group keeps the tail short.
  const int j = static_cast<int>(blockIdx.x);
  const int xcd = j % kXcds;
  const int i = j / kXcds;
  const int heads_per_group = p.group_units * p.G;
  const int group = i / (heads_per_group * p.qtiles);
  const int ii = i % (heads_per_group * p.qtiles);
  const int qt = p.qtiles - 1 - ii / heads_per_group;
  const int hg = ii % heads_per_group;
  const int u = xcd + kXcds * (group * p.group_units + hg / p.G);  // (batch, KV head) unit
  if (u >= p.B * p.H_KV) return;
  const int hk = u % p.H_KV;
  const int b = u / p.H_KV;
  const int h = hk * p.G + hg % p.G;
#endif

  // ---- sequence geometry ----
  size_t q_base, k_base, stride;
  int seq_len, rows;
  if constexpr (VARLEN) {
    int s = p.cu_seqlens[b];
    int e = p.cu_seqlens[b + 1];
    s = max(0, min(s, p.total));
    e = max(0, min(e, p.total));
    seq_len = e - s;
    rows = min(seq_len, p.row_limit);
    stride = static_cast<size_t>(p.H_Q) * D;
    q_base = static_cast<size_t>(s) * stride + static_cast<size_t>(h) * D;
    k_base = q_base;
  } else {
    seq_len = rows = p.N;
    stride = D;
    q_base = (static_cast<size_t>(b) * p.H_Q + h) * static_cast<size_t>(p.N) * D;
    k_base = (static_cast<size_t>(b) * p.H_KV + hk) * static_cast<size_t>(p.N) * D;
  }
  const int q0 = qt * BQ;
  if (q0 >= rows) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  const int wq0 = q0 + (KSPLIT ? 0 : wave * RW);  // first query row of this wave
  const int kw = KSPLIT ? 32 * wave : 0;            // first key of this wave's block inside a tile

  const half_t* __restrict__ qp = p.q + q_base;
  const half_t* __restrict__ kp = p.k + k_base;
  const half_t* __restrict__ vp = p.v + k_base;

  // key ranges: the workgroup walks to its last wave's diagonal, each wave stops at its own
  const int kend_wg = p.causal ? min(seq_len, q0 + BQ) : seq_len;
  // a wave whose rows all lie past the written rows computes nothing (it still
  // copies its share of every tile and joins the barriers)
  const int kend_w = wq0 >= rows ? 0 : (p.causal ? min(seq_len, wq0 + RW) : seq_len);
  const int ntiles = (kend_wg + kBK - 1) / kBK;

  // ---- tile copies: slot g = (wave*IPW + i)*64 + lane of a tile holds logical
  //      chunk (g % CPR) ^ swizzle(row) of row g / CPR ----
  const unsigned lds_base = static_cast<unsigned>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) half_t*)smem));
  constexpr unsigned kStageBytes = 2 * TILE * sizeof(half_t);
  constexpr unsigned kTileBytes = TILE * sizeof(half_t);
  int cp_row[IPW], cp_col[IPW];
  unsigned cp_off[IPW];  // byte offset of the lane's chunk from the tile's first row
#pragma unroll
  for (int i = 0; i < IPW; ++i) {
    const int g = (wave * IPW + i) * 64 + lane;
    cp_row[i] = g / CPR;
    cp_col[i] = ((g % CPR) ^ chunk_swizzle<DP>(g / CPR)) * 8;
    cp_off[i] = static_cast<unsigned>((cp_row[i] * stride + cp_col[i]) * sizeof(half_t));
  }
  auto issue = [&](int t) {
#ifdef FA_ABL_NOCOPY
    if (t >= NS - 1) return;
#endif
#ifdef FA_ABL_HOTCOPY
    const int kt = 0;
#else
    const int kt = t * kBK;
#endif
    const unsigned sk = lds_base + (t % NS) * kStageBytes;
    const half_t* kb = kp + static_cast<size_t>(kt) * stride;
    const half_t* vb = vp + static_cast<size_t>(kt) * stride;
    const bool tail = kt + kBK > seq_len;  // rows past the sequence end re-read its last row
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
      const int row = tail ? min(cp_row[i], seq_len - 1 - kt) : cp_row[i];
      const unsigned slot = sk + (wave * IPW + i) * 1024;
      if constexpr (VEC) {
        const unsigned off = tail ? static_cast<unsigned>((row * stride + cp_col[i]) * sizeof(half_t)) : cp_off[i];
        copy16_to_lds(kb, off, slot);
        copy16_to_lds(vb, off, slot + kTileBytes);
      } else {
        const u32x4 kx = load_row8<false>(kb + static_cast<size_t>(row) * stride, cp_col[i], D);
        const u32x4 vx = load_row8<false>(vb + static_cast<size_t>(row) * stride, cp_col[i], D);
        *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(static_cast<size_t>(slot + lane * 16)) = kx;
        *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(static_cast<size_t>(slot + kTileBytes + lane * 16)) = vx;
      }
    }
  };
#pragma unroll
  for (int t = 0; t < NS - 1; ++t)
    if (t < ntiles) issue(t);

  // ---- Q fragments: B operand of S^T; block rb, lane row wq0 + 32 rb + l32, d = 16 kk + 8 hi .. +8 ----
  half8_t qf[RB][KK];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int qrow = wq0 + 32 * rb + l32;
    const half_t* qr = qp + static_cast<size_t>(min(qrow, rows - 1)) * stride;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      u32x4 x = load_row8<VEC>(qr, kk * 16 + 8 * hi, D);
      if (qrow >= rows) x = u32x4{0u, 0u, 0u, 0u};
      qf[rb][kk] = __builtin_bit_cast(half8_t, x);
    }
  }

  float16_t oacc[DB][RB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[db][rb][r] = 0.0f;
  float m_run[RB], l_run[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    m_run[rb] = kNegBig;
    l_run[rb] = 0.0f;
  }
  const float c = p.scale_log2;

  // Per-lane LDS read byte offsets with the swizzle folded in; the
  // compile-time part of each chunk index is XORed in per read (the stage
  // base has no bits in the chunk field).
  //   K: row l32 (+32 blk), logical chunk 2 kk + hi.
  const unsigned k_lane = (l32 * DP + ((chunk_swizzle<DP>(l32) ^ hi) * 8)) * sizeof(half_t);
  //   V: source lane s = lane % 16 reads row 16 i + 8 j + 4 hi + s/4, columns
  //   32 db + 16 ((lane >> 4) & 1) + 4 (s & 3) .. +4.
  const int s16 = lane & 15;
  const int v_row = 4 * hi + (s16 >> 2);
  const int v_sw = (DP <= 64 ? ((((s16 >> 2) >> 1) & 1) << 2) : ((s16 >> 2) << 2)) | hi;
  const unsigned v_lane =
      (v_row * DP + (((2 * ((lane >> 4) & 1) + ((s16 & 3) >> 1)) ^ v_sw) * 8) + (s16 & 1) * 4) * sizeof(half_t);

  using STile = float16_t[NBLK][RB];
  // ---- S^T = K Q^T of tile t ----
  auto qk_tile = [&](const int t, STile& sacc) {
    const unsigned kaddr = lds_base + (t % NS) * kStageBytes + k_lane + kw * DP * 2;
#pragma unroll
    for (int blk = 0; blk < NBLK; ++blk)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[blk][rb][r] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
#pragma unroll
      for (int blk = 0; blk < NBLK; ++blk) {
        const half8_t a = *lds_at<half8_t>((kaddr ^ (32 * kk)) + blk * 32 * DP * 2);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
#ifdef FA_ABL_NOQK
          if (kk == 0) sacc[blk][rb][0] += static_cast<float>(a[0]);
#else
          sacc[blk][rb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[rb][kk], sacc[blk][rb], 0, 0, 0);
#endif
        }
      }
    }
  };
  // ---- softmax and O^T += V^T P^T of tile t ----
  auto softmax_pv = [&](const int t, STile& sacc, const bool masked) {
    const int kt = t * kBK + kw;  // first key of the wave's keys in this tile
    const unsigned vaddr = lds_base + (t % NS) * kStageBytes + kTileBytes + v_lane + kw * DP * 2;
    // ---- softmax (lane owns query row wq0 + 32 rb + l32) ----
    half8_t pf[RB][2 * NBLK];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      if (masked) {  // uniform: only tiles crossing the diagonal or the sequence end
        // Element r of block blk holds key kt + 4 hi + off (off = 32 blk +
        // 8 (r / 4) + r % 4, a constant); it is dead past the lane's last live
        // key, so one compare against a per-lane bound masks it.
        const int qrow = wq0 + 32 * rb + l32;
        const int last = p.causal ? min(qrow, seq_len - 1) : seq_len - 1;
        const int bound = last - kt - 4 * hi;  // live iff off <= bound
#pragma unroll
        for (int blk = 0; blk < NBLK; ++blk)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int off = blk * 32 + 8 * (r >> 2) + (r & 3);
            sacc[blk][rb][r] = off > bound ? -INFINITY : sacc[blk][rb][r];
          }
      }
      // p = exp2(s c - m) against the running max m.  A lane's partial sum can
      // only exceed 2^slack if one of its p did, i.e. some score outgrew m by
      // more than the slack (always the case on the first tile, m = -1e30):
      // only then is the tile's row max taken, m raised and O, l rescaled.
      auto exponentiate = [&](float mneg) {
        float ls = 0.0f;
#pragma unroll
        for (int i = 0; i < 2 * NBLK; ++i) {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float e = fast_exp2(fmaf(sacc[i >> 1][rb][8 * (i & 1) + j], c, mneg));
            ls += e;
            pf[rb][i][j] = static_cast<half_t>(e);
          }
        }
        return ls;
      };
      // Tile 0 always sets the max (m = -1e30 before it): skip the trial pass.
      float ls = t == 0 ? 2.0f * kRescaleLimit : exponentiate(-m_run[rb]);
      if (__builtin_amdgcn_ballot_w64(ls > kRescaleLimit) != 0) {
        float mx = sacc[0][rb][0];
#pragma unroll
        for (int blk = 0; blk < NBLK; ++blk)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[blk][rb][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * c;
        const float mn = fmaxf(m_run[rb], mx);
        const float alpha = fast_exp2(m_run[rb] - mn);
        m_run[rb] = mn;
        l_run[rb] *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[db][rb][r] *= alpha;
        ls = exponentiate(-mn);
      }
      l_run[rb] += ls;
    }
    // ---- O^T += V^T P^T ----
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int i = 0; i < 2 * NBLK; ++i) {
        half4_t part[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const unsigned src = (vaddr ^ (16 * (4 * db ^ 2 * j))) + (16 * i + 8 * j) * DP * 2;
          const short4_t x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              const_cast<__attribute__((address_space(3))) short4_t*>(lds_at<short4_t>(src)));
          part[j] = __builtin_bit_cast(half4_t, x);
        }
        const half8_t a = __builtin_shufflevector(part[0], part[1], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
#ifdef FA_ABL_NOPV
          oacc[db][rb][i] += static_cast<float>(a[0]) + static_cast<float>(pf[rb][i][0]);
#else
          oacc[db][rb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pf[rb][i], oacc[db][rb], 0, 0, 0);
#endif
        }
      }
    }
  };
  auto compute_tile = [&](const int t, const bool masked) {
    STile sacc;
    qk_tile(t, sacc);
    softmax_pv(t, sacc, masked);
  };

  for (int t = 0; t < ntiles; ++t) {
    // this wave's copies of tile t have landed (tile t+1 may still be in flight)
    if (VEC && NS > 3 && t + 2 < ntiles)
      wait_vm_lgkm0<4 * IPW>();
    else if (VEC && NS > 2 && t + 1 < ntiles)
      wait_vm_lgkm0<2 * IPW>();
    else
      wait_vm_lgkm0<0>();
    tile_barrier();  // every wave's copies of tile t landed; stage (t-1) % NS is free
    if (t + NS - 1 < ntiles) issue(t + NS - 1);
    const int kt = t * kBK + kw;
    constexpr int kWaveKeys = KSPLIT ? 32 : kBK;  // keys of a tile this wave computes
    if (kt >= kend_w) continue;  // past this wave's diagonal (still copies and joins the barriers)
    compute_tile(t, (kt + kWaveKeys > seq_len) || (p.causal && kt + kWaveKeys - 1 > wq0));
  }

  if constexpr (KSPLIT) {
    // ---- merge the four waves' partials of the shared 32 rows ----
    // Lane (l32, hi) holds O[l32][32 db + 8 rr + 4 hi + j] = oacc[db][0][4 rr + j]
    // against its wave's max m; scaled to the common max M, the waves' O and
    // l add up.  A wave that saw no key keeps m = -1e30 and weighs 0.
    __shared__ float s_mw[kPreWaves][32];
    __shared__ float s_lw[kPreWaves][32];
    __syncthreads();  // every wave is done reading the ring
    // [wave][32 rows][DP + 4] fp32: the 16-byte row pad spreads the 32 rows
    // of one column block over distinct banks
    constexpr int RS = DP + 4;
    float* red = reinterpret_cast<float*>(smem);
    if (hi == 0) s_mw[wave][l32] = m_run[0];
    __syncthreads();
    float mx = s_mw[0][l32];
#pragma unroll
    for (int w = 1; w < kPreWaves; ++w) mx = fmaxf(mx, s_mw[w][l32]);
    const float alpha = fast_exp2(m_run[0] - mx);
    const float lw = (l_run[0] + __shfl_xor(l_run[0], 32, 64)) * alpha;
    if (hi == 0) s_lw[wave][l32] = lw;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        float4_t x;
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = oacc[db][0][4 * rr + j] * alpha;
        *reinterpret_cast<float4_t*>(red + (wave * 32 + l32) * RS + db * 32 + 8 * rr + 4 * hi) = x;
      }
    __syncthreads();
    // thread: row tid / 8, columns (tid % 8) * DP / 8 .. + DP / 8
    constexpr int CPT = DP / 8;
    const int r = tid >> 3;
    const int c0 = (tid & 7) * CPT;
    const int qrow = q0 + r;
    if (qrow < rows) {
      float lt = 0.0f;
#pragma unroll
      for (int w = 0; w < kPreWaves; ++w) lt += s_lw[w][r];
      const float inv = 1.0f / lt;
      if constexpr (!VARLEN) {
        if (p.lse != nullptr && (tid & 7) == 0) {
          float m = s_mw[0][r];
#pragma unroll
          for (int w = 1; w < kPreWaves; ++w) m = fmaxf(m, s_mw[w][r]);
          p.lse[(static_cast<size_t>(b) * p.H_Q + h) * p.N + qrow] = (m + log2f(lt)) * 0.69314718055994531f;
        }
      }
      half_t* op = p.o + q_base + static_cast<size_t>(qrow) * stride;
#pragma unroll
      for (int c = 0; c < CPT; c += 4) {
        float4_t acc = *reinterpret_cast<const float4_t*>(red + r * RS + c0 + c);
#pragma unroll
        for (int w = 1; w < kPreWaves; ++w) {
          const float4_t y = *reinterpret_cast<const float4_t*>(red + (w * 32 + r) * RS + c0 + c);
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[j] += y[j];
        }
        half4_t hv;
#pragma unroll
        for (int j = 0; j < 4; ++j) hv[j] = static_cast<half_t>(acc[j] * inv);
        if constexpr (VEC) {
          *reinterpret_cast<half4_t*>(op + c0 + c) = hv;
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (c0 + c + j < D) op[c0 + c + j] = hv[j];
        }
      }
    }
    return;
  }

  // ---- finalize and store O[qrow][d] ----
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const float lt = l_run[rb] + __shfl_xor(l_run[rb], 32, 64);
    const int qrow = wq0 + 32 * rb + l32;
    if (qrow >= rows) continue;
    const float inv = 1.0f / lt;
    if constexpr (!VARLEN) {
      // l is the sum of exp2(s c - m) against the running m, so m + log2(l) is
      // the log2-sum-exp of the row whichever m the lazy rescaling settled on.
      if (p.lse != nullptr && hi == 0)
        p.lse[(static_cast<size_t>(b) * p.H_Q + h) * p.N + qrow] = (m_run[rb] + log2f(lt)) * 0.69314718055994531f;
    }
    half_t* op = p.o + q_base + static_cast<size_t>(qrow) * stride;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int d0 = db * 32 + 8 * rr + 4 * hi;
        half4_t hv;
#pragma unroll
        for (int j = 0; j < 4; ++j) hv[j] = static_cast<half_t>(oacc[db][rb][4 * rr + j] * inv);
        if constexpr (VEC) {
          *reinterpret_cast<half4_t*>(op + d0) = hv;
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (d0 + j < D) op[d0 + j] = hv[j];
        }
      }
    }
  }
}

template <int DP, bool VARLEN, bool WIDE = false, bool KSPLIT = false>
static void launch_prefill(bool vec, int blocks, const PrefillParams& p, hipStream_t st) {
  if (vec)
    hipLaunchKernelGGL((prefill_kernel<DP, VARLEN, true, WIDE, KSPLIT>), dim3(blocks), dim3(kPreThreads), 0, st, p);
  else
    hipLaunchKernelGGL((prefill_kernel<DP, VARLEN, false, WIDE, KSPLIT>), dim3(blocks), dim3(kPreThreads), 0, st, p);
}
constexpr long long kWideMaxBlocks = 1024;  // D <= 64 launches up to this size use 64-key tiles
// D <= 128 launches of at most this many 128-row workgroups run key-split
// (four times as many 32-row workgroups).
#ifndef FA_PRE_KSPLIT_MAX
#define FA_PRE_KSPLIT_MAX 64
#endif
constexpr long long kKsplitMaxBlocks = FA_PRE_KSPLIT_MAX;

static int prefill_bq(int D) { return D <= 64 ? PrefillShape<64>::BQ : (D <= 128 ? PrefillShape<128>::BQ : PrefillShape<256>::BQ); }

// Launches qtiles * H_Q * B attention workgroups (plus the varlen zero-fill
// tail); returns FA_OK or an error code.
template <bool VARLEN>
static int dispatch_prefill(const char* fn, int D, bool vec, int rows_max, PrefillParams p, hipStream_t st) {
  const bool ksplit = D <= 128 && static_cast<long long>(ceil_div(rows_max, prefill_bq(D))) * p.H_Q * p.B <= kKsplitMaxBlocks;
  p.qtiles = ceil_div(rows_max, ksplit ? PrefillShape<64, false, true>::BQ : prefill_bq(D));
#if FA_PRE_ORDER == 0
  const long long main_blocks = static_cast<long long>(p.qtiles) * p.H_Q * p.B;
#else
  const long long units = static_cast<long long>(p.B) * p.H_KV;
  const long long units_per_xcd = (units + kXcds - 1) / kXcds;
  const long long per_unit = static_cast<long long>(p.G) * p.qtiles;
  p.group_units = static_cast<int>(std::max<long long>(1, std::min<long long>(units_per_xcd, (kGroupWorkgroups + per_unit - 1) / per_unit)));
  const long long groups = (units_per_xcd + p.group_units - 1) / p.group_units;
  const long long main_blocks = groups * p.group_units * kXcds * per_unit;
#endif
  const long long blocks = main_blocks + (VARLEN ? p.B + 1 : 0);
  if (blocks > 0x7fffffffLL) return set_error(FA_ERR_UNSUPPORTED, "%s: problem too large for one launch", fn);
  if (blocks == 0) return FA_OK;
  p.zero_base = static_cast<int>(main_blocks);
  if (ksplit) {
    if (D <= 64) launch_prefill<64, VARLEN, false, true>(vec, static_cast<int>(blocks), p, st);
    else launch_prefill<128, VARLEN, false, true>(vec, static_cast<int>(blocks), p, st);
  } else if (D <= 64) {
    if (main_blocks <= kWideMaxBlocks) launch_prefill<64, VARLEN, true>(vec, static_cast<int>(blocks), p, st);
    else launch_prefill<64, VARLEN>(vec, static_cast<int>(blocks), p, st);
  }
  else if (D <= 128) launch_prefill<128, VARLEN>(vec, static_cast<int>(blocks), p, st);
  else launch_prefill<256, VARLEN>(vec, static_cast<int>(blocks), p, st);
  return check_launch(fn);
}

}  // namespace fa

using namespace fa;

static int prefill_dense(const char* fn, const void* q, const void* k, const void* v, void* o, float* lse, int B,
                         int H_Q, int H_KV, int N, int D, int causal, void* stream) {
  if (B < 0 || N < 0 || H_Q <= 0 || H_KV <= 0 || D <= 0)
    return set_error(FA_ERR_INVALID_ARG, "%s: bad sizes (B=%d H_Q=%d H_KV=%d N=%d D=%d)", fn, B, H_Q, H_KV, N, D);
  if (H_Q < H_KV || H_Q % H_KV != 0)
    return set_error(FA_ERR_INVALID_ARG, "%s: H_Q (%d) must be a multiple of H_KV (%d)", fn, H_Q, H_KV);
  if (D > 256) return set_error(FA_ERR_UNSUPPORTED, "%s: D=%d exceeds 256", fn, D);
  if (B == 0 || N == 0) return FA_OK;
  if (!q || !k || !v || !o) return set_error(FA_ERR_INVALID_ARG, "%s: null tensor pointer", fn);
  PrefillParams p = {};
  p.q = static_cast<const half_t*>(q);
  p.k = static_cast<const half_t*>(k);
  p.v = static_cast<const half_t*>(v);
  p.o = static_cast<half_t*>(o);
  p.lse = lse;
  p.B = B; p.H_Q = H_Q; p.H_KV = H_KV; p.N = N; p.D = D; p.G = H_Q / H_KV;
  p.causal = causal ? 1 : 0;
  p.scale_log2 = (1.0f / sqrtf(static_cast<float>(D))) * kLog2e;
  // Vector path: D fills the padded width exactly and every row starts 16-byte aligned.
  const bool vec = (D == 64 || D == 128 || D == 256) && aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o);
  return dispatch_prefill<false>(fn, D, vec, N, p, static_cast<hipStream_t>(stream));
}

extern "C" int fa_prefill_fp16(const void* q, const void* k, const void* v, void* o, int B, int H_Q,
                               int H_KV, int N, int D, int causal, void* stream) {
  return prefill_dense("fa_prefill_fp16", q, k, v, o, nullptr, B, H_Q, H_KV, N, D, causal, stream);
}

extern "C" int fa_prefill_fp16_lse(const void* q, const void* k, const void* v, void* o, float* lse, int B,
                                   int H, int N, int D, int causal, void* stream) {
  if (lse == nullptr && B > 0 && N > 0)
    return set_error(FA_ERR_INVALID_ARG, "fa_prefill_fp16_lse: null lse pointer");
  return prefill_dense("fa_prefill_fp16_lse", q, k, v, o, lse, B, H, H, N, D, causal, stream);
}

extern "C" int fa_varlen_prefill_fp16(const void* q, const void* k, const void* v, void* o,
                                      const int32_t* cu_seqlens, int batch, int total, int H,
                                      int D, int max_seqlen, int row_limit, int causal,
                                      void* stream) {
  const char* fn = "fa_varlen_prefill_fp16";
  if (batch < 0 || total < 0 || H <= 0 || D <= 0 || max_seqlen < 0 || row_limit < 0)
    return set_error(FA_ERR_INVALID_ARG, "%s: bad sizes (batch=%d total=%d H=%d D=%d max_seqlen=%d)", fn,
                     batch, total, H, D, max_seqlen);
  if (D > 256) return set_error(FA_ERR_UNSUPPORTED, "%s: D=%d exceeds 256", fn, D);
  if (batch == 0 || total == 0) return FA_OK;
  if (!q || !k || !v || !o || !cu_seqlens) return set_error(FA_ERR_INVALID_ARG, "%s: null pointer", fn);
  PrefillParams p = {};
  p.q = static_cast<const half_t*>(q);
  p.k = static_cast<const half_t*>(k);
  p.v = static_cast<const half_t*>(v);
  p.o = static_cast<half_t*>(o);
  p.cu_seqlens = cu_seqlens;
  p.B = batch; p.H_Q = H; p.H_KV = H; p.N = 0; p.D = D; p.G = 1;
  p.total = total;
  p.row_limit = row_limit;
  p.causal = causal ? 1 : 0;
  p.scale_log2 = (1.0f / sqrtf(static_cast<float>(D))) * kLog2e;
  const bool vec = (D == 64 || D == 128 || D == 256) && aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o);
  // Rows past min(row_limit, total) are never computed, so the grid covers that many.
  const int rows_max = row_limit < total ? row_limit : total;
  return dispatch_prefill<true>(fn, D, vec, rows_max, p, static_cast<hipStream_t>(stream));
}
