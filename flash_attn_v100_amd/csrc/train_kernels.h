// Device kernels of the training path for gfx950: fp32 forward with
// log-sum-exp, and the attention backward (dQ, dK, dV) for fp16 and fp32 MHA,
// all on MFMA.  Instantiated by train.hip (fp16 backward and fp32 forward,
// accumulators in VGPRs) and train_fp32.hip (fp32 backward, accumulators in
// AGPRs).
//
// Every product is a 32x32 MFMA tile with a 16-deep reduction step: fp16 uses
// v_mfma_f32_32x32x16_f16 directly; fp32 issues the same tile as eight
// v_mfma_f32_32x32x2_f32 (lane half h contributes reduction index h of each,
// its 8 registers the 8 steps), so both element types share one operand
// layout and exact fp32 products stay fp32.  A 32x32x16 operand gives lane l
// the 8 reduction values k = 8 (l / 32) .. +8 of row/column l % 32; the 16
// accumulator registers r of lane l hold row 8 (r / 4) + 4 (l / 32) + r % 4 of
// column l % 32.
//
// Two kernel shapes, 4 waves per workgroup, 32 rows per wave:
//  * query-major (forward, dQ): each wave keeps its 32 query rows (Q, and dO
//    for dQ) in registers and walks 32-key K/V tiles staged in LDS.  S^T = K Q^T
//    puts one query per lane, so softmax statistics, log-sum-exp and delta are
//    per-lane scalars, and the S^T accumulator converted to operand form is
//    directly the B operand of O^T = V^T P^T (or dQ^T = K^T dS^T), whose A
//    operand is read transposed from LDS.
//  * key-major (dK, dV): each wave keeps its 32 keys (K, V) in registers and
//    walks 32-row Q/dO tiles staged in LDS with their log-sum-exp and delta.
//    S = Q K^T puts one key per lane, and dV^T = dO^T P and dK^T = Q^T dS take
//    P and dS straight from the accumulators.
// Inside each 16-deep slice of a 32-row operand taken from an accumulator,
// lane half h holds rows {4h..4h+3, 8+4h..8+4h+3}; the transposed LDS reads
// deliver the matching rows (ds_read_b64_tr_b16 for fp16: one read per 4-row
// run, 16 lanes each fetching 8 bytes of a 4 x 16 block; scalar reads for fp32).
//
// Tiles stream through LDS.  fp16 tiles use the prefill's XOR-swizzled,
// unpadded layout (both read patterns above are bank-conflict free); with
// D = 64 or 128 and aligned rows they are copied HBM -> LDS by
// global_load_lds (no register staging) through a two-stage ring, one tile
// ahead, one barrier per tile.  fp32 tiles and odd D stage through registers
// into a two-stage ring (fp32 rows padded by 32 bytes).
//
// The backward runs on one stream: dQ first (each wave also computes
// delta_i = sum_d dO[i,d] O[i,d] of its rows and publishes it in the
// workspace), then dK/dV, which reads delta.  The key-major kernel does both
// dK and dV in one pass when its registers allow (fp32, D <= 64 in fp16);
// otherwise (fp16, D > 64) one pass does dV (S and P only) and another dK
// (S, dP, dS), so each fits 256 VGPRs and two waves share a SIMD.  No atomics:
// every output element is written by exactly one lane, so results are
// deterministic.
#pragma once

#include <math.h>

#include "capi_internal.h"
#include "common.h"

namespace fa {
namespace train {

typedef float float8_t __attribute__((ext_vector_type(8)));

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kRows = 32;                   // rows per wave and per streamed tile
constexpr int kBlockRows = kWaves * kRows;  // rows per workgroup
constexpr float kLn2 = 0.69314718055994531f;

template <typename T>
struct Elem;
template <>
struct Elem<half_t> {
  typedef half8_t frag;
};
template <>
struct Elem<float> {
  typedef float8_t frag;
};

__device__ __forceinline__ float16_t mma(const half8_t& a, const half8_t& b, const float16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float16_t mma(const float8_t& a, const float8_t& b, float16_t c) {
#pragma unroll
  for (int j = 0; j < 8; ++j) c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[j], b[j], c, 0, 0, 0);
  return c;
}

template <typename T>
using lds_ptr = __attribute__((address_space(3))) T*;

// LDS tile layout for 32 rows of DP elements.  off(r, c) is the element offset
// of logical (row r, column c); columns move in 8-element groups (c % 8 is
// kept), so 16-byte row reads and 8-byte transposing reads stay contiguous.
template <typename T, int DP>
struct Layout;
template <int DP>
struct Layout<half_t, DP> {  // unpadded, 16-byte chunks XOR-swizzled per row
  static constexpr int TILE = kRows * DP;
  __device__ static __forceinline__ int off(int r, int c) {
    return r * DP + ((((c >> 3) ^ chunk_swizzle<DP>(r)) << 3) | (c & 7));
  }
};
template <int DP>
struct Layout<float, DP> {  // rows padded by 32 bytes (8 banks apart mod 64)
  static constexpr int LD = DP + 8;
  static constexpr int TILE = kRows * LD;
  __device__ static __forceinline__ int off(int r, int c) { return r * LD + c; }
};

// Per-lane LDS operand reads from a tile at LDS byte address `tile`:
//   row(tile, kk)     8 elements of row lane % 32, columns 16 kk + 8 (lane / 32) ..
//   tr(tile, r0, db)  element j = M[r0 + 8 (j / 4) + 4 (lane / 32) + j % 4][32 db + lane % 32]
// (r0 in {0, 16}).  The fp16 reader folds the swizzle into per-lane byte
// offsets once; each read then XORs in the compile-time part of its chunk
// index (tile bases are multiples of the row length, so they have no bits in
// the chunk field).
template <typename T, int DP>
struct Reader;
template <int DP>
struct Reader<half_t, DP> {
  unsigned row_lane, tr_lane;
  __device__ explicit Reader(int lane) {
    const int l32 = lane & 31, hi = lane >> 5, s16 = lane & 15;
    row_lane = static_cast<unsigned>((l32 * DP + ((chunk_swizzle<DP>(l32) ^ hi) * 8)) * 2);
    // source lane s16 of each 16-lane group reads row 4 hi + s16 / 4 (+ r0 + 8 jj),
    // columns 32 db + 16 ((lane >> 4) & 1) + 4 (s16 & 3) .. +4
    const int v_sw = (DP <= 64 ? (((s16 >> 3) & 1) << 2) : ((s16 >> 2) << 2)) | hi;
    const int v_row = 4 * hi + (s16 >> 2);
    tr_lane = static_cast<unsigned>(
        (v_row * DP + (((2 * ((lane >> 4) & 1) + ((s16 & 3) >> 1)) ^ v_sw) * 8) + (s16 & 1) * 4) * 2);
  }
  __device__ __forceinline__ half8_t row(unsigned tile, int kk) const {
    return *lds_at<half8_t>((tile + row_lane) ^ (32 * kk));
  }
  __device__ __forceinline__ half8_t tr(unsigned tile, int r0, int db) const {
    half4_t part[2];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const unsigned src = ((tile + tr_lane) ^ (16 * (4 * db ^ 2 * jj))) + (r0 + 8 * jj) * DP * 2;
      const short4_t x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          const_cast<__attribute__((address_space(3))) short4_t*>(lds_at<short4_t>(src)));
      part[jj] = __builtin_bit_cast(half4_t, x);
    }
    return __builtin_shufflevector(part[0], part[1], 0, 1, 2, 3, 4, 5, 6, 7);
  }
};
template <int DP>
struct Reader<float, DP> {
  int lane;
  __device__ explicit Reader(int lane_) : lane(lane_) {}
  __device__ __forceinline__ float8_t row(unsigned tile, int kk) const {
    const int off = Layout<float, DP>::off(lane & 31, 16 * kk + 8 * (lane >> 5));
    return *lds_at<float8_t>(tile + off * 4);
  }
  __device__ __forceinline__ float8_t tr(unsigned tile, int r0, int db) const {
    const int hi = lane >> 5;
    const int col = 32 * db + (lane & 31);
    const __attribute__((address_space(3))) float* t = lds_at<float>(tile);
    float8_t f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = t[Layout<float, DP>::off(r0 + 8 * (j >> 2) + 4 * hi + (j & 3), col)];
    return f;
  }
};

// Eight elements of global row `row` (length d) from column `col`, zero past d;
// VEC: d == padded width and 16-byte aligned rows, so one vector load serves.
template <typename T, bool VEC>
__device__ __forceinline__ typename Elem<T>::frag load_frag(const T* row, int col, int d) {
  typedef typename Elem<T>::frag F;
  if constexpr (VEC) {
    (void)d;
    return *reinterpret_cast<const F*>(row + col);
  } else {
    F f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = (col + j < d) ? row[col + j] : static_cast<T>(0.0f);
    return f;
  }
}

template <typename T>
__device__ __forceinline__ typename Elem<T>::frag zero_frag() {
  typename Elem<T>::frag f;
#pragma unroll
  for (int j = 0; j < 8; ++j) f[j] = static_cast<T>(0.0f);
  return f;
}

// Operand slice `sl` (accumulator registers 8 sl .. 8 sl + 7) converted to T.
template <typename T>
__device__ __forceinline__ typename Elem<T>::frag acc_frag(const float16_t& a, int sl) {
  typename Elem<T>::frag f;
#pragma unroll
  for (int j = 0; j < 8; ++j) f[j] = static_cast<T>(a[8 * sl + j]);
  return f;
}

// Streams 32-row tiles of two [N, D] row-major tensors (and, with VECS, two
// per-row float vectors) through an LDS ring.  A stage holds
//   [tensor A tile | tensor B tile | VECS: 64 floats of vector 0 | 64 of vector 1]
// (only the first 32 floats of each vector slot are used).
//  DMA (fp16, D = DP, 16-byte aligned rows): stages filled by global_load_lds,
//    one tile ahead; rows past `rows` re-read the last row (callers mask them).
//  otherwise: stages filled through registers; rows past `rows` are 0
//    and vector 0 / vector 1 read +inf / 0 there.
// Vector 0 is stored pre-multiplied by log2(e) on the register path only; DMA
// consumers scale at the read (vec_scale()).
template <typename T, int DP, bool DMA, bool VECS>
struct TileRing {
  typedef typename Elem<T>::frag F;
  typedef Layout<T, DP> L;
  static constexpr int NS = 2;  // three DMA stages measured 4.7 % slower (config 7 backward 367 vs 350 us)
  static constexpr int VEC_FLOATS = VECS ? 128 : 0;
  static constexpr int STAGE_BYTES = 2 * L::TILE * static_cast<int>(sizeof(T)) + VEC_FLOATS * 4;
  static constexpr int BYTES = NS * STAGE_BYTES;
  static constexpr int CPR = DP / 8;            // 8-element groups per row
  static constexpr int CHUNKS = kRows * CPR;    // groups per tile
  static constexpr int PER_THREAD = (CHUNKS + kThreads - 1) / kThreads;
  // DMA instructions this wave issues per tile (waves 0 and 1 also copy a vector)
  static constexpr int DMA_PER_TILE = 2 * PER_THREAD;

  unsigned lds_base;  // byte address of stage 0
  int tid, lane, wave;
  // register path staging
  F a[DMA ? 1 : PER_THREAD], b[DMA ? 1 : PER_THREAD];
  float v0 = 0.0f, v1 = 0.0f;
  // DMA path: per copy, the tile row and byte offset of this lane's chunk
  int cp_row[PER_THREAD];
  unsigned cp_off[PER_THREAD];

  __device__ TileRing(void* smem, int tid_, int d)
      : tid(tid_), lane(tid_ & 63), wave(__builtin_amdgcn_readfirstlane(tid_ >> 6)) {
    lds_base = static_cast<unsigned>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char*)smem));
    if constexpr (DMA) {
      static_assert(sizeof(T) == 2 && CHUNKS % kThreads == 0, "DMA tiles are whole fp16 chunks per thread");
#pragma unroll
      for (int i = 0; i < PER_THREAD; ++i) {
        // slot g (16-byte LDS chunk) = i * 256 + tid holds logical chunk
        // (g % CPR) ^ swizzle(row) of row g / CPR
        const int g = i * kThreads + tid;
        cp_row[i] = g / CPR;
        const int lc = (g % CPR) ^ chunk_swizzle<DP>(g / CPR);
        cp_off[i] = static_cast<unsigned>((cp_row[i] * d + lc * 8) * 2);
      }
    }
  }
  __device__ __forceinline__ unsigned addr_a(int stage) const { return lds_base + stage * STAGE_BYTES; }
  __device__ __forceinline__ unsigned addr_b(int stage) const { return addr_a(stage) + L::TILE * sizeof(T); }
  __device__ __forceinline__ lds_ptr<T> tile_a(int stage) const {
    return reinterpret_cast<lds_ptr<T>>(static_cast<size_t>(lds_base + stage * STAGE_BYTES));
  }
  __device__ __forceinline__ lds_ptr<T> tile_b(int stage) const { return tile_a(stage) + L::TILE; }
  __device__ __forceinline__ const __attribute__((address_space(3))) float* vec(int stage, int which) const {
    return reinterpret_cast<const __attribute__((address_space(3))) float*>(
        static_cast<size_t>(lds_base + stage * STAGE_BYTES + 2 * L::TILE * sizeof(T) + which * 256));
  }

  // DMA path: copy rows [r0, r0 + 32) of pa/pb (row stride d == DP) and, with
  // VECS, va/vb[r0 .. r0 + 32) into `stage`.
  __device__ __forceinline__ void dma(const T* pa, const T* pb, const float* va, const float* vb, int r0, int rows,
                                      int d, int stage) const {
    const T* ba = pa + static_cast<size_t>(r0) * d;
    const T* bb = pb + static_cast<size_t>(r0) * d;
    const unsigned sbase = lds_base + stage * STAGE_BYTES;
    const bool tail = r0 + kRows > rows;
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      unsigned off = cp_off[i];
      if (tail) {
        const int row = min(cp_row[i], rows - 1 - r0);
        off = static_cast<unsigned>(static_cast<int>(off) + (row - cp_row[i]) * d * 2);
      }
      const unsigned slot = sbase + (i * kThreads + wave * 64) * 16;
      copy16_to_lds(reinterpret_cast<const half_t*>(ba), off, slot);
      copy16_to_lds(reinterpret_cast<const half_t*>(bb), off, slot + L::TILE * sizeof(T));
    }
    if constexpr (VECS) {
      if (wave < 2) {
        const float* base = (wave == 0 ? va : vb) + r0;
        const unsigned off = static_cast<unsigned>(min(lane & 31, rows - 1 - r0)) * 4;
        copy4_to_lds(base, off, sbase + 2 * L::TILE * sizeof(T) + wave * 256);
      }
    }
  }
  // Waits until this wave's copies of every tile but the newest `pending` ones
  // have landed (DMA path).
  __device__ __forceinline__ void wait_dma(bool one_pending) const {
    const bool extra = VECS && wave < 2;
    if (one_pending) {
      if (extra) wait_vm_lgkm0<DMA_PER_TILE + 1>();
      else wait_vm_lgkm0<DMA_PER_TILE>();
    } else {
      wait_vm_lgkm0<0>();
    }
  }

  // Register path: load rows [r0, r0 + 32) (zero past `rows`) into registers ...
  template <bool VEC>
  __device__ __forceinline__ void load(const T* pa, const T* pb, const float* va, const float* vb, int r0, int rows,
                                       int d) {
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      const int c = tid + i * kThreads;
      const int row = c / CPR;
      const int col = (c % CPR) * 8;
      if ((CHUNKS % kThreads == 0 || c < CHUNKS) && r0 + row < rows) {
        a[i] = load_frag<T, VEC>(pa + static_cast<size_t>(r0 + row) * d, col, d);
        b[i] = load_frag<T, VEC>(pb + static_cast<size_t>(r0 + row) * d, col, d);
      } else {
        a[i] = zero_frag<T>();
        b[i] = zero_frag<T>();
      }
    }
    if constexpr (VECS) {
      if (tid < kRows) {
        const int r = r0 + tid;
        v0 = r < rows ? va[r] * kLog2e : INFINITY;  // padding rows: P = 0
        v1 = r < rows ? vb[r] : 0.0f;
      }
    }
  }
  // ... and store them into `stage`.
  __device__ __forceinline__ void store(int stage) const {
    lds_ptr<T> ta = tile_a(stage);
    lds_ptr<T> tb = tile_b(stage);
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      const int c = tid + i * kThreads;
      if (CHUNKS % kThreads == 0 || c < CHUNKS) {
        const int row = c / CPR;
        const int col = (c % CPR) * 8;
        *reinterpret_cast<__attribute__((address_space(3))) F*>(ta + L::off(row, col)) = a[i];
        *reinterpret_cast<__attribute__((address_space(3))) F*>(tb + L::off(row, col)) = b[i];
      }
    }
    if constexpr (VECS) {
      if (tid < kRows) {
        auto* v = const_cast<__attribute__((address_space(3))) float*>(vec(stage, 0));
        v[tid] = v0;
        v[64 + tid] = v1;
      }
    }
  }
};

// The fp16 key-major passes walk their query tiles last to first (0: first
// to last): the 128-key blocks of one (batch, head) run together on one XCD
// and all end at the last query tile, so walking backwards they read each Q /
// dO tile at about the same time and share it through L2.
#ifndef FA_BWD_REV
#define FA_BWD_REV 1
#endif
#ifndef FA_BWD_GROUP
#define FA_BWD_GROUP 4
#endif

struct TrainParams {
  const void* q;
  const void* k;
  const void* v;
  const void* o;     // backward: forward output
  const void* dout;  // backward
  void* out;         // forward: O; dQ kernel: dQ
  void* dk;
  void* dv;
  float* lse;        // forward: written if non-null; backward: read
  float* delta;      // backward workspace [B*H*N]
  int delta_ready;   // dQ kernel: delta is already in the workspace (read it, do not recompute)
  int BH, N, D, causal;
  int nblk;          // 128-row blocks per (batch, head)
  float scale;       // 1/sqrt(D)
  float scale_log2;  // scale * log2(e)
};

// Causal calls deal an XCD's units in groups of kBwdGroupUnits, each group's
// blocks interleaved heaviest first across its units (the 128-row blocks of
// a causal unit range from 1 to N/128 tiles of work, so one unit at a time
// left the lightest blocks of every unit trailing): config 7 350 -> 320 us,
// 16 x 16 heads x 512 keys 171 -> 148 us; groups of 2 and 8 measured close;
// non-causal calls (equal blocks) keep one unit at a time.
constexpr int kBwdGroupUnits = FA_BWD_GROUP;
__host__ __device__ inline int bwd_group_units(const TrainParams& p) { return p.causal ? kBwdGroupUnits : 1; }

// Workgroup -> ((batch, head) unit bh, 128-row block blk).  With at least 8
// units, every block of a unit runs on one XCD (the dispatcher deals workgroup
// j to XCD j % 8), so the unit's streamed tiles are shared through that XCD's
// L2, and an XCD walks its units group by group, heaviest block first
// (heavy_last: the last block carries the most work).  Returns false for the
// padding workgroups of the last round.
__device__ __forceinline__ bool map_block(const TrainParams& p, bool heavy_last, int& bh, int& blk) {
  const int j = blockIdx.x;
  const int nb = p.nblk;
  int b;
  if (p.BH >= 8) {
    const int i = j / 8;
    const int gu = bwd_group_units(p);
    const int group = i / (gu * nb), ii = i % (gu * nb);
    bh = j % 8 + 8 * (group * gu + ii % gu);
    b = ii / gu;
    if (bh >= p.BH) return false;
  } else {
    bh = j / nb;
    b = j % nb;
  }
  blk = heavy_last ? nb - 1 - b : b;
  return true;
}

inline int train_grid(const TrainParams& p) {
  const int gu = bwd_group_units(p);
  return p.BH >= 8 ? 8 * ceil_div(ceil_div(p.BH, 8), gu) * gu * p.nblk : p.BH * p.nblk;
}

// Drives a TileRing over `ntiles` tiles starting at row r_first and calls
// compute(stage, tile) for the tiles [c_begin, c_end) of this wave (every wave
// copies and joins the barriers of all tiles).  The three tile ranges are
// separate loops so that the accumulating loop carries no per-tile branch
// around the MFMAs (which would make the compiler copy the accumulators).
// REV walks the tiles last to first (`tile` passed to compute is still the
// tile's index from r_first): workgroups that share a stream but start at
// different tiles and end together then read each tile at about the same
// time, so the copies after the first hit L2.
template <typename Ring, bool DMA, bool VEC, bool REV = false, typename T, typename Compute>
__device__ __forceinline__ void run_ring(Ring& ring, const T* pa, const T* pb, const float* va, const float* vb,
                                         int r_first, int ntiles, int c_begin, int c_end, int rows, int d,
                                         Compute&& compute) {
  c_begin = max(0, min(c_begin, ntiles));
  c_end = max(c_begin, min(c_end, ntiles));
  if constexpr (REV) {
    const int b = ntiles - c_end;
    c_end = ntiles - c_begin;
    c_begin = b;
  }
  auto tile_of = [&](int t) { return REV ? ntiles - 1 - t : t; };  // stream position -> tile
  auto row_of = [&](int t) { return r_first + tile_of(t) * kRows; };
  if constexpr (DMA) {
    constexpr int NS = Ring::NS;
#pragma unroll
    for (int s = 0; s < NS - 1; ++s)
      if (s < ntiles) ring.dma(pa, pb, va, vb, row_of(s), rows, d, s);
    auto step = [&](int t) {
      ring.wait_dma(NS > 2 && t + 1 < ntiles);  // this wave's copies of tile t landed (tile t + 1 may be in flight)
      tile_barrier();                  // everyone's did; stage (t - 1) % NS is free
      if (t + NS - 1 < ntiles) ring.dma(pa, pb, va, vb, row_of(t + NS - 1), rows, d, (t + NS - 1) % NS);
    };
    for (int t = 0; t < c_begin; ++t) step(t);
    for (int t = c_begin; t < c_end; ++t) {
      step(t);
      compute(t % NS, tile_of(t));
    }
    for (int t = c_end; t < ntiles; ++t) step(t);
  } else {
    if (ntiles > 0) {
      ring.template load<VEC>(pa, pb, va, vb, row_of(0), rows, d);
      ring.store(0);
    }
    auto pre = [&](int t) {
      if (t + 1 < ntiles) ring.template load<VEC>(pa, pb, va, vb, row_of(t + 1), rows, d);
      __syncthreads();
    };
    auto post = [&](int t) {
      if (t + 1 < ntiles) ring.store((t + 1) & 1);
    };
    for (int t = 0; t < c_begin; ++t) {
      pre(t);
      post(t);
    }
    for (int t = c_begin; t < c_end; ++t) {
      pre(t);
      compute(t & 1, tile_of(t));
      post(t);
    }
    for (int t = c_end; t < ntiles; ++t) {
      pre(t);
      post(t);
    }
  }
}

// ---------------------------------------------------------------------------
// Query-major kernel: MODE 0 = fp32 forward (O, optional LSE), MODE 1 = dQ + delta.
template <typename T, int DP, bool VEC, int MODE>
__global__ __launch_bounds__(kThreads) void query_major_kernel(TrainParams p) {
  typedef typename Elem<T>::frag F;
  constexpr int KK = DP / 16;  // 16-deep reduction steps over d
  constexpr int DB = DP / 32;  // 32-row blocks of d in the transposed products
  constexpr bool DMA = VEC && sizeof(T) == 2;
  typedef TileRing<T, DP, DMA, false> Ring;
  __shared__ __attribute__((aligned(1024))) char smem[Ring::BYTES];

  const int N = p.N, D = p.D;
  int bh, blk;
  if (!map_block(p, p.causal != 0, bh, blk)) return;
  const int q0 = blk * kBlockRows;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  const int wq0 = q0 + wave * kRows;
  const int qrow = wq0 + l32;
  const bool qvalid = qrow < N;
  const size_t base = static_cast<size_t>(bh) * N * D;
  const T* __restrict__ qp = static_cast<const T*>(p.q) + base;
  const T* __restrict__ kp = static_cast<const T*>(p.k) + base;
  const T* __restrict__ vp = static_cast<const T*>(p.v) + base;

  // resident B operands: lane's query row, d = 16 kk + 8 hi .. +8
  F qf[KK], df[KK];
  float delta = 0.0f, lse2 = 0.0f;
  {
    const T* qr = qp + static_cast<size_t>(min(qrow, N - 1)) * D;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qf[kk] = qvalid ? load_frag<T, VEC>(qr, 16 * kk + 8 * hi, D) : zero_frag<T>();
  }
  if constexpr (MODE == 1) {
    const T* dr = static_cast<const T*>(p.dout) + base + static_cast<size_t>(min(qrow, N - 1)) * D;
    const T* orow = static_cast<const T*>(p.o) + base + static_cast<size_t>(min(qrow, N - 1)) * D;
    float part = 0.0f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      df[kk] = qvalid ? load_frag<T, VEC>(dr, 16 * kk + 8 * hi, D) : zero_frag<T>();
      if (!p.delta_ready) {
        const F of = qvalid ? load_frag<T, VEC>(orow, 16 * kk + 8 * hi, D) : zero_frag<T>();
#pragma unroll
        for (int j = 0; j < 8; ++j) part = fmaf(static_cast<float>(df[kk][j]), static_cast<float>(of[j]), part);
      }
    }
    delta = part + __shfl_xor(part, 32, 64);
    if (qvalid) {
      if (p.delta_ready) delta = p.delta[static_cast<size_t>(bh) * N + qrow];  // the same value, from delta_kernel
      else if (hi == 0) p.delta[static_cast<size_t>(bh) * N + qrow] = delta;
      lse2 = p.lse[static_cast<size_t>(bh) * N + qrow] * kLog2e;
    } else {
      lse2 = INFINITY;  // padding rows: P = 0
    }
  }

  float16_t acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.0f;
  float m_run = kNegBig, l_run = 0.0f;  // forward only (log2 domain)
  const float c = p.scale_log2;

  const int kend = p.causal ? min(N, q0 + kBlockRows) : N;  // keys this workgroup needs
  // keys this wave needs (none when all its rows lie past N)
  const int kend_w = wq0 >= N ? 0 : (p.causal ? min(N, wq0 + kRows) : N);
  const int ntiles = (kend + kRows - 1) / kRows;

  Ring ring(smem, tid, D);
  const Reader<T, DP> rd(lane);
  // this wave computes key tiles [0, ceil(kend_w / 32)): later ones are past its diagonal
  run_ring<Ring, DMA, VEC>(ring, kp, vp, nullptr, nullptr, 0, ntiles, 0, (kend_w + kRows - 1) / kRows, N, D,
                           [&](int stage, int t) {
    const int kt = t * kRows;
    const unsigned ks = ring.addr_a(stage);
    const unsigned vs = ring.addr_b(stage);
    // S^T = K Q^T: lane <-> query, register r <-> key kt + 8 (r/4) + 4 hi + r%4
    float16_t s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) s = mma(rd.row(ks, kk), qf[kk], s);
    const bool masked = (kt + kRows > N) || (p.causal && kt + kRows - 1 > wq0);
    if (masked) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kt + 8 * (r >> 2) + 4 * hi + (r & 3);
        if (key >= N || (p.causal && key > qrow)) s[r] = -INFINITY;
      }
    }
    float16_t pm;  // P^T (forward) or dS^T (dQ)
    if constexpr (MODE == 0) {
      float mx = s[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * c;
      const float mn = fmaxf(m_run, mx);
      const float alpha = fast_exp2(m_run - mn);
      m_run = mn;
      float ls = 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        pm[r] = fast_exp2(fmaf(s[r], c, -mn));
        ls += pm[r];
      }
      l_run = fmaf(l_run, alpha, ls);
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;
    } else {
      // dP^T = V dO^T
      float16_t dp;
#pragma unroll
      for (int r = 0; r < 16; ++r) dp[r] = 0.0f;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) dp = mma(rd.row(vs, kk), df[kk], dp);
#pragma unroll
      for (int r = 0; r < 16; ++r) pm[r] = fast_exp2(fmaf(s[r], c, -lse2)) * (dp[r] - delta);
    }
    const F pf0 = acc_frag<T>(pm, 0), pf1 = acc_frag<T>(pm, 1);
    // forward: O^T += V^T P^T;  dQ: dQ^T += K^T dS^T
    const unsigned src = (MODE == 0) ? vs : ks;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      acc[db] = mma(rd.tr(src, 0, db), pf0, acc[db]);
      acc[db] = mma(rd.tr(src, 16, db), pf1, acc[db]);
    }
  });

  // ---- store: lane's row, d = 32 db + 8 (r/4) + 4 hi + r%4 ----
  float mul;
  if constexpr (MODE == 0) {
    const float lt = l_run + __shfl_xor(l_run, 32, 64);
    mul = 1.0f / lt;
    if (p.lse != nullptr && qvalid && hi == 0) p.lse[static_cast<size_t>(bh) * N + qrow] = (m_run + log2f(lt)) * kLn2;
  } else {
    mul = p.scale;
  }
  if (!qvalid) return;
  T* op = static_cast<T*>(p.out) + base + static_cast<size_t>(qrow) * D;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int d0 = 32 * db + 8 * rr + 4 * hi;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (VEC || d0 + j < D) op[d0 + j] = static_cast<T>(acc[db][4 * rr + j] * mul);
    }
}

// ---------------------------------------------------------------------------
// Key-major kernel for 32 keys per wave: PASS 0 = dV, 1 = dK, 2 = both.
constexpr int kPassDV = 0, kPassDK = 1, kPassBoth = 2;
template <typename T, int DP, bool VEC, int PASS>
__global__ __launch_bounds__(kThreads) void dkdv_kernel(TrainParams p) {
  constexpr bool DO_DV = PASS != kPassDK;
  constexpr bool DO_DK = PASS != kPassDV;
  typedef typename Elem<T>::frag F;
  constexpr int KK = DP / 16;
  constexpr int DB = DP / 32;
  constexpr bool DMA = VEC && sizeof(T) == 2;
  typedef TileRing<T, DP, DMA, true> Ring;
  __shared__ __attribute__((aligned(1024))) char smem[Ring::BYTES];

  const int N = p.N, D = p.D;
  int bh, blk;
  if (!map_block(p, false, bh, blk)) return;
  const int k0 = blk * kBlockRows;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  const int wk0 = k0 + wave * kRows;
  const int krow = wk0 + l32;
  const bool kvalid = krow < N;
  const size_t base = static_cast<size_t>(bh) * N * D;
  const T* __restrict__ qp = static_cast<const T*>(p.q) + base;
  const T* __restrict__ dop = static_cast<const T*>(p.dout) + base;
  const float* __restrict__ lse = p.lse + static_cast<size_t>(bh) * N;
  const float* __restrict__ dlt = p.delta + static_cast<size_t>(bh) * N;

  F kf[KK], vf[KK];
  {
    const T* kr = static_cast<const T*>(p.k) + base + static_cast<size_t>(min(krow, N - 1)) * D;
    const T* vr = static_cast<const T*>(p.v) + base + static_cast<size_t>(min(krow, N - 1)) * D;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      kf[kk] = kvalid ? load_frag<T, VEC>(kr, 16 * kk + 8 * hi, D) : zero_frag<T>();
      if constexpr (DO_DK) vf[kk] = kvalid ? load_frag<T, VEC>(vr, 16 * kk + 8 * hi, D) : zero_frag<T>();
    }
  }
  float16_t dk[DB], dv[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      dk[db][r] = 0.0f;
      dv[db][r] = 0.0f;
    }
  const float c = p.scale_log2;

  // query tiles this workgroup needs: causal skips rows before its first key
  const int qstart = p.causal ? k0 : 0;
  const int ntiles = (N - qstart + kRows - 1) / kRows;

  Ring ring(smem, tid, D);
  const Reader<T, DP> rd(lane);
  // a tile whose last query precedes this wave's first key contributes nothing:
  // causal waves start at the tile holding query wk0
  const int c_begin = wk0 >= N ? ntiles : (p.causal ? (wk0 - qstart) / kRows : 0);  // no keys: no compute
  // (the register-staged fp32 pass measured no gain from it)
  // The dV pass never reads delta, and runs concurrently with the kernel that
  // writes it: its second per-row stream is pointed at lse instead (staged,
  // never used), so it touches nothing that kernel writes.
  const float* __restrict__ vb_rows = DO_DK ? dlt : lse;
  run_ring<Ring, DMA, VEC, FA_BWD_REV != 0 && DMA>(ring, qp, dop, lse, vb_rows, qstart, ntiles, c_begin, ntiles, N, D, [&](int stage, int t) {
    const int qt = qstart + t * kRows;
    const unsigned qs = ring.addr_a(stage);
    const unsigned ds = ring.addr_b(stage);
    // S = Q K^T and dP = dO V^T: lane <-> key, register r <-> query qt + 8 (r/4) + 4 hi + r%4
    float16_t s, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = 0.0f;
      dp[r] = 0.0f;
    }
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      s = mma(rd.row(qs, kk), kf[kk], s);
      if constexpr (DO_DK) dp = mma(rd.row(ds, kk), vf[kk], dp);
    }
    // query qi = qt + 8 (r/4) + 4 hi + r%4 contributes iff qi >= krow (causal) and qi < N;
    // with lo = qi - krow and hi_lim = N - qi, both are tests on (8 (r/4) + r%4)
    const bool tail = qt + kRows > N;
    const bool diag = p.causal && qt < wk0 + kRows - 1;
    const int lo = diag ? qt + 4 * hi - krow : 0;
    const int lim = tail ? N - qt - 4 * hi : kRows;
    const __attribute__((address_space(3))) float* lv = ring.vec(stage, 0);
    const __attribute__((address_space(3))) float* dvv = ring.vec(stage, 1);
    const float lmul = DMA ? kLog2e : 1.0f;  // the register path stores lse pre-scaled
    const bool need_mask = tail || diag;  // wave-uniform: diagonal or last tile only
    float16_t pm, dsm;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const float4_t l4 = *reinterpret_cast<const __attribute__((address_space(3))) float4_t*>(lv + 8 * rr + 4 * hi);
      float4_t d4;
      if constexpr (DO_DK) d4 = *reinterpret_cast<const __attribute__((address_space(3))) float4_t*>(dvv + 8 * rr + 4 * hi);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 4 * rr + j;
        pm[r] = fast_exp2(fmaf(s[r], c, -l4[j] * lmul));
        if constexpr (DO_DK) dsm[r] = dp[r] - d4[j];
      }
    }
    if (need_mask) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int rel = 8 * (r >> 2) + (r & 3);
        pm[r] = (rel + lo >= 0 && rel < lim) ? pm[r] : 0.0f;
      }
    }
    if constexpr (DO_DK) {
#pragma unroll
      for (int r = 0; r < 16; ++r) dsm[r] *= pm[r];
    }
    if constexpr (DO_DV) {
      const F pf0 = acc_frag<T>(pm, 0), pf1 = acc_frag<T>(pm, 1);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        dv[db] = mma(rd.tr(ds, 0, db), pf0, dv[db]);
        dv[db] = mma(rd.tr(ds, 16, db), pf1, dv[db]);
      }
    }
    if constexpr (DO_DK) {
      const F sf0 = acc_frag<T>(dsm, 0), sf1 = acc_frag<T>(dsm, 1);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        dk[db] = mma(rd.tr(qs, 0, db), sf0, dk[db]);
        dk[db] = mma(rd.tr(qs, 16, db), sf1, dk[db]);
      }
    }
  });

  if (!kvalid) return;
  T* dkp = static_cast<T*>(p.dk) + base + static_cast<size_t>(krow) * D;
  T* dvp = static_cast<T*>(p.dv) + base + static_cast<size_t>(krow) * D;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int d0 = 32 * db + 8 * rr + 4 * hi;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (VEC || d0 + j < D) {
          if constexpr (DO_DK) dkp[d0 + j] = static_cast<T>(dk[db][4 * rr + j] * p.scale);
          if constexpr (DO_DV) dvp[d0 + j] = static_cast<T>(dv[db][4 * rr + j]);
        }
    }
}

// delta_i = sum_d dO[i,d] O[i,d] for every row, into the workspace, with the
// query-major kernel's exact arithmetic: two fma chains per row, over
// d = 16 kk + 8 h + j (h = 0, 1; kk = 0 .. DP/16 - 1; j = 0 .. 7; zero past D),
// then their sum.  Two threads per row.
template <typename T, int DP, bool VEC>
__global__ __launch_bounds__(256) void delta_kernel(TrainParams p) {
  typedef typename Elem<T>::frag F;
  const long long t = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  const long long rows = static_cast<long long>(p.BH) * p.N;
  const long long row = min(t >> 1, rows - 1);  // (rows past the end redo the last row, written once)
  const int h = static_cast<int>(t & 1);
  const T* dr = static_cast<const T*>(p.dout) + row * p.D;
  const T* orow = static_cast<const T*>(p.o) + row * p.D;
  float part = 0.0f;
#pragma unroll
  for (int kk = 0; kk < DP / 16; ++kk) {
    const F df = load_frag<T, VEC>(dr, 16 * kk + 8 * h, p.D);
    const F of = load_frag<T, VEC>(orow, 16 * kk + 8 * h, p.D);
#pragma unroll
    for (int j = 0; j < 8; ++j) part = fmaf(static_cast<float>(df[j]), static_cast<float>(of[j]), part);
  }
  const float delta = part + __shfl_xor(part, 1, 64);
  if (h == 0 && (t >> 1) < rows) p.delta[row] = delta;
}

// ---------------------------------------------------------------------------
// Launch helpers (the backward is instantiated per element type by train.hip
// and train_fp32.hip; the fp32 forward, which fits 256 VGPRs, by train.hip).

// Non-blocking, default-priority streams (which = 0, 1) of the current
// device for the concurrent passes of a backward issued on `caller`: one pair
// per caller stream (created on first use, kept for the process; nullptr if
// one cannot be created).  Defined in train.hip.
hipStream_t backward_side_stream(hipStream_t caller, int which);
// The calling thread's four fork/join events for the current device (created
// once, reused by every later backward call of that thread); false if they
// cannot be made.
bool backward_events(hipEvent_t (&ev)[4]);

template <typename T, int DP, bool VEC>
void launch_backward_dp(const TrainParams& p, hipStream_t st) {
  const dim3 grid(train_grid(p));
  // fp16 at D > 64 splits dV and dK into two passes to fit 256 VGPRs
#ifndef FA_BWD_SPLIT_DKDV
#define FA_BWD_SPLIT_DKDV 1
#endif
  constexpr bool kSplit = FA_BWD_SPLIT_DKDV && sizeof(T) == 2 && DP > 64;
  {
    // Concurrent streams: delta (a short kernel) then dQ on `st`; the dK/dV
    // pass (or the dK pass) on a side stream once delta is there; with split
    // passes, the dV pass, which needs neither, on another side stream from
    // the start.  Everything joins back into `st`.  Each kernel leaves most
    // of the MFMA pipe idle on its own.  (Not while `st` is being captured
    // into a graph: the capture then keeps the launches in order on `st`.)
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    const bool capturing = hipStreamIsCapturing(st, &capture) != hipSuccess || capture != hipStreamCaptureStatusNone;
    hipStream_t side_v = capturing || !kSplit ? nullptr : backward_side_stream(st, 0);
    hipStream_t side_k = capturing ? nullptr : backward_side_stream(st, 1);
    hipEvent_t ev[4] = {};  // fork, delta ready, dV done, dK(/dV) done
    bool ok = side_k != nullptr && (!kSplit || side_v != nullptr) && backward_events(ev);
    if (kSplit)
      ok = ok && hipEventRecord(ev[0], st) == hipSuccess && hipStreamWaitEvent(side_v, ev[0], 0) == hipSuccess;
    if (ok) {
      bool v_joined = true;
      if constexpr (kSplit) {
        hipLaunchKernelGGL((dkdv_kernel<T, DP, VEC, kPassDV>), grid, dim3(kThreads), 0, side_v, p);
        v_joined = hipEventRecord(ev[2], side_v) == hipSuccess;
      }
      const long long rows = static_cast<long long>(p.BH) * p.N;
      hipLaunchKernelGGL((delta_kernel<T, DP, VEC>), dim3(static_cast<unsigned>((2 * rows + 255) / 256)), dim3(256), 0,
                         st, p);
      TrainParams pq = p;
      pq.delta_ready = 1;
      const bool k_forked = hipEventRecord(ev[1], st) == hipSuccess && hipStreamWaitEvent(side_k, ev[1], 0) == hipSuccess;
      hipLaunchKernelGGL((query_major_kernel<T, DP, VEC, 1>), grid, dim3(kThreads), 0, st, pq);
      hipStream_t sk = k_forked ? side_k : st;
      if constexpr (kSplit)
        hipLaunchKernelGGL((dkdv_kernel<T, DP, VEC, kPassDK>), grid, dim3(kThreads), 0, sk, p);
      else
        hipLaunchKernelGGL((dkdv_kernel<T, DP, VEC, kPassBoth>), grid, dim3(kThreads), 0, sk, p);
      // joins; should one fail, wait for that stream on the host instead
      if (k_forked && (hipEventRecord(ev[3], side_k) != hipSuccess || hipStreamWaitEvent(st, ev[3], 0) != hipSuccess))
        (void)hipStreamSynchronize(side_k);
      if (kSplit && (!v_joined || hipStreamWaitEvent(st, ev[2], 0) != hipSuccess)) (void)hipStreamSynchronize(side_v);
      return;
    }
    (void)hipGetLastError();  // a failed fork leaves no error behind: run in order below
  }
  hipLaunchKernelGGL((query_major_kernel<T, DP, VEC, 1>), grid, dim3(kThreads), 0, st, p);
  if constexpr (kSplit) {
    hipLaunchKernelGGL((dkdv_kernel<T, DP, VEC, kPassDV>), grid, dim3(kThreads), 0, st, p);
    hipLaunchKernelGGL((dkdv_kernel<T, DP, VEC, kPassDK>), grid, dim3(kThreads), 0, st, p);
  } else {
    hipLaunchKernelGGL((dkdv_kernel<T, DP, VEC, kPassBoth>), grid, dim3(kThreads), 0, st, p);
  }
}

// dQ (+ delta) then dK/dV for any 1 <= D <= 128.  fp16 tiles need DP >= 64
// (the swizzle covers 8 or 16 chunks per row), so D <= 64 runs at DP = 64.
template <typename T>
void launch_backward(const TrainParams& p, bool vec_ok, hipStream_t st) {
  const int D = p.D;
  if constexpr (sizeof(T) == 4) {
    if (D <= 32) {
      vec_ok && D == 32 ? launch_backward_dp<T, 32, true>(p, st) : launch_backward_dp<T, 32, false>(p, st);
      return;
    }
  }
  if (D <= 64) {
    vec_ok && D == 64 ? launch_backward_dp<T, 64, true>(p, st) : launch_backward_dp<T, 64, false>(p, st);
  } else {
    vec_ok && D == 128 ? launch_backward_dp<T, 128, true>(p, st) : launch_backward_dp<T, 128, false>(p, st);
  }
}

// fp32 forward (O and optional log-sum-exp) for any 1 <= D <= 128.
inline void launch_forward_fp32(const TrainParams& p, bool vec_ok, hipStream_t st) {
  const int D = p.D;
  const dim3 grid(train_grid(p));
  if (D <= 32) {
    if (vec_ok && D == 32) hipLaunchKernelGGL((query_major_kernel<float, 32, true, 0>), grid, dim3(kThreads), 0, st, p);
    else hipLaunchKernelGGL((query_major_kernel<float, 32, false, 0>), grid, dim3(kThreads), 0, st, p);
  } else if (D <= 64) {
    if (vec_ok && D == 64) hipLaunchKernelGGL((query_major_kernel<float, 64, true, 0>), grid, dim3(kThreads), 0, st, p);
    else hipLaunchKernelGGL((query_major_kernel<float, 64, false, 0>), grid, dim3(kThreads), 0, st, p);
  } else {
    if (vec_ok && D == 128) hipLaunchKernelGGL((query_major_kernel<float, 128, true, 0>), grid, dim3(kThreads), 0, st, p);
    else hipLaunchKernelGGL((query_major_kernel<float, 128, false, 0>), grid, dim3(kThreads), 0, st, p);
  }
}

// Entry point of the fp32 backward translation unit (train_fp32.hip).
void backward_fp32(const TrainParams& p, bool vec_ok, hipStream_t st);

}  // namespace train
}  // namespace fa
