// Training path for gfx950: fp32 forward with log-sum-exp, and the attention
// backward (dQ, dK, dV) for fp16 and fp32 MHA, all on MFMA.
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
// The backward runs as two launches on one stream: dQ first (each wave also
// computes delta_i = sum_d dO[i,d] O[i,d] of its rows and publishes it in the
// workspace), then dK/dV, which reads delta.  No atomics: every output element
// is written by exactly one lane, so results are deterministic.
// The MFMA accumulators of the backward live in AGPRs (this file is built
// without the VGPR-form option): they are only ever accumulated and stored.
#include <math.h>

#include "capi_internal.h"
#include "common.h"

namespace fa {
namespace train {

typedef float float8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kRows = 32;                 // rows per wave and per streamed tile
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

// LDS tiles are row-major with a 32-byte pad per row: rows are 8 banks apart
// (mod 64), which keeps both the 16-byte row reads and the 4 x 16 transposing
// reads free of bank conflicts within each group of lanes served together.
template <typename T, int DP>
struct Tile {
  static constexpr int LD = DP + 32 / static_cast<int>(sizeof(T));  // row stride, elements
  static constexpr int ELEMS = kRows * LD;
};

template <typename T>
using lds_ptr = __attribute__((address_space(3))) T*;

template <typename T>
__device__ __forceinline__ typename Elem<T>::frag lds_row_frag(const lds_ptr<T> tile, int ld, int row, int col) {
  return *reinterpret_cast<const __attribute__((address_space(3))) typename Elem<T>::frag*>(tile + row * ld + col);
}

// Operand element j = M[r0 + 8 (j / 4) + 4 hi + j % 4][c0 + lane % 32] of an LDS tile.
__device__ __forceinline__ half8_t lds_tr_frag(const lds_ptr<half_t> tile, int ld, int r0, int c0, int lane) {
  const int s16 = lane & 15;
  const int hi = lane >> 5;
  const int col = c0 + 16 * ((lane >> 4) & 1) + 4 * (s16 & 3);
  half4_t part[2];
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    const int row = r0 + 8 * jj + 4 * hi + (s16 >> 2);
    const short4_t x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        reinterpret_cast<__attribute__((address_space(3))) short4_t*>(tile + row * ld + col));
    part[jj] = __builtin_bit_cast(half4_t, x);
  }
  return __builtin_shufflevector(part[0], part[1], 0, 1, 2, 3, 4, 5, 6, 7);
}
__device__ __forceinline__ float8_t lds_tr_frag(const lds_ptr<float> tile, int ld, int r0, int c0, int lane) {
  const int hi = lane >> 5;
  const int col = c0 + (lane & 31);
  float8_t f;
#pragma unroll
  for (int j = 0; j < 8; ++j) f[j] = tile[(r0 + 8 * (j >> 2) + 4 * hi + (j & 3)) * ld + col];
  return f;
}

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

// Streams 32-row tiles of two [N, D] row-major tensors (plus, optionally, two
// per-row float vectors) through a two-stage LDS ring.  Each thread moves
// whole 8-element chunks; rows at or past `rows` are zero.
template <typename T, int DP, bool VEC>
struct TilePair {
  typedef typename Elem<T>::frag F;
  static constexpr int CPR = DP / 8;                       // chunks per row
  static constexpr int CHUNKS = kRows * CPR;               // chunks per tile
  static constexpr int PER_THREAD = (CHUNKS + kThreads - 1) / kThreads;
  F a[PER_THREAD], b[PER_THREAD];

  __device__ __forceinline__ void load(const T* pa, const T* pb, int r0, int rows, int d, int tid) {
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
  }
  __device__ __forceinline__ void store(lds_ptr<T> ta, lds_ptr<T> tb, int tid) const {
    constexpr int LD = Tile<T, DP>::LD;
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      const int c = tid + i * kThreads;
      if (CHUNKS % kThreads == 0 || c < CHUNKS) {
        const int row = c / CPR;
        const int col = (c % CPR) * 8;
        *reinterpret_cast<__attribute__((address_space(3))) F*>(ta + row * LD + col) = a[i];
        *reinterpret_cast<__attribute__((address_space(3))) F*>(tb + row * LD + col) = b[i];
      }
    }
  }
};

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
  int BH, N, D, causal;
  float scale;       // 1/sqrt(D)
  float scale_log2;  // scale * log2(e)
};

// ---------------------------------------------------------------------------
// Query-major kernel: MODE 0 = fp32 forward (O, optional LSE), MODE 1 = dQ + delta.
template <typename T, int DP, bool VEC, int MODE>
__global__ __launch_bounds__(kThreads) void query_major_kernel(TrainParams p) {
  typedef typename Elem<T>::frag F;
  constexpr int KK = DP / 16;  // 16-deep reduction steps over d
  constexpr int DB = DP / 32;  // 32-row blocks of d in the transposed products
  constexpr int LD = Tile<T, DP>::LD;
  constexpr int TE = Tile<T, DP>::ELEMS;
  __shared__ __attribute__((aligned(16))) T smem[2 * 2 * TE];

  const int N = p.N, D = p.D;
  const int bh = blockIdx.y;
  const int q0 = blockIdx.x * kBlockRows;
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
      const F of = qvalid ? load_frag<T, VEC>(orow, 16 * kk + 8 * hi, D) : zero_frag<T>();
#pragma unroll
      for (int j = 0; j < 8; ++j) part = fmaf(static_cast<float>(df[kk][j]), static_cast<float>(of[j]), part);
    }
    delta = part + __shfl_xor(part, 32, 64);
    if (qvalid) {
      if (hi == 0) p.delta[static_cast<size_t>(bh) * N + qrow] = delta;
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
  const int kend_w = p.causal ? min(N, wq0 + kRows) : N;     // keys this wave needs
  const int ntiles = (kend + kRows - 1) / kRows;
  lds_ptr<T> lds = (__attribute__((address_space(3))) T*)smem;

  TilePair<T, DP, VEC> st;
  st.load(kp, vp, 0, N, D, tid);
  st.store(lds, lds + TE, tid);
  for (int t = 0; t < ntiles; ++t) {
    const int kt = t * kRows;
    if (t + 1 < ntiles) st.load(kp, vp, kt + kRows, N, D, tid);
    __syncthreads();
    const lds_ptr<T> ks = lds + (t & 1) * 2 * TE;
    const lds_ptr<T> vs = ks + TE;
    if (kt < kend_w) {
      // S^T = K Q^T: lane <-> query, register r <-> key kt + 8 (r/4) + 4 hi + r%4
      float16_t s;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = 0.0f;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) s = mma(lds_row_frag<T>(ks, LD, l32, 16 * kk + 8 * hi), qf[kk], s);
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
        for (int kk = 0; kk < KK; ++kk) dp = mma(lds_row_frag<T>(vs, LD, l32, 16 * kk + 8 * hi), df[kk], dp);
#pragma unroll
        for (int r = 0; r < 16; ++r) pm[r] = fast_exp2(fmaf(s[r], c, -lse2)) * (dp[r] - delta);
      }
      const F pf0 = acc_frag<T>(pm, 0), pf1 = acc_frag<T>(pm, 1);
      // forward: O^T += V^T P^T;  dQ: dQ^T += K^T dS^T
      const lds_ptr<T> src = (MODE == 0) ? vs : ks;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        acc[db] = mma(lds_tr_frag(src, LD, 0, 32 * db, lane), pf0, acc[db]);
        acc[db] = mma(lds_tr_frag(src, LD, 16, 32 * db, lane), pf1, acc[db]);
      }
    }
    if (t + 1 < ntiles) {
      lds_ptr<T> nk = lds + ((t + 1) & 1) * 2 * TE;
      st.store(nk, nk + TE, tid);
    }
  }

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
// Key-major kernel: dK and dV for 32 keys per wave.
template <typename T, int DP, bool VEC>
__global__ __launch_bounds__(kThreads) void dkdv_kernel(TrainParams p) {
  typedef typename Elem<T>::frag F;
  constexpr int KK = DP / 16;
  constexpr int DB = DP / 32;
  constexpr int LD = Tile<T, DP>::LD;
  constexpr int TE = Tile<T, DP>::ELEMS;
  __shared__ __attribute__((aligned(16))) T smem[2 * 2 * TE];
  __shared__ __attribute__((aligned(16))) float svec[2][2][kRows];  // [stage][lse2, delta][row]

  const int N = p.N, D = p.D;
  const int bh = blockIdx.y;
  const int k0 = blockIdx.x * kBlockRows;
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
      vf[kk] = kvalid ? load_frag<T, VEC>(vr, 16 * kk + 8 * hi, D) : zero_frag<T>();
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
  const int t0 = qstart / kRows;
  const int ntiles = (N + kRows - 1) / kRows - t0;
  lds_ptr<T> lds = (__attribute__((address_space(3))) T*)smem;

  TilePair<T, DP, VEC> st;
  float vec_lse = 0.0f, vec_dlt = 0.0f;  // threads < 32: one row of the next tile
  auto load_vec = [&](int r0) {
    if (tid < kRows) {
      const int r = r0 + tid;
      vec_lse = r < N ? lse[r] * kLog2e : INFINITY;  // padding rows: P = 0
      vec_dlt = r < N ? dlt[r] : 0.0f;
    }
  };
  auto store_vec = [&](int stage) {
    if (tid < kRows) {
      svec[stage][0][tid] = vec_lse;
      svec[stage][1][tid] = vec_dlt;
    }
  };
  if (ntiles > 0) {
    st.load(qp, dop, t0 * kRows, N, D, tid);
    load_vec(t0 * kRows);
    st.store(lds, lds + TE, tid);
    store_vec(0);
  }
  for (int t = 0; t < ntiles; ++t) {
    const int qt = (t0 + t) * kRows;
    if (t + 1 < ntiles) {
      st.load(qp, dop, qt + kRows, N, D, tid);
      load_vec(qt + kRows);
    }
    __syncthreads();
    const int stage = t & 1;
    const lds_ptr<T> qs = lds + stage * 2 * TE;
    const lds_ptr<T> ds = qs + TE;
    // a tile whose last query precedes this wave's first key contributes nothing
    if (!(p.causal && qt + kRows - 1 < wk0)) {
      // S = Q K^T and dP = dO V^T: lane <-> key, register r <-> query qt + 8 (r/4) + 4 hi + r%4
      float16_t s, dp;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] = 0.0f;
        dp[r] = 0.0f;
      }
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        s = mma(lds_row_frag<T>(qs, LD, l32, 16 * kk + 8 * hi), kf[kk], s);
        dp = mma(lds_row_frag<T>(ds, LD, l32, 16 * kk + 8 * hi), vf[kk], dp);
      }
      if (p.causal && qt < wk0 + kRows - 1) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qi = qt + 8 * (r >> 2) + 4 * hi + (r & 3);
          if (krow > qi) s[r] = -INFINITY;
        }
      }
      float16_t pm, dsm;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const float4_t l4 = *reinterpret_cast<const float4_t*>(&svec[stage][0][8 * rr + 4 * hi]);
        const float4_t d4 = *reinterpret_cast<const float4_t*>(&svec[stage][1][8 * rr + 4 * hi]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * rr + j;
          pm[r] = fast_exp2(fmaf(s[r], c, -l4[j]));
          dsm[r] = pm[r] * (dp[r] - d4[j]);
        }
      }
      const F pf0 = acc_frag<T>(pm, 0), pf1 = acc_frag<T>(pm, 1);
      const F sf0 = acc_frag<T>(dsm, 0), sf1 = acc_frag<T>(dsm, 1);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        dv[db] = mma(lds_tr_frag(ds, LD, 0, 32 * db, lane), pf0, dv[db]);
        dv[db] = mma(lds_tr_frag(ds, LD, 16, 32 * db, lane), pf1, dv[db]);
        dk[db] = mma(lds_tr_frag(qs, LD, 0, 32 * db, lane), sf0, dk[db]);
        dk[db] = mma(lds_tr_frag(qs, LD, 16, 32 * db, lane), sf1, dk[db]);
      }
    }
    if (t + 1 < ntiles) {
      lds_ptr<T> nq = lds + ((t + 1) & 1) * 2 * TE;
      st.store(nq, nq + TE, tid);
      store_vec((t + 1) & 1);
    }
  }

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
          dkp[d0 + j] = static_cast<T>(dk[db][4 * rr + j] * p.scale);
          dvp[d0 + j] = static_cast<T>(dv[db][4 * rr + j]);
        }
    }
}

// ---------------------------------------------------------------------------
// Host launchers.

template <typename T, int DP, bool VEC>
static void launch_bwd(const TrainParams& p, hipStream_t st) {
  const dim3 grid(ceil_div(p.N, kBlockRows), p.BH);
  hipLaunchKernelGGL((query_major_kernel<T, DP, VEC, 1>), grid, dim3(kThreads), 0, st, p);
  hipLaunchKernelGGL((dkdv_kernel<T, DP, VEC>), grid, dim3(kThreads), 0, st, p);
}

template <typename T>
static int dispatch_bwd(const char* fn, const TrainParams& p, bool vec_ok, hipStream_t st) {
  const int D = p.D;
  const bool vec = vec_ok && (D == 32 || D == 64 || D == 128);
  if (D <= 32) vec ? launch_bwd<T, 32, true>(p, st) : launch_bwd<T, 32, false>(p, st);
  else if (D <= 64) vec ? launch_bwd<T, 64, true>(p, st) : launch_bwd<T, 64, false>(p, st);
  else vec ? launch_bwd<T, 128, true>(p, st) : launch_bwd<T, 128, false>(p, st);
  return check_launch(fn);
}

template <int DP, bool VEC>
static void launch_fwd32(const TrainParams& p, hipStream_t st) {
  const dim3 grid(ceil_div(p.N, kBlockRows), p.BH);
  hipLaunchKernelGGL((query_major_kernel<float, DP, VEC, 0>), grid, dim3(kThreads), 0, st, p);
}

static int check_sizes(const char* fn, int B, int H, int N, int D) {
  if (B < 0 || H <= 0 || N < 0 || D <= 0)
    return set_error(FA_ERR_INVALID_ARG, "%s: bad sizes (B=%d H=%d N=%d D=%d)", fn, B, H, N, D);
  if (D > 128) return set_error(FA_ERR_UNSUPPORTED, "%s: D=%d exceeds 128", fn, D);
  if (static_cast<long long>(B) * H > 65535)
    return set_error(FA_ERR_UNSUPPORTED, "%s: B*H=%lld exceeds 65535", fn, static_cast<long long>(B) * H);
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
  p.scale = 1.0f / sqrtf(static_cast<float>(D));
  p.scale_log2 = p.scale * kLog2e;
  const bool vec = (D == 32 || D == 64 || D == 128) && aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (D <= 32) vec ? launch_fwd32<32, true>(p, st) : launch_fwd32<32, false>(p, st);
  else if (D <= 64) vec ? launch_fwd32<64, true>(p, st) : launch_fwd32<64, false>(p, st);
  else vec ? launch_fwd32<128, true>(p, st) : launch_fwd32<128, false>(p, st);
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
  p.scale = 1.0f / sqrtf(static_cast<float>(D));
  p.scale_log2 = p.scale * kLog2e;
  const bool vec = aligned16(dout) && aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out) &&
                   aligned16(dq) && aligned16(dk) && aligned16(dv);
  hipStream_t st = static_cast<hipStream_t>(stream);
  return fp32 ? dispatch_bwd<float>(fn, p, vec, st) : dispatch_bwd<half_t>(fn, p, vec, st);
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
