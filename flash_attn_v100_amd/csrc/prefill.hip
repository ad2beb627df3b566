// MFMA-tiled online-softmax prefill for gfx950 (dense MHA/GQA and packed varlen).
//
// Workgroup = 4 waves = 128 query rows (32 per wave) of one (batch, head);
// the KV sequence is walked in 64-key tiles staged in LDS:
//   sK  [64][DP + 8]      key-major, read as the A operand of S^T = K Q^T
//   sVt [DP][64 + 8]      V transposed, read as the A operand of O^T = V^T P^T
// Both products use v_mfma_f32_32x32x16_f16.  Computing the transposed scores
// puts one query row per lane (lane l owns query l%32 and 16 keys of each 32-key
// block), so the row max needs a single cross-lane exchange (lanes l, l^32),
// the row sum stays lane-partial until the end, and the fp32 S accumulator,
// converted to fp16, is directly the B operand of the PV product: the key order
// inside each 16-wide k-slice of that MFMA is chosen to match the accumulator
// layout, and sVt is read in that same order (two 8-byte reads per operand).
// The next tile's K/V global loads are issued before the current tile's MFMAs
// so their HBM latency overlaps compute.
#include <math.h>

#include "capi_internal.h"
#include "common.h"

namespace fa {

constexpr int kPreWaves = 4;
constexpr int kPreThreads = kPreWaves * 64;
constexpr int kBQ = 32 * kPreWaves;  // query rows per workgroup
constexpr int kBK = 64;              // keys per tile
constexpr int kKPad = 8;             // halves of padding per sK row
constexpr int kVPad = 8;             // halves of padding per sVt row

struct PrefillParams {
  const half_t* q;
  const half_t* k;
  const half_t* v;
  half_t* o;
  const int32_t* cu_seqlens;  // varlen only
  int B, H_Q, H_KV, N, D, G;
  int total, row_limit;       // varlen only
  int causal;
  float scale_log2;
};

template <int N>
struct HalfVec;
template <>
struct HalfVec<2> { typedef half2_t type; };
template <>
struct HalfVec<4> { typedef half4_t type; };
template <>
struct HalfVec<8> { typedef half8_t type; };

template <int DP, bool VARLEN, bool VEC>
__global__ __launch_bounds__(kPreThreads) void prefill_kernel(PrefillParams p) {
  constexpr int KK = DP / 16;         // 16-wide d slices of the QK^T product
  constexpr int DB = DP / 32;         // 32-row d blocks of the PV product
  constexpr int CPR = DP / 8;         // 16-byte chunks per row
  constexpr int R = kBK * CPR / kPreThreads;  // consecutive key rows per staging thread
  constexpr int KPITCH = DP + kKPad;
  constexpr int VPITCH = kBK + kVPad;
  typedef typename HalfVec<R>::type halfR;

  __shared__ __attribute__((aligned(16))) half_t sK[kBK * KPITCH];
  __shared__ __attribute__((aligned(16))) half_t sVt[DP * VPITCH];

  const int D = p.D;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int hk = h / p.G;

  // ---- sequence geometry ----
  size_t q_base, k_base;     // element offsets of row 0, column 0 of this head
  size_t q_stride, k_stride; // elements between consecutive rows
  int seq_len, rows;
  if constexpr (VARLEN) {
    int s = p.cu_seqlens[b];
    int e = p.cu_seqlens[b + 1];
    s = max(0, min(s, p.total));
    e = max(0, min(e, p.total));
    seq_len = e - s;
    rows = min(seq_len, p.row_limit);
    q_stride = k_stride = static_cast<size_t>(p.H_Q) * D;
    q_base = static_cast<size_t>(s) * q_stride + static_cast<size_t>(h) * D;
    k_base = q_base;
  } else {
    seq_len = rows = p.N;
    q_stride = k_stride = D;
    q_base = (static_cast<size_t>(b) * p.H_Q + h) * static_cast<size_t>(p.N) * D;
    k_base = (static_cast<size_t>(b) * p.H_KV + hk) * static_cast<size_t>(p.N) * D;
  }
  // Heaviest (last) query tiles are dispatched first.
  const int q0 = (gridDim.x - 1 - blockIdx.x) * kBQ;
  if (q0 >= rows) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  const int qrow = q0 + wave * 32 + l32;  // query row owned by this lane

  const half_t* __restrict__ qp = p.q + q_base;
  const half_t* __restrict__ kp = p.k + k_base;
  const half_t* __restrict__ vp = p.v + k_base;

  // ---- Q fragments: B operand of S^T, lane holds q row l32, d = kk*16 + 8*hi .. +8 ----
  half8_t qf[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
    u32x4 x = u32x4{0u, 0u, 0u, 0u};
    if (qrow < rows) x = load_row8<VEC>(qp + static_cast<size_t>(qrow) * q_stride, kk * 16 + 8 * hi, D);
    qf[kk] = __builtin_bit_cast(half8_t, x);
  }

  const int kend = p.causal ? min(seq_len, q0 + kBQ) : seq_len;
  const int ntiles = (kend + kBK - 1) / kBK;

  // staging assignment: chunk c of rows key0 .. key0+R-1
  const int sc = tid % CPR;
  const int skey0 = (tid / CPR) * R;

  u32x4 kreg[R], vreg[R];
  auto fetch = [&](int kt) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int key = kt + skey0 + r;
      kreg[r] = u32x4{0u, 0u, 0u, 0u};
      vreg[r] = u32x4{0u, 0u, 0u, 0u};
      if (key < seq_len) {
        kreg[r] = load_row8<VEC>(kp + static_cast<size_t>(key) * k_stride, sc * 8, D);
        vreg[r] = load_row8<VEC>(vp + static_cast<size_t>(key) * k_stride, sc * 8, D);
      }
    }
  };

  float16_t oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[db][r] = 0.0f;
  float m_run = kNegBig;  // running max (log2 domain) of query qrow
  float l_run = 0.0f;     // lane-partial running sum

  if (ntiles > 0) fetch(0);

  for (int t = 0; t < ntiles; ++t) {
    const int kt = t * kBK;
    __syncthreads();  // previous tile's LDS reads are done
#pragma unroll
    for (int r = 0; r < R; ++r)
      *reinterpret_cast<u32x4*>(&sK[(skey0 + r) * KPITCH + sc * 8]) = kreg[r];
    {
      half8_t vh[R];
#pragma unroll
      for (int r = 0; r < R; ++r) vh[r] = __builtin_bit_cast(half8_t, vreg[r]);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        halfR col;
#pragma unroll
        for (int r = 0; r < R; ++r) col[r] = vh[r][j];
        *reinterpret_cast<halfR*>(&sVt[(sc * 8 + j) * VPITCH + skey0]) = col;
      }
    }
    __syncthreads();
    if (t + 1 < ntiles) fetch(kt + kBK);

    // ---- S^T = K Q^T : two 32-key blocks ----
    float16_t sacc[2];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[blk][r] = 0.0f;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const half8_t a = *reinterpret_cast<const half8_t*>(&sK[(blk * 32 + l32) * KPITCH + kk * 16 + 8 * hi]);
        sacc[blk] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[kk], sacc[blk], 0, 0, 0);
      }
    }

    // ---- mask + online softmax (lane owns query qrow) ----
    const bool need_mask = (kt + kBK > seq_len) || (p.causal && kt + kBK - 1 > q0 + wave * 32);
    float mx = -INFINITY;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float s = sacc[blk][r] * p.scale_log2;
        if (need_mask) {
          const int key = kt + blk * 32 + 8 * (r >> 2) + 4 * hi + (r & 3);
          if (key >= seq_len || (p.causal && key > qrow)) s = -INFINITY;
        }
        sacc[blk][r] = s;
        mx = fmaxf(mx, s);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = fast_exp2(m_run - m_new);
    m_run = m_new;
    l_run *= alpha;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;

    half8_t pf[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float e = fast_exp2(sacc[i >> 1][8 * (i & 1) + j] - m_new);
        l_run += e;
        pf[i][j] = static_cast<half_t>(e);
      }
    }

    // ---- O^T += V^T P^T ----
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const half_t* vrow = &sVt[(db * 32 + l32) * VPITCH];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const half4_t lo = *reinterpret_cast<const half4_t*>(vrow + 16 * i + 4 * hi);
        const half4_t hi4 = *reinterpret_cast<const half4_t*>(vrow + 16 * i + 8 + 4 * hi);
        const half8_t a = __builtin_shufflevector(lo, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
        oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pf[i], oacc[db], 0, 0, 0);
      }
    }
  }

  // ---- finalize and store O[qrow][d] ----
  l_run += __shfl_xor(l_run, 32, 64);
  if (qrow >= rows) return;
  const float inv = 1.0f / l_run;
  half_t* op = p.o + q_base + static_cast<size_t>(qrow) * q_stride;
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int d0 = db * 32 + 8 * rr + 4 * hi;
      half4_t hv;
#pragma unroll
      for (int j = 0; j < 4; ++j) hv[j] = static_cast<half_t>(oacc[db][4 * rr + j] * inv);
      if constexpr (VEC) {
        if (d0 < D) *reinterpret_cast<half4_t*>(op + d0) = hv;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (d0 + j < D) op[d0 + j] = hv[j];
      }
    }
  }
}

template <int DP, bool VARLEN>
static void launch_prefill(bool vec, dim3 grid, const PrefillParams& p, hipStream_t st) {
  if (vec)
    hipLaunchKernelGGL((prefill_kernel<DP, VARLEN, true>), grid, dim3(kPreThreads), 0, st, p);
  else
    hipLaunchKernelGGL((prefill_kernel<DP, VARLEN, false>), grid, dim3(kPreThreads), 0, st, p);
}

template <bool VARLEN>
static void dispatch_prefill(int D, bool vec, dim3 grid, const PrefillParams& p, hipStream_t st) {
  if (D <= 64) launch_prefill<64, VARLEN>(vec, grid, p, st);
  else if (D <= 128) launch_prefill<128, VARLEN>(vec, grid, p, st);
  else launch_prefill<256, VARLEN>(vec, grid, p, st);
}

}  // namespace fa

using namespace fa;

extern "C" int fa_prefill_fp16(const void* q, const void* k, const void* v, void* o, int B, int H_Q,
                               int H_KV, int N, int D, int causal, void* stream) {
  const char* fn = "fa_prefill_fp16";
  if (B < 0 || N < 0 || H_Q <= 0 || H_KV <= 0 || D <= 0)
    return set_error(FA_ERR_INVALID_ARG, "%s: bad sizes (B=%d H_Q=%d H_KV=%d N=%d D=%d)", fn, B, H_Q, H_KV, N, D);
  if (H_Q < H_KV || H_Q % H_KV != 0)
    return set_error(FA_ERR_INVALID_ARG, "%s: H_Q (%d) must be a multiple of H_KV (%d)", fn, H_Q, H_KV);
  if (D > 256) return set_error(FA_ERR_UNSUPPORTED, "%s: D=%d exceeds 256", fn, D);
  if (B == 0 || N == 0) return FA_OK;
  if (!q || !k || !v || !o) return set_error(FA_ERR_INVALID_ARG, "%s: null tensor pointer", fn);
  if (B > 65535 || H_Q > 65535) return set_error(FA_ERR_UNSUPPORTED, "%s: B/H_Q exceed the grid limits", fn);
  PrefillParams p = {};
  p.q = static_cast<const half_t*>(q);
  p.k = static_cast<const half_t*>(k);
  p.v = static_cast<const half_t*>(v);
  p.o = static_cast<half_t*>(o);
  p.B = B; p.H_Q = H_Q; p.H_KV = H_KV; p.N = N; p.D = D; p.G = H_Q / H_KV;
  p.causal = causal ? 1 : 0;
  p.scale_log2 = (1.0f / sqrtf(static_cast<float>(D))) * kLog2e;
  // Vector path: D fills the padded width exactly and every row starts 16-byte aligned.
  const bool vec = (D == 64 || D == 128 || D == 256) && aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o);
  dim3 grid(ceil_div(N, kBQ), H_Q, B);
  dispatch_prefill<false>(D, vec, grid, p, static_cast<hipStream_t>(stream));
  return check_launch(fn);
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
  if (batch == 0 || total == 0 || row_limit == 0) return FA_OK;
  if (!q || !k || !v || !o || !cu_seqlens) return set_error(FA_ERR_INVALID_ARG, "%s: null pointer", fn);
  if (batch > 65535 || H > 65535) return set_error(FA_ERR_UNSUPPORTED, "%s: batch/H exceed the grid limits", fn);
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
  dim3 grid(ceil_div(rows_max, kBQ), H, batch);
  dispatch_prefill<true>(D, vec, grid, p, static_cast<hipStream_t>(stream));
  return check_launch(fn);
}
