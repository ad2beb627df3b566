// MFMA-tiled online-softmax prefill for gfx950 (dense MHA/GQA and packed varlen).
//
// Workgroup = 4 waves; each wave owns RW = 64 query rows (32 when D > 128) of one
// (batch, head), so a workgroup covers 4*RW rows.  The KV sequence is walked in
// BK-key tiles (64 keys for D <= 64, 32 above, for the register budget) staged
// in LDS, both row-major:
//   sK [BK][DP + 8]    read (16 B per lane) as the A operand of S^T = K Q^T
//   sV [BK][DP + 32]   read with ds_read_b64_tr_b16 as the A operand of O^T = V^T P^T
// Both products use v_mfma_f32_32x32x16_f16, and each K / V operand read from LDS
// feeds RB = RW/32 MFMAs (one per 32-row query block), halving LDS traffic per
// FLOP against one block per wave.
//
// S^T = K Q^T puts one query row per lane (lane l owns query l%32 of each block
// and 16 keys of each 32-key block): the row max needs one exchange (lanes l,
// l^32) and the row sum stays lane-partial until the end.  The fp32 S^T
// accumulator, converted to fp16, is directly the B operand of the PV product:
// inside each 16-key slice lane half h holds keys {4h..4h+3, 8+4h..8+4h+3}, and
// the transposing LDS read delivers V in exactly that key order (one read per
// 4-key run: 16 source lanes read a 4-key x 16-column block of row-major V and
// lane i receives the 4 keys of column i).  The V row pitch is 64 bytes past a
// multiple of 256, which makes those reads, and the 16-byte row writes, free of
// bank conflicts.
//
// Online softmax with lazy rescaling: the max used for the exponentials is only
// refreshed when a tile's max exceeds it by 2^8 (wave-uniform test), so the O
// accumulators are rarely touched outside the MFMAs.  Only tiles that cross
// the causal diagonal or the sequence end apply the mask (a wave-uniform
// branch around the mask step alone, so the MFMA code exists once and the
// accumulators never move between register files); each wave stops at its
// own diagonal.  Work items are ordered heaviest first across the
// whole grid (all (batch, head) pairs of the last query tile, then the next).
// For D <= 128 the next tile's K/V global loads are issued before the current
// tile's MFMAs.
#include <math.h>

#include "capi_internal.h"
#include "common.h"

namespace fa {

constexpr int kPreWaves = 4;
constexpr int kPreThreads = kPreWaves * 64;
constexpr int kKPad = 8;    // halves of padding per sK row
constexpr int kVPad = 32;   // halves of padding per sV row (pitch = 64 B mod 256 B)

struct PrefillParams {
  const half_t* q;
  const half_t* k;
  const half_t* v;
  half_t* o;
  const int32_t* cu_seqlens;  // varlen only
  int B, H_Q, H_KV, N, D, G;
  int total, row_limit;       // varlen only
  int causal;
  int qtiles;                 // query tiles per (batch, head) in the grid
  float scale_log2;           // (1/sqrt(D)) * log2(e)
};

template <int DP>
struct PrefillShape {
  static constexpr int RB = DP <= 64 ? 2 : 1;   // 32-row query blocks per wave
  static constexpr int RW = 32 * RB;            // query rows per wave
  static constexpr int BQ = kPreWaves * RW;     // query rows per workgroup
  static constexpr int BK = DP <= 128 ? 64 : 32;  // keys per tile (register budget)
};

typedef short short4_t __attribute__((ext_vector_type(4)));

// Four fp16 values of V for the PV A operand: keys base..base+3 of column
// col0 + (lane % 16), via the transposing LDS read (see the file comment).
__device__ __forceinline__ half4_t read_v_tr(const half_t* sV, int pitch, int key_base, int col0, int lane) {
  const int s = lane & 15;
  const half_t* src = sV + (key_base + (s >> 2)) * pitch + col0 + 4 * (s & 3);
  const short4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) short4_t*)(__builtin_amdgcn_readfirstlane(0) + src));
  return __builtin_bit_cast(half4_t, v);
}

template <int DP, bool VARLEN, bool VEC>
__global__ __launch_bounds__(kPreThreads) void prefill_kernel(PrefillParams p) {
  using Shape = PrefillShape<DP>;
  constexpr int RB = Shape::RB;
  constexpr int RW = Shape::RW;
  constexpr int BQ = Shape::BQ;
  constexpr int kBK = Shape::BK;
  constexpr int NBLK = kBK / 32;              // 32-key blocks per tile
  constexpr int KK = DP / 16;                 // 16-wide d slices of QK^T
  constexpr int DB = DP / 32;                 // 32-row d blocks of PV
  constexpr int CPR = DP / 8;                 // 16-byte chunks per row
  constexpr int RPT = kBK * CPR / kPreThreads;  // 16-byte chunks per thread per tile
  constexpr int KP = DP + kKPad;
  constexpr int VP = DP + kVPad;
  constexpr float kRescaleSlack = 8.0f;

  __shared__ __attribute__((aligned(16))) half_t sK[PrefillShape<DP>::BK * KP];
  __shared__ __attribute__((aligned(16))) half_t sV[PrefillShape<DP>::BK * VP];

  const int D = p.D;
  // Heaviest work first: all (batch, head) pairs of the last query tile, then the next.
  const int pairs = p.H_Q * p.B;
  const int qt = p.qtiles - 1 - static_cast<int>(blockIdx.x / pairs);
  const int rem = blockIdx.x % pairs;
  const int h = rem % p.H_Q;
  const int b = rem / p.H_Q;
  const int hk = h / p.G;

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
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  const int wq0 = q0 + wave * RW;  // first query row of this wave

  const half_t* __restrict__ qp = p.q + q_base;
  const half_t* __restrict__ kp = p.k + k_base;
  const half_t* __restrict__ vp = p.v + k_base;

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

  // key ranges: the workgroup walks to its last wave's diagonal, each wave stops at its own
  const int kend_wg = p.causal ? min(seq_len, q0 + BQ) : seq_len;
  const int kend_w = p.causal ? min(seq_len, wq0 + RW) : seq_len;
  const int ntiles = (kend_wg + kBK - 1) / kBK;

  // staging: thread owns 16-byte chunk (tid % CPR) of rows (tid / CPR) + r * (256 / CPR)
  constexpr int RSTEP = kPreThreads / CPR;
  const int sc = tid % CPR;
  const int srow = tid / CPR;
  u32x4 kreg[RPT], vreg[RPT];
  auto fetch = [&](int kt) {
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
      const int key = kt + srow + r * RSTEP;
      const int kc = min(key, seq_len - 1);
      kreg[r] = load_row8<VEC>(kp + static_cast<size_t>(kc) * stride, sc * 8, D);
      vreg[r] = load_row8<VEC>(vp + static_cast<size_t>(kc) * stride, sc * 8, D);
      if (key >= seq_len) {
        kreg[r] = u32x4{0u, 0u, 0u, 0u};
        vreg[r] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  };

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

  auto compute_tile = [&](const int kt, const bool masked) {
    // ---- S^T = K Q^T ----
    float16_t sacc[NBLK][RB];
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
        const half8_t a = *reinterpret_cast<const half8_t*>(&sK[(blk * 32 + l32) * KP + kk * 16 + 8 * hi]);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          sacc[blk][rb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[rb][kk], sacc[blk][rb], 0, 0, 0);
      }
    }
    // ---- softmax (lane owns query row wq0 + 32 rb + l32) ----
    half8_t pf[RB][2 * NBLK];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      if (masked) {  // uniform: only tiles crossing the diagonal or the sequence end
        const int qrow = wq0 + 32 * rb + l32;
#pragma unroll
        for (int blk = 0; blk < NBLK; ++blk)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kt + blk * 32 + 8 * (r >> 2) + 4 * hi + (r & 3);
            const bool dead = key >= seq_len || (p.causal && key > qrow);
            sacc[blk][rb][r] = dead ? -INFINITY : sacc[blk][rb][r];
          }
      }
      float mx = sacc[0][rb][0];
#pragma unroll
      for (int blk = 0; blk < NBLK; ++blk)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[blk][rb][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * c;
      if (__builtin_amdgcn_ballot_w64(mx > m_run[rb] + kRescaleSlack) != 0) {
        const float mn = fmaxf(m_run[rb], mx);
        const float alpha = fast_exp2(m_run[rb] - mn);
        m_run[rb] = mn;
        l_run[rb] *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[db][rb][r] *= alpha;
      }
      const float mneg = -m_run[rb];
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
      l_run[rb] += ls;
    }
    // ---- O^T += V^T P^T ----
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const int col0 = db * 32 + 16 * ((lane >> 4) & 1);
#pragma unroll
      for (int i = 0; i < 2 * NBLK; ++i) {
        const half4_t lo = read_v_tr(sV, VP, 16 * i + 4 * hi, col0, lane);
        const half4_t hi4 = read_v_tr(sV, VP, 16 * i + 8 + 4 * hi, col0, lane);
        const half8_t a = __builtin_shufflevector(lo, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          oacc[db][rb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pf[rb][i], oacc[db][rb], 0, 0, 0);
      }
    }
  };

  // D > 128 has no registers to spare for a prefetched tile: it loads each tile
  // at the top of its own iteration instead.
  constexpr bool kPrefetch = DP <= 128;
  if (kPrefetch && ntiles > 0) fetch(0);
  for (int t = 0; t < ntiles; ++t) {
    const int kt = t * kBK;
    if (!kPrefetch) fetch(kt);
    __syncthreads();  // previous tile's LDS reads are done
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
      const int row = srow + r * RSTEP;
      *reinterpret_cast<u32x4*>(&sK[row * KP + sc * 8]) = kreg[r];
      *reinterpret_cast<u32x4*>(&sV[row * VP + sc * 8]) = vreg[r];
    }
    __syncthreads();
    if (kPrefetch && t + 1 < ntiles) fetch(kt + kBK);
    if (kt >= kend_w) continue;  // past this wave's diagonal (still joins the barriers)
    compute_tile(kt, (kt + kBK > seq_len) || (p.causal && kt + kBK - 1 > wq0));
  }

  // ---- finalize and store O[qrow][d] ----
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const float lt = l_run[rb] + __shfl_xor(l_run[rb], 32, 64);
    const int qrow = wq0 + 32 * rb + l32;
    if (qrow >= rows) continue;
    const float inv = 1.0f / lt;
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

template <int DP, bool VARLEN>
static void launch_prefill(bool vec, int blocks, const PrefillParams& p, hipStream_t st) {
  if (vec)
    hipLaunchKernelGGL((prefill_kernel<DP, VARLEN, true>), dim3(blocks), dim3(kPreThreads), 0, st, p);
  else
    hipLaunchKernelGGL((prefill_kernel<DP, VARLEN, false>), dim3(blocks), dim3(kPreThreads), 0, st, p);
}

static int prefill_bq(int D) { return D <= 64 ? PrefillShape<64>::BQ : (D <= 128 ? PrefillShape<128>::BQ : PrefillShape<256>::BQ); }

// Launches over qtiles * H_Q * B workgroups; returns FA_OK or an error code.
template <bool VARLEN>
static int dispatch_prefill(const char* fn, int D, bool vec, int rows_max, PrefillParams p, hipStream_t st) {
  p.qtiles = ceil_div(rows_max, prefill_bq(D));
  const long long blocks = static_cast<long long>(p.qtiles) * p.H_Q * p.B;
  if (blocks > 0x7fffffffLL) return set_error(FA_ERR_UNSUPPORTED, "%s: problem too large for one launch", fn);
  if (blocks == 0) return FA_OK;
  if (D <= 64) launch_prefill<64, VARLEN>(vec, static_cast<int>(blocks), p, st);
  else if (D <= 128) launch_prefill<128, VARLEN>(vec, static_cast<int>(blocks), p, st);
  else launch_prefill<256, VARLEN>(vec, static_cast<int>(blocks), p, st);
  return check_launch(fn);
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
  return dispatch_prefill<false>(fn, D, vec, N, p, static_cast<hipStream_t>(stream));
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
