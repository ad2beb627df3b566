// Split-KV ("flash-decoding") single-token attention for gfx950.
//
// One kernel family serves the four decode entry points of the reference
// (contiguous MHA/GQA decode, continuous batching, paged decode, INT8 decode):
//
//   grid  = B * H_KV * head_groups * splits workgroups of 256 threads (4 waves)
//   block = one KV head's key range [split*chunk, min(len_b, (split+1)*chunk))
//           for GB query heads of that KV head's group, so each K/V byte is read
//           from HBM once per group instead of once per query head.
//
// Inside a wave a key row of D fp16 is spread over LPR = DP/8 lanes, each lane
// holding 16 contiguous bytes, so every dwordx4 load instruction reads
// 64/LPR whole rows (fully coalesced 128-byte lines).  QK^T is v_dot2_f32_f16
// over the lane's 8 columns followed by a DPP reduction over the LPR lanes of
// the row; each group of LPR lanes keeps its own online-softmax state
// (m, l, acc[8]) for the rows it owns, and the states are merged across lanes
// and waves only once, at the end of the split.  A sequence covered by one
// split writes the fp16 output directly; otherwise each split writes a
// (log2-sum-exp, normalised output) partial, bumps its unit's arrival counter,
// and the last split to arrive merges the partials -- one kernel per call, no
// separate combine launch.  The last split also resets the counter, so a
// zero-filled workspace stays zero-filled between calls (and across graph
// replays) without any memset.
#include <math.h>

#include "capi_internal.h"
#include "common.h"

namespace fa {

enum DecodeMode : int { kModeDecode = 0, kModeCB = 1, kModePaged = 2, kModeInt8 = 3 };

constexpr int kDecWaves = 4;
constexpr int kDecThreads = kDecWaves * 64;
constexpr int kPage = 16;             // PAGE_BLOCK_SIZE of the paged cache
constexpr int kMaxChunk = 8192;       // keys per split, upper bound
constexpr int kChunkQuantum = 128;    // split boundaries are multiples of this
constexpr int kTargetBlocks = 8192;   // aim for this many split workgroups

struct DecodeParams {
  const half_t* q;
  const half_t* k;
  const half_t* v;
  half_t* o;
  const int32_t* lens;         // CB: cache_lens; paged: seq_lens
  const int32_t* block_table;  // paged
  long long bt_numel;
  const float* q_scale;        // INT8
  const float* k_scale;        // INT8
  float* ws_o;                 // [B*H_Q, S, DP] normalised partial outputs
  float* ws_lse;               // [B*H_Q, S] log2-sum-exp of each partial
  unsigned* counters;          // [kCounterSlots] arrivals per unit of a launch; zero between calls
  int unit_base;               // first unit of this launch
  int B, H_Q, H_KV, N, D, G;
  int fixed_len;               // decode / INT8: number of attended keys
  int chunk, num_splits, num_hg;
  int max_num_blocks, num_pages;
  float scale_log2;            // (1/sqrt(D)) * log2(e)
  float scale;                 // 1/sqrt(D) (INT8 score formula)
};

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

// clamp(roundf(x), -127, 127) as an int; fminf/fmaxf map NaN to +127.
__device__ __forceinline__ int quant_i8(float x) {
  float r = __builtin_roundf(x);
  r = fmaxf(-127.0f, fminf(127.0f, r));
  return static_cast<int>(r);
}

__device__ __forceinline__ void quant8(u32x4 raw, float inv, int& lo, int& hi) {
  half8_t h = __builtin_bit_cast(half8_t, raw);
  int b[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) b[j] = quant_i8(static_cast<float>(h[j]) * inv) & 0xFF;
  lo = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
  hi = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
}

template <int DP, int GB, int MODE, bool VEC>
__global__ __launch_bounds__(kDecThreads) void decode_splitkv_kernel(DecodeParams p) {
  constexpr int LPR = DP / 8;       // lanes per key row
  constexpr int RPW = 64 / LPR;     // rows per wave per load instruction
  constexpr int U = 8;              // load instructions in flight per tile
  constexpr int TILE = RPW * U;     // keys per wave per iteration

  const int S = p.num_splits;
  const int split = blockIdx.x % S;
  const int slot = blockIdx.x / S;      // this launch's counter slot
  const int rest = p.unit_base + slot;  // (b, h_kv, head group) unit
  const int hg = rest % p.num_hg;
  const int pair = rest / p.num_hg;
  const int b = pair / p.H_KV;
  const int hkv = pair % p.H_KV;
  const int D = p.D;
  const int G = p.G;
  const int g_base = hg * GB;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int rg = lane / LPR;
  const int col = (lane % LPR) * 8;

  const int L = seq_len_of<MODE>(p, b);
  const int k0 = split * p.chunk;
  const int k1 = min(L, k0 + p.chunk);

  if (k0 >= k1) {
    // No key at all (L <= 0): the reference's acc/l_i is 0/0 there.  Split 0
    // writes the NaN; other empty splits just leave.
    if (L <= 0 && split == 0) {
      for (int i = tid; i < GB * D; i += kDecThreads) {
        const int g = i / D, d = i % D;
        if (g_base + g < G) {
          const int h = hkv * G + g_base + g;
          p.o[(static_cast<size_t>(b) * p.H_Q + h) * D + d] = static_cast<half_t>(__builtin_nanf(""));
        }
      }
    }
    return;
  }

  __shared__ int s_pages[MODE == kModePaged ? kMaxChunk / kPage : 1];
  __shared__ int s_bad;
  if constexpr (MODE == kModePaged) {
    // A sequence longer than its table row would read the next row's page ids.
    if (tid == 0) s_bad = static_cast<long long>(L) > static_cast<long long>(p.max_num_blocks) * kPage;
    __syncthreads();
    const int np = (k1 - k0 + kPage - 1) / kPage;
    for (int i = tid; i < np; i += kDecThreads) {
      const long long idx = static_cast<long long>(b) * p.max_num_blocks + k0 / kPage + i;
      int id = (idx >= 0 && idx < p.bt_numel) ? p.block_table[idx] : -1;
      if (id < 0 || id >= p.num_pages) {
        s_bad = 1;
        id = 0;
      }
      s_pages[i] = id;
    }
    __syncthreads();
  }

  const size_t kv_head_base =
      (static_cast<size_t>(b) * p.H_KV + hkv) * static_cast<size_t>(p.N) * D;
  auto row_off = [&](int t) -> size_t {
    if constexpr (MODE == kModePaged) {
      const int pg = s_pages[(t - k0) >> 4];
      return ((static_cast<size_t>(pg) * p.H_KV + hkv) * kPage + (t & (kPage - 1))) * D;
    } else {
      return kv_head_base + static_cast<size_t>(t) * D;
    }
  };

  // ---- query fragments (this lane's 8 columns of each of the GB heads) ----
  uint32_t qf[GB][4];
  int qi[GB][2];
  float qsc[GB];
  float inv_ks = 0.0f, ks = 0.0f;
  if constexpr (MODE == kModeInt8) {
    ks = p.k_scale[static_cast<size_t>(b) * p.H_KV + hkv];
    inv_ks = 1.0f / ks;
  }
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    const bool hv = g_base + g < G;
    const int h = hkv * G + g_base + g;
    u32x4 x = u32x4{0u, 0u, 0u, 0u};
    if (hv) x = load_row8<VEC>(p.q + (static_cast<size_t>(b) * p.H_Q + h) * D, col, D);
    if constexpr (MODE == kModeInt8) {
      const float qs = hv ? p.q_scale[static_cast<size_t>(b) * p.H_Q + h] : 1.0f;
      qsc[g] = qs;
      quant8(x, 1.0f / qs, qi[g][0], qi[g][1]);
      if (!hv) qi[g][0] = qi[g][1] = 0;
    } else {
      qf[g][0] = x.x; qf[g][1] = x.y; qf[g][2] = x.z; qf[g][3] = x.w;
    }
  }

  float m[GB], l[GB], acc[GB][8];
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    m[g] = kNegBig;
    l[g] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[g][j] = 0.0f;
  }

  for (int t0 = k0 + wave * TILE; t0 < k1; t0 += kDecWaves * TILE) {
    u32x4 kf[U], vf[U];
    bool valid[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = t0 + u * RPW + rg;
      valid[u] = t < k1;
      kf[u] = u32x4{0u, 0u, 0u, 0u};
      if (valid[u]) kf[u] = load_row8<VEC>(p.k + row_off(t), col, D);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = t0 + u * RPW + rg;
      vf[u] = u32x4{0u, 0u, 0u, 0u};
      if (valid[u]) vf[u] = load_row8<VEC>(p.v + row_off(t), col, D);
    }

    float s[U][GB];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if constexpr (MODE == kModeInt8) {
        int klo, khi;
        quant8(kf[u], inv_ks, klo, khi);
#pragma unroll
        for (int g = 0; g < GB; ++g) {
          int di = __builtin_amdgcn_sdot4(qi[g][0], klo, 0, false);
          di = __builtin_amdgcn_sdot4(qi[g][1], khi, di, false);
          di = group_sum_i<LPR>(di);
          const float sc = static_cast<float>(di) * qsc[g] * ks * p.scale;
          s[u][g] = valid[u] ? sc * kLog2e : -INFINITY;
        }
      } else {
#pragma unroll
        for (int g = 0; g < GB; ++g) {
          float d = dot2(qf[g][0], kf[u].x, 0.0f);
          d = dot2(qf[g][1], kf[u].y, d);
          d = dot2(qf[g][2], kf[u].z, d);
          d = dot2(qf[g][3], kf[u].w, d);
          d = group_sum<LPR>(d);
          s[u][g] = valid[u] ? d * p.scale_log2 : -INFINITY;
        }
      }
    }

    float vv[U][8];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      half8_t h = __builtin_bit_cast(half8_t, vf[u]);
#pragma unroll
      for (int j = 0; j < 8; ++j) vv[u][j] = static_cast<float>(h[j]);
    }

#pragma unroll
    for (int g = 0; g < GB; ++g) {
      float mt = s[0][g];
#pragma unroll
      for (int u = 1; u < U; ++u) mt = fmaxf(mt, s[u][g]);
      const float mn = fmaxf(m[g], mt);
      const float alpha = fast_exp2(m[g] - mn);
      m[g] = mn;
      l[g] *= alpha;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[g][j] *= alpha;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float pu = fast_exp2(s[u][g] - mn);
        l[g] += pu;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[g][j] = fmaf(pu, vv[u][j], acc[g][j]);
      }
    }
  }

  // ---- merge the RPW row-group states of this wave ----
#pragma unroll
  for (int off = LPR; off < 64; off <<= 1) {
#pragma unroll
    for (int g = 0; g < GB; ++g) {
      const float mo = __shfl_xor(m[g], off, 64);
      const float lo = __shfl_xor(l[g], off, 64);
      const float mn = fmaxf(m[g], mo);
      const float a = fast_exp2(m[g] - mn);
      const float c = fast_exp2(mo - mn);
      l[g] = l[g] * a + lo * c;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float ao = __shfl_xor(acc[g][j], off, 64);
        acc[g][j] = acc[g][j] * a + ao * c;
      }
      m[g] = mn;
    }
  }

  // ---- merge the waves through LDS and write ----
  __shared__ float s_m[kDecWaves][GB];
  __shared__ float s_l[kDecWaves][GB];
  __shared__ float s_acc[kDecWaves][GB][DP];
  if (rg == 0) {
#pragma unroll
    for (int g = 0; g < GB; ++g) {
#pragma unroll
      for (int j = 0; j < 8; ++j) s_acc[wave][g][col + j] = acc[g][j];
      if (lane == 0) {
        s_m[wave][g] = m[g];
        s_l[wave][g] = l[g];
      }
    }
  }
  __syncthreads();

  bool bad = false;
  if constexpr (MODE == kModePaged) bad = s_bad != 0;
  // Splits that hold keys of this sequence (>= 1 here, since k0 < k1).
  const int sb = min(S, (L + p.chunk - 1) / p.chunk);

  for (int i = tid; i < GB * DP; i += kDecThreads) {
    const int g = i / DP, d = i % DP;
    if (g_base + g >= G || d >= D) continue;
    float mx = s_m[0][g];
#pragma unroll
    for (int w = 1; w < kDecWaves; ++w) mx = fmaxf(mx, s_m[w][g]);
    float lsum = 0.0f, a = 0.0f;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) {
      const float e = fast_exp2(s_m[w][g] - mx);
      lsum += s_l[w][g] * e;
      a += s_acc[w][g][d] * e;
    }
    float outv = a / lsum;
    float lse = mx + __log2f(lsum);
    if (bad) outv = lse = __builtin_nanf("");
    const int h = hkv * G + g_base + g;
    const size_t bh = static_cast<size_t>(b) * p.H_Q + h;
    if (sb == 1) {
      p.o[bh * D + d] = static_cast<half_t>(outv);
    } else {
      const size_t e = bh * S + split;
      store_coherent(&p.ws_o[e * DP + d], outv);
      if (d == 0) store_coherent(&p.ws_lse[e], lse);
    }
  }
  if (sb == 1) return;

  // ---- the last split of this (b, h_kv, head group) to finish merges all partials ----
  // Partials travel through device-coherent (L2-bypassing, sc1) stores and loads,
  // so no whole-L2 writeback/invalidate fence is needed: each thread waits for its
  // stores to complete, the barrier orders that before thread 0's counter atomic,
  // and the last arrival reads the partials with coherent loads.
  __shared__ int s_last;
  wait_vmem_stores();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = atomicAdd(&p.counters[slot], 1u);
    s_last = (prev == static_cast<unsigned>(sb - 1));
  }
  __syncthreads();
  if (!s_last) return;

  for (int i = tid; i < GB * DP; i += kDecThreads) {
    const int g = i / DP, d = i % DP;
    if (g_base + g >= G || d >= D) continue;
    const int h = hkv * G + g_base + g;
    const size_t bh = static_cast<size_t>(b) * p.H_Q + h;
    const float* lse = p.ws_lse + bh * S;
    const float* po = p.ws_o + bh * S * DP;
    float mx = -INFINITY;
    for (int sp = 0; sp < sb; ++sp) mx = fmaxf(mx, load_coherent(&lse[sp]));
    float num = 0.0f, den = 0.0f;
    for (int sp = 0; sp < sb; ++sp) {
      const float w = fast_exp2(load_coherent(&lse[sp]) - mx);
      den += w;
      num += w * load_coherent(&po[static_cast<size_t>(sp) * DP + d]);
    }
    p.o[bh * D + d] = static_cast<half_t>(num / den);
  }
  // Leave the counter at zero for the next call on this workspace.
  if (tid == 0) atomicExch(&p.counters[slot], 0u);
}

// ---------------------------------------------------------------------------
// Host side: split planning and dispatch.

struct DecodePlan {
  int dp, gb, num_hg, chunk, splits;
};

static int pick_dp(int d) { return d <= 64 ? 64 : (d <= 128 ? 128 : 256); }
static int pick_gb(int g) { return g <= 1 ? 1 : (g <= 2 ? 2 : (g <= 4 ? 4 : 8)); }

static DecodePlan make_plan(int B, int H_Q, int H_KV, int max_len, int D) {
  DecodePlan pl;
  const int G = H_Q / H_KV;
  pl.dp = pick_dp(D);
  pl.gb = pick_gb(G);
  pl.num_hg = ceil_div(G, pl.gb);
  const long long units = static_cast<long long>(B) * H_KV * pl.num_hg;
  long long want = (static_cast<long long>(max_len > 0 ? max_len : 1) * units + kTargetBlocks - 1) / kTargetBlocks;
  long long chunk = ((want + kChunkQuantum - 1) / kChunkQuantum) * kChunkQuantum;
  if (chunk < kChunkQuantum) chunk = kChunkQuantum;
  if (chunk > kMaxChunk) chunk = kMaxChunk;
  pl.chunk = static_cast<int>(chunk);
  pl.splits = max_len > 0 ? ceil_div(max_len, chunk) : 1;
  return pl;
}

static size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// Workspace layout: [counters: kCounterSlots x u32][lse: B*H_Q*S f32][partials: B*H_Q*S*DP f32],
// each region 256-byte aligned.  Needed only when a sequence can span several
// splits.  The counter region has the same size and place for every call, so
// one workspace can serve calls of any shape: no call's partials ever land on
// another call's counters.  A launch covers at most kCounterSlots units; larger
// problems are issued as several launches over unit ranges.
constexpr size_t kCounterSlots = 65536;

struct WorkspaceLayout {
  size_t counters, lse, o, total;
};

static WorkspaceLayout plan_layout(const DecodePlan& pl, int B, int H_Q, int H_KV) {
  (void)H_KV;
  WorkspaceLayout w = {0, 0, 0, 0};
  if (pl.splits <= 1) return w;
  const size_t entries = static_cast<size_t>(B) * H_Q * pl.splits;
  w.counters = 0;
  w.lse = align256(kCounterSlots * sizeof(unsigned));
  w.o = w.lse + align256(entries * sizeof(float));
  w.total = w.o + entries * pl.dp * sizeof(float);
  return w;
}

template <int DP, int GB, int MODE, bool VEC>
static void launch_split(const DecodeParams& p, int blocks, hipStream_t st) {
  hipLaunchKernelGGL((decode_splitkv_kernel<DP, GB, MODE, VEC>), dim3(blocks), dim3(kDecThreads), 0, st, p);
}

template <int DP, int MODE, bool VEC>
static void dispatch_gb(int gb, const DecodeParams& p, int blocks, hipStream_t st) {
  switch (gb) {
    case 1: launch_split<DP, 1, MODE, VEC>(p, blocks, st); break;
    case 2: launch_split<DP, 2, MODE, VEC>(p, blocks, st); break;
    case 4: launch_split<DP, 4, MODE, VEC>(p, blocks, st); break;
    default: launch_split<DP, 8, MODE, VEC>(p, blocks, st); break;
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
static int run_decode(const char* fn, DecodeParams p, int max_len, void* ws, size_t ws_bytes, void* stream) {
  const DecodePlan pl = make_plan(p.B, p.H_Q, p.H_KV, max_len, p.D);
  const WorkspaceLayout wl = plan_layout(pl, p.B, p.H_Q, p.H_KV);
  const size_t need = wl.total;
  if (need > 0 && (ws == nullptr || ws_bytes < need))
    return set_error(FA_ERR_WORKSPACE, "%s: workspace of %zu bytes required, %zu given", fn, need, ws_bytes);
  if (p.B == 0) return FA_OK;
  p.G = p.H_Q / p.H_KV;
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
  const bool vec = (p.D % 8 == 0) && aligned16(p.q) && aligned16(p.k) && aligned16(p.v);
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
  return plan_layout(make_plan(B, H_Q, H_KV, max_len, D), B, H_Q, H_KV).total;
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
  return run_decode<kModeDecode>(fn, p, N, workspace, workspace_bytes, stream);
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
  // Splits cover tokens [0, 16*max_num_blocks); a sequence longer than its
  // table row is reported as NaN by the last split (the reference would read
  // the next row's page ids there).
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
  return run_decode<kModeInt8>(fn, p, N, workspace, workspace_bytes, stream);
}
