// Shared device helpers for the gfx950 (CDNA4) attention kernels.
//
// Wavefronts are 64 lanes.  Cross-lane reductions inside a 16-lane DPP row use
// quad_perm / row_half_mirror / row_mirror moves (no LDS traffic); wider
// reductions fall back to ds_swizzle/bpermute through __shfl_xor.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
// Finite "no score yet" sentinel for running maxima in the log2 domain.  Every
// real score of fp16 inputs is far above it, and exp2(sentinel - real) == 0.
constexpr float kNegBig = -1.0e30f;

// DPP control words (GFX9 encoding).
constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_mov_i(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xF, 0xF, false);
}

// Sum over aligned groups of W lanes (W in {8, 16, 32, 64}); every lane of the
// group receives the group total.
template <int W>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(W == 8 || W == 16 || W == 32 || W == 64, "group width");
  x += dpp_mov<kDppQuadXor1>(x);
  x += dpp_mov<kDppQuadXor2>(x);
  x += dpp_mov<kDppRowHalfMirror>(x);
  if constexpr (W >= 16) x += dpp_mov<kDppRowMirror>(x);
  if constexpr (W >= 32) x += __shfl_xor(x, 16, 64);
  if constexpr (W >= 64) x += __shfl_xor(x, 32, 64);
  return x;
}
template <int W>
__device__ __forceinline__ int group_sum_i(int x) {
  static_assert(W == 8 || W == 16 || W == 32 || W == 64, "group width");
  x += dpp_mov_i<kDppQuadXor1>(x);
  x += dpp_mov_i<kDppQuadXor2>(x);
  x += dpp_mov_i<kDppRowHalfMirror>(x);
  if constexpr (W >= 16) x += dpp_mov_i<kDppRowMirror>(x);
  if constexpr (W >= 32) x += __shfl_xor(x, 16, 64);
  if constexpr (W >= 64) x += __shfl_xor(x, 32, 64);
  return x;
}

// Max over the 64 lanes of a wave; every lane receives it.
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp_mov<kDppQuadXor1>(x));
  x = fmaxf(x, dpp_mov<kDppQuadXor2>(x));
  x = fmaxf(x, dpp_mov<kDppRowHalfMirror>(x));
  x = fmaxf(x, dpp_mov<kDppRowMirror>(x));
  x = fmaxf(x, __shfl_xor(x, 16, 64));
  x = fmaxf(x, __shfl_xor(x, 32, 64));
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t as_u32(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), c, false);
}

// Device-coherent scalar store / load: relaxed atomics at agent scope, which
// gfx950 issues as sc1 global stores/loads that bypass the (per-XCD, not
// mutually coherent) L2 caches.  Used for data handed between workgroups.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// gfx950 lane swaps, in place: permlane32_swap exchanges lanes 32-63 of `a`
// with lanes 0-31 of `b`; permlane16_swap exchanges the odd 16-lane rows of
// `a` with the even rows of `b`.  Inline asm: the compiler's two-result
// builtins were observed to reuse one result register for both results
// (ROCm 7.2, hipcc -O3), which silently drops the swap.
__device__ __forceinline__ void permlane32_swap(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void permlane16_swap(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

// 16-byte device-coherent (sc1, write-through) store of a float4.
__device__ __forceinline__ void store_coherent4(float* p, float4_t v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}


// s_waitcnt vmcnt(0): this thread's vector memory operations, stores included,
// have completed.  (GFX9 encoding: vmcnt 0, expcnt 7, lgkmcnt 15.)
__device__ __forceinline__ void wait_vmem() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): every vector memory load and store done
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
__device__ __forceinline__ void wait_vmem_stores() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Eight fp16 values starting at column `col` of a row of length `d`, zero past d.
// VEC: the caller guarantees col + 8 <= d and a 16-byte aligned address, so one
// unconditional dwordx4 load serves (the kernels use it when d equals their
// padded width and every base pointer is 16-byte aligned).
// NT: nontemporal (streaming) load, for data read exactly once.
template <bool VEC, bool NT = false>
__device__ __forceinline__ u32x4 load_row8(const half_t* row, int col, int d) {
  if constexpr (VEC) {
    (void)d;
    if constexpr (NT)
      return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row + col));
    else
      return *reinterpret_cast<const u32x4*>(row + col);
  } else {
    half8_t h;
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = (col + j < d) ? row[col + j] : (half_t)0.0f;
    return __builtin_bit_cast(u32x4, h);
  }
}

// ---- LDS tiles of fp16 rows (DP = 64, 128 or 256 halves, unpadded) ----
// Physical 16-byte chunk of logical chunk c in tile row r is c ^ chunk_swizzle(r).
// Row reads (16 B per lane, lane l reading row l % 32 at one logical chunk):
// 16 lanes read rows 0..15 at one logical chunk -> 16 distinct bank groups.
// Transposing reads (ds_read_b64_tr_b16, 16 lanes reading a 4-row x 16-column
// block): 32 lanes read rows 4k..4k+3 at 4 consecutive chunks -> 16 distinct
// bank groups (rows are 128 B apart for DP = 64, so there the row parity also
// selects the half of the 256-byte bank window).
template <int DP>
__device__ __forceinline__ int chunk_swizzle(int r) {
  if constexpr (DP <= 64)
    return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
  else
    return ((r & 3) << 2) | ((r >> 2) & 3);
}

typedef short short4_t __attribute__((ext_vector_type(4)));

// s_waitcnt vmcnt(N) lgkmcnt(0).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70);
}

// A wave-uniform pointer as SGPRs (readfirstlane of both halves): the copy
// helpers below take their base as an asm "s" operand, which does not
// compile when the compiler cannot prove the value uniform; for a value
// already in SGPRs this costs nothing.
template <typename T>
__device__ __forceinline__ const T* sgpr_ptr(const T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const T*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// One 16-byte-per-lane copy HBM -> LDS (global_load_lds_dwordx4, scalar base +
// 32-bit lane byte offset): lane i's 16 bytes land at LDS byte address
// lds_addr + 16 i.  Issued from asm so that the compiler does not track the
// copy (it would otherwise wait for every copy in flight before the
// transposing LDS reads); the caller waits with vmcnt before a barrier.  M0,
// which holds the LDS address, is restored afterwards.
__device__ __forceinline__ void copy16_to_lds(const half_t* base, unsigned lane_off, unsigned lds_addr) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dwordx4 %2, %3\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(lane_off), "s"(sgpr_ptr(base))
      : "memory");
}

// copy16_to_lds with a nontemporal (streaming) read of data used once.
__device__ __forceinline__ void copy16_to_lds_nt(const half_t* base, unsigned lane_off, unsigned lds_addr) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dwordx4 %2, %3 nt\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(lane_off), "s"(sgpr_ptr(base))
      : "memory");
}

// s_waitcnt vmcnt(N) alone (LDS and scalar loads not waited for).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | (0xF << 8));
}

// As copy16_to_lds with 4 bytes per lane (global_load_lds_dword): lane i's
// dword lands at lds_addr + 4 i.
__device__ __forceinline__ void copy4_to_lds(const float* base, unsigned lane_off, unsigned lds_addr) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dword %2, %3\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(lane_off), "s"(sgpr_ptr(base))
      : "memory");
}

template <typename T>
__device__ __forceinline__ const __attribute__((address_space(3))) T* lds_at(unsigned byte_addr) {
  return reinterpret_cast<const __attribute__((address_space(3))) T*>(static_cast<size_t>(byte_addr));
}

// Workgroup barrier that neither waits for outstanding LDS DMA nor lets the
// compiler move memory operations across it (the caller waits explicitly).
__device__ __forceinline__ void tile_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

}  // namespace fa
