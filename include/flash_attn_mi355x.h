/*
 * C ABI of the MI355X (gfx950) attention hot path.
 *
 * Plain pointers and sizes only: no torch, no HIP types in the signatures
 * (`stream` is a hipStream_t passed as void*, NULL = the null stream).  Every
 * tensor is a dense row-major fp16 array in device memory unless stated.  The
 * library never allocates: split-KV decode entry points take a caller-owned
 * device workspace whose size comes from fa_decode_workspace_size().  The
 * workspace must be zero-filled before its first use; every call leaves it
 * zero-filled again when it completes, so one workspace serves any number of
 * calls issued in order on one stream (calls that may overlap need separate
 * workspaces).  All calls are asynchronous on `stream` and otherwise stateless.
 *
 * Return value: FA_OK (0) or an FA_ERR_* code; fa_last_error() gives a
 * human-readable message for the calling thread's most recent failure.
 *
 * Each entry point replaces one kernel launch of the reference extension
 * (acproject/flash_attn_v100); the reference interface it stands in for is cited
 * as file:line under the reference tree.
 */
#ifndef FLASH_ATTN_MI355X_H
#define FLASH_ATTN_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  FA_OK = 0,
  FA_ERR_INVALID_ARG = 1,   /* shape / pointer / size argument rejected     */
  FA_ERR_WORKSPACE = 2,     /* workspace missing or smaller than required   */
  FA_ERR_UNSUPPORTED = 3,   /* valid request outside what the kernels cover */
  FA_ERR_HIP = 4            /* a HIP runtime call or kernel launch failed   */
};

/* Message describing the calling thread's last non-OK return. */
const char* fa_last_error(void);

/* Library version string ("<major>.<minor>.<patch> gfx950"). */
const char* fa_version(void);

/*
 * Causal / full self-attention prefill, MFMA-tiled.
 *   q [B, H_Q, N, D], k/v [B, H_KV, N, D], o [B, H_Q, N, D]; H_Q % H_KV == 0,
 *   1 <= D <= 256.  Causal masks key j > query i.  Scale 1/sqrt(D).
 * Replaces the launches behind forward_fp16 (flash_attn_kernel.cu:1915-1962),
 * forward_fp16_wmma (:2425-2468) and forward_prefill_gqa_fp16 (:2740-2794,
 * launch_prefill_gqa_fp16 :316-366).
 */
int fa_prefill_fp16(const void* q, const void* k, const void* v, void* o,
                    int B, int H_Q, int H_KV, int N, int D, int causal,
                    void* stream);

/*
 * fp16 MHA prefill that also returns the natural-log log-sum-exp of each
 * query row's scaled scores, lse [B, H, N] fp32 (the statistic the backward
 * consumes).  q/k/v/o [B, H, N, D], 1 <= D <= 256 (the binding keeps the
 * reference's D <= 128).
 * Replaces the launch behind forward_fp16_with_lse (flash_attn_kernel.cu:2008-2050,
 * kernel flash_attn_kernel_fp16 with a non-null LSE, :1295-1297).
 */
int fa_prefill_fp16_lse(const void* q, const void* k, const void* v, void* o,
                        float* lse, int B, int H, int N, int D, int causal,
                        void* stream);

/*
 * fp32 MHA prefill (fp32 MFMA), optionally with log-sum-exp.
 *   q/k/v/o fp32 [B, H, N, D], 1 <= D <= 128; lse fp32 [B, H, N]
 *   or NULL.  Causal masks key j > query i.
 * Replaces the launches behind forward (flash_attn_kernel.cu:508-550) and
 * forward_with_lse (:1964-2006), kernel flash_attn_kernel (:369-506).
 */
int fa_prefill_fp32(const void* q, const void* k, const void* v, void* o,
                    float* lse, int B, int H, int N, int D, int causal,
                    void* stream);

/*
 * Workspace bytes fa_backward_fp16/_fp32 need (one fp32 per query row).
 */
size_t fa_backward_workspace_size(int B, int H, int N);

/*
 * Attention backward for MHA: given dout, q, k, v, the forward output `out`
 * and its log-sum-exp `lse` [B, H, N] fp32, writes dq, dk, dv (same shape and
 * type as q).  fp16 variant: every tensor but lse is fp16 (gradients
 * accumulate in fp32 and are rounded once); fp32 variant: all fp32.
 * 1 <= D <= 128.  Two or three launches on `stream` (dQ with the row
 * statistic delta = rowsum(dout * out) into the workspace, then dK/dV, as one
 * pass or as a dV and a dK pass); deterministic (no atomics).  The workspace needs no initialisation.
 * Outside graph capture delta comes from a short kernel of its own and the
 * dK/dV work (fp16 at D > 64: the dV and the dK pass) runs on library-owned
 * side streams of the device (non-blocking, default priority) concurrently
 * with the dQ kernel, forked
 * from `stream` by events and joined back into it before return, so all of
 * the call's work is ordered before later work on `stream`; while `stream`
 * is being captured into a graph every launch stays on `stream`.  Results
 * are bit-identical either way.
 * Replaces flash_attn_backward (flash_attn_kernel.cu:2173-2264), kernels
 * flash_attn_backward_tiled_kernel_fp32/_fp16 (:2056-2171).
 */
int fa_backward_fp16(const void* dout, const void* q, const void* k,
                     const void* v, const void* out, const float* lse,
                     void* dq, void* dk, void* dv, int B, int H, int N, int D,
                     int causal, void* workspace, size_t workspace_bytes,
                     void* stream);
int fa_backward_fp32(const void* dout, const void* q, const void* k,
                     const void* v, const void* out, const float* lse,
                     void* dq, void* dk, void* dv, int B, int H, int N, int D,
                     int causal, void* workspace, size_t workspace_bytes,
                     void* stream);

/*
 * Packed variable-length prefill.
 *   q/k/v/o [total, H, D]; cu_seqlens int32 [batch + 1] in device memory.
 *   Sequence b owns rows [cu[b], cu[b+1]); only its first `row_limit` rows get
 *   attention outputs (the reference's grid covers tile*ceil(max_seqlen/tile)
 *   rows per sequence, with tile 32 for D <= 128 and 8 above); every other row
 *   of o is set to zero, as in the reference's zero-initialised output.
 * Replaces launch_varlen_prefill_fp16_on_stream (flash_attn_kernel.cu:3302-3352)
 * behind forward_varlen_prefill_fp16 (:3354-3387) and its _stream variant
 * (:3675-3712).
 */
int fa_varlen_prefill_fp16(const void* q, const void* k, const void* v, void* o,
                           const int32_t* cu_seqlens, int batch, int total,
                           int H, int D, int max_seqlen, int row_limit,
                           int causal, void* stream);

/*
 * Workspace bytes the split-KV decode entry points need for a call with these
 * sizes.  max_len = N (contiguous decode / INT8), max_N (continuous batching)
 * or 16 * max_num_blocks (paged).  May be 0.
 */
size_t fa_decode_workspace_size(int B, int H_Q, int H_KV, int max_len, int D);

/*
 * Single-token decode against a contiguous KV cache (MHA when H_Q == H_KV).
 *   q/o [B, H_Q, 1, D], k/v [B, H_KV, N, D]; 0 <= cache_len < N.
 *   causal: keys j > cache_len are masked; otherwise all N keys attend.
 * Replaces the launches behind forward_decode_fp16 (flash_attn_kernel.cu:1863-1913),
 * forward_decode_gqa_fp16 (:1800-1833, launch_decode_gqa_fp16_on_stream
 * :251-303), its _out (:1835-1861) and _stream (:3639-3673) variants.
 */
int fa_decode_fp16(const void* q, const void* k, const void* v, void* o,
                   int B, int H_Q, int H_KV, int N, int D, int causal,
                   int cache_len, void* workspace, size_t workspace_bytes,
                   void* stream);

/*
 * fa_decode_fp16 without a caller workspace, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, hosts that forbid
 * device allocation).  It has no counterpart in the reference.  Same
 * arguments and results as fa_decode_fp16; the split workspace is a static
 * 16 MiB device array of the library, one per GPU, held until the process
 * ends, so the call allocates nothing.  A call whose workspace would exceed
 * it returns FA_ERR_UNSUPPORTED (fa_decode_workspace_size gives the need of
 * the widest plan; small-batch decode such as B=1, 32:8 heads, 4097 keys,
 * D=128 needs about 1.3 MB).  Calls that may overlap on one GPU share that
 * array and race: issue them in order (one stream, or joined streams).
 */
int fa_decode_fp16_noalloc(const void* q, const void* k, const void* v, void* o,
                           int B, int H_Q, int H_KV, int N, int D, int causal,
                           int cache_len, void* stream);

/*
 * GQA decode against an INT8 KV cache with per-token fp16 scales.
 *   k_int8/v_int8 int8 [B, H_KV, N, D]; k_scale/v_scale fp16 [B, H_KV, N].
 *   Element (t, d) is used as half(code * scale[t]); keys k <= cache_len are
 *   attended (cache_len unchecked: >= N attends all N keys, < 0 none -> NaN).
 *   Workspace as for fa_decode_fp16 (max_len = N).
 * Replaces flash_attn_kernel_decode_int8_kv_cache_gqa (flash_attn_kernel.cu:4020-4159)
 * behind flash_attn_forward_decode_int8_kv_cache_gqa (:4161-4221, bound at flash_attn.cpp:249).
 */
int fa_decode_int8_kv_cache_gqa(const void* q, const void* k_int8, const void* v_int8,
                                const void* k_scale, const void* v_scale, void* o, int B,
                                int H_Q, int H_KV, int N, int D, int cache_len,
                                void* workspace, size_t workspace_bytes, void* stream);

/*
 * Sliding-window (+ attention-sink) GQA decode against a contiguous cache.
 *   Attends key k iff k < sink_size, or window_start <= k <= cache_len with
 *   window_start = max(0, min(cache_len + 1, N) - window_size); no keys -> NaN.
 *   cache_len is not range-checked (keys stay inside [0, N)).  Workspace as for
 *   fa_decode_fp16 (max_len = N).
 * Replaces flash_attn_kernel_decode_sliding_window_gqa (flash_attn_kernel.cu:4346-4482)
 * behind flash_attn_forward_decode_sliding_window_gqa (:4484-4535, bound at flash_attn.cpp:251).
 */
int fa_decode_sliding_window_gqa(const void* q, const void* k, const void* v, void* o, int B,
                                 int H_Q, int H_KV, int N, int D, int cache_len,
                                 int window_size, int sink_size, void* workspace,
                                 size_t workspace_bytes, void* stream);

/*
 * Continuous-batching decode: per-sequence cache lengths.
 *   q/o [B, H_Q, 1, D], k/v [B, H_KV, max_N, D], cache_lens int32 [B] (device).
 *   Sequence b attends keys [0, min(cache_lens[b] + 1, max_N)); an empty range
 *   yields NaN, as 0/0 does in the reference.
 * Replaces the launch in flash_attn_forward_continuous_batching_fp16
 * (continuous_batching_kernel.cu:338-406).
 */
int fa_continuous_batching_fp16(const void* q, const void* k, const void* v,
                                void* o, const int32_t* cache_lens, int B,
                                int H_Q, int H_KV, int max_N, int D, int causal,
                                void* workspace, size_t workspace_bytes,
                                void* stream);

/*
 * Paged GQA decode, 16-token pages.
 *   q/o [B, H_Q, 1, D]; k_cache/v_cache [num_pages, H_KV, 16, D];
 *   block_table int32 (device), read as flat[b * max_num_blocks + t / 16] for
 *   token t (block_table_numel bounds that read); seq_lens int32 [B] (device).
 *   Sequence b attends tokens [0, seq_lens[b]).  seq_lens[b] <= 0 yields NaN
 *   (0/0, as in the reference).  A sequence longer than 16 * max_num_blocks
 *   reads on into the next table row, exactly as the reference's flat read
 *   does.  A page id outside [0, num_pages) or a table index past
 *   block_table_numel yields NaN for that sequence (the reference reads out of
 *   bounds there).
 * Replaces the launch in flash_attn_forward_paged_decode_gqa_fp16
 * (flash_attn_kernel.cu:3516-3584).
 */
int fa_paged_decode_gqa_fp16(const void* q, const void* k_cache,
                             const void* v_cache, void* o,
                             const int32_t* block_table,
                             int64_t block_table_numel,
                             const int32_t* seq_lens, int B, int H_Q, int H_KV,
                             int D, int num_pages, int max_num_blocks,
                             void* workspace, size_t workspace_bytes,
                             void* stream);

/*
 * INT8 GQA decode: Q and K quantized to int8 (clamp(round(x / scale), +-127)),
 * integer dot products, score = dot * q_s * k_s / sqrt(D); V stays fp16.
 *   q/o [B, H_Q, 1, D], k/v [B, H_KV, N, D] fp16; q_scale float32 [B * H_Q];
 *   k_scale float32, read as flat[b * H_KV + h_kv] (the reference kernel's own
 *   indexing); keys j > cache_len always masked; 0 <= cache_len < N.
 * Replaces the launch in flash_attn_forward_decode_int8_gqa
 * (flash_attn_kernel.cu:2941-3003).
 */
int fa_decode_int8_gqa(const void* q, const void* k, const void* v, void* o,
                       const float* q_scale, const float* k_scale, int B,
                       int H_Q, int H_KV, int N, int D, int cache_len,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * KV-cache token eviction.  Per batch row b, the num_evict tokens with the
 * lowest attn_scores[b, :] (ties: lower index first, i.e. a stable ascending
 * sort) are dropped; the kept K/V rows of every KV head are written, in their
 * original order, to the front of k_out/v_out and the remaining rows are
 * zero.  keep_mask int32 [B, N] receives 1 for kept and 0 for evicted tokens.
 *   k/v/k_out/v_out fp16 [B, H_KV, N, D], attn_scores fp32 [B, N], N <= 1024;
 *   num_evict <= 0 keeps all, >= N drops all.  Scores with NaN are outside
 *   the contract.  One launch on `stream`.
 * Replaces token_eviction_forward (flash_attn_kernel.cu:4296-4344), kernel
 * token_eviction_kernel (:4223-4294).
 */
int fa_token_eviction(const void* k, const void* v, const float* attn_scores,
                      void* k_out, void* v_out, int32_t* keep_mask, int B,
                      int H_KV, int N, int D, int num_evict, void* stream);

/*
 * Speculative-decoding verification, one batch row per workgroup.
 *   target_probs fp32 [B, K+1, V], draft_probs fp32 [B, K, V], draft_tokens
 *   int64 [B, K], random_vals fp32 [B, K]; 1 <= K <= 8.  Writes
 *   accepted_count int32 [B] and every element of output_tokens int64 [B, K+1]:
 *   accepted draft tokens; at the first rejection i the residual sample
 *   (max(target - draft, 0) normalised, or target itself when that is all
 *   zero), the bonus token from target row i+1 and -1 after it; with no
 *   rejection the bonus from target row K.  Every running sum is accumulated
 *   serially in fp32 in vocabulary order, as the reference does; divisions are
 *   IEEE fp32.  Draft token ids outside [0, V) count as probability 0.
 * Replaces speculative_verify_forward (flash_attn_kernel.cu:3972-4018), kernel
 * speculative_verify_kernel (:3853-3970).
 */
int fa_speculative_verify(const float* target_probs, const float* draft_probs,
                          const int64_t* draft_tokens, const float* random_vals,
                          int32_t* accepted_count, int64_t* output_tokens, int B,
                          int K, int vocab_size, void* stream);

/*
 * Tensor-parallel head-range copies (same device).
 *   full fp16 [B, total_heads, N, D], local fp16 [B, head_count, N, D];
 *   0 <= head_start, 0 <= head_count, head_start + head_count <= total_heads.
 *   fa_scatter_heads: local[b, h] = full[b, head_start + h];
 *   fa_gather_heads:  full[b, head_start + h] = local[b, h] (other heads of
 *   full untouched).  An empty range (head_count, B, N or D zero) is a no-op.
 * Replace scatter_heads_forward (flash_attn_kernel.cu:678-719, kernel
 * scatter_heads_kernel :622-648) and gather_heads_forward (:721-762, kernel
 * gather_heads_kernel :650-676).
 */
int fa_scatter_heads(const void* full, void* local, int B, int total_heads,
                     int head_start, int head_count, int N, int D,
                     void* stream);
int fa_gather_heads(void* full, const void* local, int B, int total_heads,
                    int head_start, int head_count, int N, int D,
                    void* stream);

/*
 * fp16 accumulate of the tensor-parallel all-reduce (same device):
 *   dst[i] = half(float(dst[i]) + float(src[i])) for i < n, rounded to nearest
 *   even once; src == dst doubles dst; partially overlapping buffers are
 *   outside the contract.
 * Replaces cross_gpu_allreduce_fp16 (flash_attn_kernel.cu:597-620, kernel
 * cross_gpu_reduce_kernel :586-595).
 */
int fa_cross_gpu_allreduce_fp16(void* dst, const void* src, size_t n,
                                void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* FLASH_ATTN_MI355X_H */
