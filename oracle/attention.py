"""CPU restatement of the reference's attention semantics (TEST INFRASTRUCTURE ONLY).

This module is the checker for the HIP kernels of ``flash_attn_v100_amd``. Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it; the product path never calls it and has no CPU
fallback.

Every function restates one entry point of the reference extension
(``flash_attn_v100``, sources under ``/root/reference``) as plain masked-softmax
attention computed with PyTorch eager math on the CPU::

    O = softmax(Q K^T / sqrt(D) + M) V      (fp16 inputs, fp32/fp64 arithmetic)

The reference kernels are online-softmax loops (``m_i``/``l_i``/``acc``) whose
result is mathematically this closed form; what differs between entry points is
the mask ``M``, the index maps (GQA head mapping, paged address, packed varlen
rows) and the INT8 quantization, which are restated exactly and cited line by
line.  ``compute_dtype`` selects float32 (the CPU baseline; the reference test
scripts' own precision) or float64 (error budgeting).

Pinning: ``tests/test_oracle.py`` checks each function against an independent
pure-Python fp64 loop restatement (``oracle/brute.py``) on tiny inputs, against
closed forms (cache_len=0 -> V[0], identical keys -> mean(V), a dominant key ->
its V row), against invariants (GQA == MHA on repeat-interleaved KV, paged ==
contiguous on the gathered cache, varlen == per-segment prefill, continuous
batching == per-row decode on the truncated cache, a sliding window that
covers every key == plain decode, an INT8 cache with power-of-two scales ==
decode on the exactly dequantized cache) and against the committed fixtures in
``tests/golden/``.
"""
from __future__ import annotations

import math

import torch

# Page size of the paged KV cache: ``PAGE_BLOCK_SIZE = 16`` (flash_attn_kernel.cu:3389).
PAGE_BLOCK_SIZE = 16
# Query-tile heights of the reference varlen kernels; they decide which packed
# rows are ever written (flash_attn_kernel.cu:3336-3338 grid.x = ceil(max_seqlen/32)
# for D<=128, :3319-3320 ceil(max_seqlen/8) for D>128).
VARLEN_TILE_SMALL_D = 32
VARLEN_TILE_LARGE_D = 8
MAX_D_SMALL = 128  # MAX_D (flash_attn_kernel.cu:35)


def host_scale_f32(d: int) -> torch.Tensor:
    """``1.0f / std::sqrt((float)D)`` evaluated in float32 as the host wrappers do
    (e.g. flash_attn_kernel.cu:1944, :2983)."""
    return torch.tensor(1.0, dtype=torch.float32) / torch.sqrt(torch.tensor(float(d), dtype=torch.float32))


def _softmax_rows(scores: torch.Tensor) -> torch.Tensor:
    """Row softmax where a row with no unmasked key yields NaN.

    The reference divides ``acc / l_i`` with ``l_i == 0`` and ``acc == 0`` for such
    rows (e.g. flash_attn_kernel.cu:3511), i.e. 0/0 = NaN.  ``torch.softmax``
    over an all ``-inf`` row gives the same NaN.
    """
    return torch.softmax(scores, dim=-1)


def _attend(q, k, v, mask, compute_dtype):
    """q [..., M, D], k/v [..., L, D], mask broadcastable to [..., M, L] (True = masked)."""
    d = q.shape[-1]
    qf = q.to(compute_dtype)
    kf = k.to(compute_dtype)
    vf = v.to(compute_dtype)
    # Scale is 1/sqrt(D), computed on the host (flash_attn_kernel.cu:265, :1944).
    scores = torch.matmul(qf, kf.transpose(-1, -2)) * (1.0 / math.sqrt(d))
    if mask is not None:
        scores = scores.masked_fill(mask, float("-inf"))
    probs = _softmax_rows(scores)
    if probs.shape[-1] == 0:
        return torch.full(probs.shape[:-1] + (d,), float("nan"), dtype=compute_dtype)
    return torch.matmul(probs, vf)


def expand_kv(k: torch.Tensor, h_q: int) -> torch.Tensor:
    """GQA head map ``h_kv = h_q / (H_Q / H_KV)`` (flash_attn_kernel.cu:1662, :2489;
    continuous_batching_kernel.cu:62), i.e. ``repeat_interleave`` on the head dim."""
    h_kv = k.shape[1]
    return k.repeat_interleave(h_q // h_kv, dim=1)


def prefill(q, k, v, causal: bool, compute_dtype=torch.float32):
    """``forward_fp16`` / ``forward_fp16_wmma`` / ``forward_prefill_gqa_fp16``.

    Q [B,H_Q,N,D], K/V [B,H_KV,N,D].  Causal masks key ``k_idx > q_idx`` (square,
    top-left aligned): flash_attn_kernel.cu:1223 (a1), :2364 (a2 WMMA, mask applied
    to the scaled score), :996 (D>128 path).  Non-causal attends all N keys.
    """
    n = q.shape[2]
    k = expand_kv(k, q.shape[1])
    v = expand_kv(v, q.shape[1])
    mask = None
    if causal:
        mask = torch.triu(torch.ones(n, n, dtype=torch.bool), diagonal=1)
    return _attend(q, k, v, mask, compute_dtype)


def decode(q, k, v, causal: bool, cache_len: int, compute_dtype=torch.float32):
    """``forward_decode_fp16`` (H_Q == H_KV) / ``forward_decode_gqa_fp16``.

    Q [B,H_Q,1,D], K/V [B,H_KV,N,D].  Causal masks ``k_idx > cache_len``
    (flash_attn_kernel.cu:1556, :1719, :846); non-causal attends all N rows.
    """
    n = k.shape[2]
    k = expand_kv(k, q.shape[1])
    v = expand_kv(v, q.shape[1])
    mask = None
    if causal:
        mask = (torch.arange(n) > cache_len).view(1, 1, 1, n)
    return _attend(q, k, v, mask, compute_dtype)


def continuous_batching(q, k, v, cache_lens, causal: bool, compute_dtype=torch.float32):
    """``forward_continuous_batching_fp16``.

    Per batch row b only keys ``[0, min(cache_lens[b]+1, max_N))`` are read
    (continuous_batching_kernel.cu:66-69); causal additionally masks
    ``k_idx > cache_lens[b]`` (:122), which cannot fire inside that range, so both
    ``causal`` values give the same result.  An empty range (cache_len < 0) gives
    0/0 = NaN (:192).
    """
    b_, h_q, _, d = q.shape
    max_n = k.shape[2]
    k = expand_kv(k, h_q)
    v = expand_kv(v, h_q)
    lens = torch.as_tensor(cache_lens).to(torch.int64).cpu()
    cur = torch.clamp(lens + 1, max=max_n)
    idx = torch.arange(max_n).view(1, max_n)
    mask = idx >= cur.view(-1, 1)
    if causal:
        mask = mask | (idx > lens.view(-1, 1))
    return _attend(q, k, v, mask.view(b_, 1, 1, max_n), compute_dtype)


def paged_gather(k_cache, v_cache, block_table, seq_lens, max_num_blocks):
    """Gather the paged cache into contiguous [B,H_KV,L,D] tensors plus a length mask.

    Token ``t`` of sequence ``b`` lives at page
    ``block_table.flat[b*max_num_blocks + t/16]``, row ``t%16``, element address
    ``((phys*H_KV + h_kv)*16 + row)*D + col`` (flash_attn_kernel.cu:3418, :3438,
    :3446).  ``max_num_blocks`` is the row stride into the flattened table, exactly
    as the kernel uses it.  Returns (k, v, lens) with L = max(seq_lens, 0).
    """
    bt = block_table.reshape(-1).to(torch.int64).cpu()
    lens = torch.as_tensor(seq_lens).to(torch.int64).cpu()
    b_ = lens.numel()
    h_kv, page, d = k_cache.shape[1], k_cache.shape[2], k_cache.shape[3]
    assert page == PAGE_BLOCK_SIZE
    lmax = max(int(lens.max().item()), 0) if b_ else 0
    k = torch.zeros(b_, h_kv, lmax, d, dtype=k_cache.dtype)
    v = torch.zeros_like(k)
    for b in range(b_):
        n = int(lens[b])
        if n <= 0:
            continue
        t = torch.arange(n)
        phys = bt[b * max_num_blocks + t // PAGE_BLOCK_SIZE]
        row = t % PAGE_BLOCK_SIZE
        k[b, :, :n] = k_cache[phys, :, row].permute(1, 0, 2)
        v[b, :, :n] = v_cache[phys, :, row].permute(1, 0, 2)
    return k, v, lens


def paged_decode(q, k_cache, v_cache, block_table, seq_lens, max_num_blocks,
                 compute_dtype=torch.float32):
    """``forward_paged_decode_gqa_fp16``: attends exactly tokens ``[0, seq_lens[b])``
    of the paged cache (no causal argument, flash_attn_kernel.cu:3432-3490);
    ``seq_lens[b] <= 0`` gives NaN (0/0 at :3511)."""
    k, v, lens = paged_gather(k_cache, v_cache, block_table, seq_lens, max_num_blocks)
    b_, h_q = q.shape[0], q.shape[1]
    lmax = k.shape[2]
    k = expand_kv(k, h_q)
    v = expand_kv(v, h_q)
    mask = torch.arange(lmax).view(1, lmax) >= lens.view(-1, 1)
    return _attend(q, k, v, mask.view(b_, 1, 1, lmax), compute_dtype)


def varlen_row_limit(max_seqlen: int, d: int) -> int:
    """Number of leading rows of each sequence the reference ever writes.

    The grid's x extent is ``ceil(max_seqlen / tile)`` query tiles per sequence
    (flash_attn_kernel.cu:3319-3320 and :3336-3337) with tile 32 for D<=128 and 8
    for D>128, so rows at local index >= ``tile*ceil(max_seqlen/tile)`` stay at the
    zero the output was initialised with (:3382).
    """
    tile = VARLEN_TILE_SMALL_D if d <= MAX_D_SMALL else VARLEN_TILE_LARGE_D
    return ((max_seqlen + tile - 1) // tile) * tile


def varlen_prefill(q, k, v, cu_seqlens, max_seqlen: int, causal: bool,
                   compute_dtype=torch.float32):
    """``forward_varlen_prefill_fp16`` on packed Q/K/V [total, H, D].

    Sequence b spans packed rows ``[cu[b], cu[b+1])`` (flash_attn_kernel.cu:3021-3023);
    its queries attend only keys of the same range (:3061) and causal masks
    ``k_idx > q_idx`` (:3087); empty or negative-length ranges are skipped (:3025,
    :3030); rows beyond :func:`varlen_row_limit` are never written (left 0).
    """
    total, h, d = q.shape
    cu = torch.as_tensor(cu_seqlens).to(torch.int64).cpu()
    out = torch.zeros(total, h, d, dtype=compute_dtype)
    limit = varlen_row_limit(max_seqlen, d)
    for b in range(cu.numel() - 1):
        s, e = int(cu[b]), int(cu[b + 1])
        n = e - s
        if n <= 0:
            continue
        rows = min(n, limit)
        qs = q[s:s + rows].permute(1, 0, 2).unsqueeze(0)  # [1,H,rows,D]
        ks = k[s:e].permute(1, 0, 2).unsqueeze(0)
        vs = v[s:e].permute(1, 0, 2).unsqueeze(0)
        mask = None
        if causal:
            mask = torch.arange(n).view(1, n) > torch.arange(rows).view(rows, 1)
        o = _attend(qs, ks, vs, mask, compute_dtype)[0].permute(1, 0, 2)
        out[s:s + rows] = o
    return out


def round_half_away(x: torch.Tensor) -> torch.Tensor:
    """C ``roundf``: round half away from zero, evaluated in float64 so the
    ``+0.5`` is exact for every float32 input."""
    x64 = x.to(torch.float64)
    return (torch.sign(x64) * torch.floor(torch.abs(x64) + 0.5)).to(x.dtype)


def quantize_int8(x_f16: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """``int8 = clamp(roundf(x / s), -127, 127)`` (flash_attn_kernel.cu:2837, :2856).

    The division is evaluated as ``x * (1/s)`` in float32 with ``1/s`` correctly
    rounded.  That is this oracle's choice, shared with the HIP kernel, so the
    two produce identical integer codes.  The reference divides under
    ``--use_fast_math`` (setup.py:25), whose exact rounding of ``x / s`` is not
    known here: a quotient that lands within one ulp of a rounding tie (k + 0.5)
    may round to the neighbouring code in the reference, so INT8 codes at ties
    are parity-unpinned against the reference (the rel-L2 tolerance covers the
    effect on the output).  Clamping uses fmin/fmax semantics (a NaN quotient
    becomes +127, as ``fmaxf(-127, fminf(127, NaN))`` does).
    """
    inv = (torch.ones_like(s, dtype=torch.float32) / s.to(torch.float32))
    y = x_f16.to(torch.float32) * inv
    r = round_half_away(y)
    r = torch.fmin(torch.full_like(r, 127.0), r)
    r = torch.fmax(torch.full_like(r, -127.0), r)
    return r.to(torch.int32)


def int8_k_scale_per_head(k_scale: torch.Tensor, b_: int, h_kv: int) -> torch.Tensor:
    """The scale the reference kernel actually uses for head (b, h_kv).

    The host requires ``k_scale.shape == [B, H_KV, N]`` (flash_attn_kernel.cu:2970-2971)
    but the kernel reads ``K_scale[b*H_KV + h_kv]`` of the flattened tensor (:2825),
    i.e. element ``b*H_KV + h_kv`` of ``k_scale.reshape(-1)``.
    """
    flat = k_scale.reshape(-1).to(torch.float32)
    return flat[: b_ * h_kv].view(b_, h_kv)


def decode_int8(q, k, v, q_scale, k_scale, cache_len: int, compute_dtype=torch.float32):
    """``forward_decode_int8_gqa`` (flash_attn_kernel.cu:2796-2939).

    1. ``qi = clamp(roundf(q/q_s))`` with ``q_s = q_scale[b, h_q]`` (:2824, :2837).
    2. ``ki = clamp(roundf(k/k_s))`` with ``k_s`` from :func:`int8_k_scale_per_head`.
    3. ``score = (sum_d qi*ki) * q_s * k_s * (1/sqrt(D))`` with an exact integer
       dot (:2871-2888).
    4. Keys ``k_idx > cache_len`` are always masked (:2866).
    5. V stays fp16; softmax and PV in float (:2908-2921).
    """
    b_, h_q, _, d = q.shape
    h_kv, n = k.shape[1], k.shape[2]
    qs = q_scale.reshape(b_, h_q).to(torch.float32)
    ks = int8_k_scale_per_head(k_scale, b_, h_kv)
    qi = quantize_int8(q, qs.view(b_, h_q, 1, 1))                 # [B,H_Q,1,D]
    ki = quantize_int8(k, ks.view(b_, h_kv, 1, 1))                # [B,H_KV,N,D]
    ki = expand_kv(ki, h_q)
    dots = torch.matmul(qi.to(torch.float64), ki.to(torch.float64).transpose(-1, -2))  # exact
    ks_q = ks.repeat_interleave(h_q // h_kv, dim=1)
    # Reference order: (float)int_dot * q_s * k_s * scale, all float32 (:2888).
    scale = host_scale_f32(d)
    scores = dots.to(torch.float32) * qs.view(b_, h_q, 1, 1) * ks_q.view(b_, h_q, 1, 1) * scale
    scores = scores.to(compute_dtype)
    mask = (torch.arange(n) > cache_len).view(1, 1, 1, n)
    scores = scores.masked_fill(mask, float("-inf"))
    probs = _softmax_rows(scores)
    return torch.matmul(probs, expand_kv(v, h_q).to(compute_dtype))


def decode_int8_dequant_reference(q, k, v, q_scale, k_scale, cache_len: int):
    """Quantize-dequantize form of :func:`decode_int8` (float64): attention of the
    dequantized ``qi*q_s`` against ``ki*k_s``.  Equal to :func:`decode_int8` up to
    float rounding; used to check that restatement."""
    b_, h_q, _, d = q.shape
    h_kv = k.shape[1]
    qs = q_scale.reshape(b_, h_q).to(torch.float32)
    ks = int8_k_scale_per_head(k_scale, b_, h_kv)
    qd = quantize_int8(q, qs.view(b_, h_q, 1, 1)).to(torch.float64) * qs.view(b_, h_q, 1, 1).double()
    kd = quantize_int8(k, ks.view(b_, h_kv, 1, 1)).to(torch.float64) * ks.view(b_, h_kv, 1, 1).double()
    return decode(qd, kd, v.double(), True, cache_len, compute_dtype=torch.float64)


def sliding_window_mask(n: int, cache_len: int, window_size: int, sink_size: int) -> torch.Tensor:
    """True where key k is masked for ``forward_decode_sliding_window_gqa``.

    effective_end = min(cache_len + 1, N), window_start = max(0, effective_end -
    window_size) (flash_attn_kernel.cu:4386-4387); key k is kept iff
    ``k < sink_size`` or ``window_start <= k <= cache_len`` (:4413-4416).
    """
    k = torch.arange(n)
    eff_end = min(cache_len + 1, n)
    wstart = max(0, eff_end - window_size)
    keep = (k < sink_size) | ((k >= wstart) & (k <= cache_len))
    return ~keep


def decode_sliding_window(q, k, v, cache_len: int, window_size: int, sink_size: int,
                          compute_dtype=torch.float32):
    """``forward_decode_sliding_window_gqa`` (flash_attn_kernel.cu:4346-4535).

    GQA map as in decode; the ``causal`` argument is unused by the reference;
    no attended key gives 0/0 = NaN.
    """
    n = k.shape[2]
    mask = sliding_window_mask(n, cache_len, window_size, sink_size).view(1, 1, 1, n)
    return _attend(q, expand_kv(k, q.shape[1]), expand_kv(v, q.shape[1]), mask, compute_dtype)


def dequant_int8_cache(x_i8: torch.Tensor, scale_f16: torch.Tensor) -> torch.Tensor:
    """INT8 KV-cache element -> fp16: ``__float2half((float)x * __half2float(scale[token]))``
    (flash_attn_kernel.cu:4083-4086); the fp32 product of an int8 and an fp16 is exact."""
    return (x_i8.to(torch.float32) * scale_f16.to(torch.float32).unsqueeze(-1)).to(torch.float16)


def decode_int8_kv_cache(q, k_i8, v_i8, k_scale, v_scale, cache_len: int,
                         compute_dtype=torch.float32):
    """``forward_decode_int8_kv_cache_gqa`` (flash_attn_kernel.cu:4020-4221).

    K/V int8 [B,H_KV,N,D] with fp16 per-token scales [B,H_KV,N], dequantized to
    fp16 before use; keys ``k > cache_len`` are always masked (:4094, no causal
    flag, cache_len unchecked); no attended key gives NaN.
    """
    n = k_i8.shape[2]
    kd = dequant_int8_cache(k_i8, k_scale)
    vd = dequant_int8_cache(v_i8, v_scale)
    mask = (torch.arange(n) > cache_len).view(1, 1, 1, n)
    return _attend(q, expand_kv(kd, q.shape[1]), expand_kv(vd, q.shape[1]), mask, compute_dtype)


def _causal_mask(n: int) -> torch.Tensor:
    """Square top-left causal mask, True where key > query (flash_attn_kernel.cu:445, :2084)."""
    return torch.triu(torch.ones(n, n, dtype=torch.bool), diagonal=1)


def prefill_lse(q, k, v, causal: bool, compute_dtype=torch.float32):
    """``forward_with_lse`` (fp32) / ``forward_fp16_with_lse`` (fp16): MHA forward
    plus ``LSE[b,h,i] = m_i + log(l_i)`` (flash_attn_kernel.cu:502-504, :1295-1297),
    i.e. the natural-log log-sum-exp of the row's scaled, masked scores.

    Returns ``(out, lse)``; out as :func:`prefill`, lse [B,H,N] in compute_dtype.
    """
    d = q.shape[-1]
    n = q.shape[2]
    scores = torch.matmul(q.to(compute_dtype), k.to(compute_dtype).transpose(-1, -2)) * (1.0 / math.sqrt(d))
    if causal:
        scores = scores.masked_fill(_causal_mask(n), float("-inf"))
    lse = torch.logsumexp(scores, dim=-1)
    out = torch.matmul(torch.exp(scores - lse.unsqueeze(-1)), v.to(compute_dtype))
    return out, lse


def backward(dout, q, k, v, out, lse, causal: bool, compute_dtype=torch.float64):
    """``backward`` (flash_attn_kernel.cu:2173-2264; per-(query, key) kernels :2056-2171).

    Uses the caller's ``out`` and ``lse`` as the reference does (it never
    recomputes them).  For every unmasked pair (i, j) (causal masks j > i,
    :2084):
        p_ij   = exp(scale * q_i . k_j - LSE_i)                 (:2103)
        delta_i = dO_i . O_i,   ds_ij = p_ij (dO_i . v_j - delta_i) scale   (:2104)
        dQ_i += ds_ij k_j,  dK_j += ds_ij q_i,  dV_j += p_ij dO_i    (:2106-2110)
    Returns ``(dq, dk, dv)`` in compute_dtype.
    """
    cd = compute_dtype
    d = q.shape[-1]
    n = q.shape[2]
    scale = 1.0 / math.sqrt(d)
    qf, kf, vf, dof, of = (t.to(cd) for t in (q, k, v, dout, out))
    s = torch.matmul(qf, kf.transpose(-1, -2)) * scale
    p = torch.exp(s - lse.to(cd).unsqueeze(-1))
    if causal:
        p = p.masked_fill(_causal_mask(n), 0.0)
    delta = (dof * of).sum(-1, keepdim=True)
    dp = torch.matmul(dof, vf.transpose(-1, -2))
    ds = p * (dp - delta) * scale
    dq = torch.matmul(ds, kf)
    dk = torch.matmul(ds.transpose(-1, -2), qf)
    dv = torch.matmul(p.transpose(-1, -2), dof)
    return dq, dk, dv


def token_eviction(k, v, attn_scores, num_evict: int):
    """``token_eviction`` (flash_attn_kernel.cu:4223-4344).

    Per batch row, the reference bubble-sorts the scores ascending, swapping
    only on ``s[j] > s[j+1]`` (:4258-4270, a stable sort), marks the first
    ``num_evict`` sorted tokens evicted (:4272-4277), and copies the kept K/V
    rows of every head, in order, to the front of zero-filled outputs
    (:4281-4293; outputs are ``zeros_like``, :4317-4318).  Returns
    ``(k_out, v_out, valid_mask)`` with valid_mask int32 [B, N].
    """
    B, H, N, D = k.shape
    order = torch.sort(attn_scores, dim=1, stable=True).indices
    mask = torch.ones(B, N, dtype=torch.int32)
    ne = max(0, min(int(num_evict), N))
    k_out = torch.zeros_like(k)
    v_out = torch.zeros_like(v)
    for b in range(B):
        mask[b, order[b, :ne]] = 0
        kept = torch.nonzero(mask[b], as_tuple=False).flatten()
        k_out[b, :, :kept.numel()] = k[b, :, kept]
        v_out[b, :, :kept.numel()] = v[b, :, kept]
    return k_out, v_out, mask


def _first_index_quirk(cond) -> int:
    """The reference's ``if (cond_v && tok == 0) tok = v`` scan over v ascending
    (flash_attn_kernel.cu:3914-3918, :3924-3928, :3939-3942, :3960-3964): the first
    index where cond holds, except that a hit at v = 0 leaves ``tok == 0`` and so
    is replaced by the next hit; no hit gives 0."""
    import numpy as np

    hits = np.flatnonzero(cond)
    if hits.size == 0:
        return 0
    if hits[0] != 0:
        return int(hits[0])
    return int(hits[1]) if hits.size > 1 else 0


def speculative_verify(target_probs, draft_probs, draft_tokens, random_vals, K: int):
    """``speculative_verify`` (flash_attn_kernel.cu:3853-4018), one batch row at a time.

    fp32 throughout, with every running sum accumulated serially in index
    order as the reference's single thread does (numpy ``cumsum`` is a serial
    float32 accumulation): for i < K accept draft token t when
    ``r_i < fminf(1, p/(q + 1e-10f))`` (:3885-3893); at the first rejection
    sample from max(target - draft, 0) / Z with r_i (:3900-3919; from target
    itself when Z == 0, :3920-3930), write -1 after it (:3933-3935) and a bonus
    token from target row i+1 with r_i (:3937-3945); with no rejection the bonus
    comes from target row K with r_{K-1} (:3953-3965).  Divisions are IEEE fp32
    (the reference's fast-math build rounds them approximately; parity at that
    rounding boundary is unpinned).  Returns (accepted int32 [B], tokens int64 [B, K+1]).
    """
    import numpy as np

    tp = target_probs.detach().cpu().numpy().astype(np.float32)
    dp = draft_probs.detach().cpu().numpy().astype(np.float32)
    tok = draft_tokens.detach().cpu().numpy().astype(np.int64)
    rv = random_vals.detach().cpu().numpy().astype(np.float32)
    B = tp.shape[0]
    one, eps = np.float32(1.0), np.float32(1e-10)
    accepted = np.zeros(B, dtype=np.int32)
    out = np.full((B, K + 1), -1, dtype=np.int64)
    for b in range(B):
        acc, rejected = 0, False
        for i in range(K):
            t = int(tok[b, i])
            p_tok, q_tok = tp[b, i, t], dp[b, i, t]
            accept = min(one, np.float32(p_tok / np.float32(q_tok + eps)))
            r = rv[b, i]
            if r < accept:
                out[b, i] = t
                acc += 1
                continue
            rejected = True
            diff = (tp[b, i] - dp[b, i]).astype(np.float32)
            pos = diff > 0
            Z = np.cumsum(np.where(pos, diff, np.float32(0)), dtype=np.float32)[-1]
            if Z > 0:
                terms = np.where(pos, (diff / Z).astype(np.float32), np.float32(0))
                cs = np.cumsum(terms, dtype=np.float32)
                out[b, i] = _first_index_quirk(pos & (r < cs))
            else:
                cs = np.cumsum(tp[b, i], dtype=np.float32)
                out[b, i] = _first_index_quirk(r < cs)
            out[b, i + 1:K] = -1
            cs = np.cumsum(tp[b, i + 1], dtype=np.float32)
            out[b, i + 1] = _first_index_quirk(cs >= rv[b, min(i, K - 1)])
            break
        if not rejected:
            cs = np.cumsum(tp[b, K], dtype=np.float32)
            out[b, K] = _first_index_quirk(cs >= rv[b, K - 1])
        accepted[b] = acc
    return torch.from_numpy(accepted), torch.from_numpy(out)


def _head_range_index(B: int, total_heads: int, head_start: int, head_count: int, N: int, D: int):
    """Flat (local_idx, full_idx) pairs of the reference's per-element index map
    (flash_attn_kernel.cu:632-647 scatter, :660-675 gather): element ``idx`` of
    the local tensor is ``b = idx // (count*N*D)``, ``local_h = rem1 // (N*D)``,
    ``rem2 = rem1 % (N*D)`` and maps to ``full_idx = b*total*N*D +
    (local_h + start)*N*D + rem2`` when ``local_h + start < total``."""
    import numpy as np

    eph = N * D
    n_local = B * head_count * eph
    idx = np.arange(n_local, dtype=np.int64)
    if n_local == 0:
        return idx, idx
    b = idx // (head_count * eph)
    rem1 = idx % (head_count * eph)
    local_h = rem1 // eph
    rem2 = rem1 % eph
    global_h = local_h + head_start
    keep = global_h < total_heads
    full_idx = b * total_heads * eph + global_h * eph + rem2
    return idx[keep], full_idx[keep]


def scatter_heads(full, local, total_heads: int, head_start: int, head_count: int):
    """``scatter_heads`` (flash_attn_kernel.cu:622-648, :678-719): returns the new
    ``local`` with ``local.flat[idx] = full.flat[full_idx]`` over the reference's
    index map; elements the map does not reach keep their value."""
    B, _, N, D = full.shape
    li, fi = _head_range_index(B, total_heads, head_start, head_count, N, D)
    out = local.detach().cpu().clone().reshape(-1)
    out[torch.from_numpy(li)] = full.detach().cpu().reshape(-1)[torch.from_numpy(fi)]
    return out.reshape(local.shape)


def gather_heads(full, local, total_heads: int, head_start: int, head_count: int):
    """``gather_heads`` (flash_attn_kernel.cu:650-676, :721-762): returns the new
    ``full`` with ``full.flat[full_idx] = local.flat[idx]``; other heads untouched."""
    B, _, N, D = full.shape
    li, fi = _head_range_index(B, total_heads, head_start, head_count, N, D)
    out = full.detach().cpu().clone().reshape(-1)
    out[torch.from_numpy(fi)] = local.detach().cpu().reshape(-1)[torch.from_numpy(li)]
    return out.reshape(full.shape)


def allreduce_fp16(dst, src):
    """``cross_gpu_allreduce_fp16`` (flash_attn_kernel.cu:586-595, :597-620):
    ``dst[i] = __float2half(__half2float(dst[i]) + __half2float(src[i]))`` --
    widen, one fp32 add (round to nearest even), one narrowing (round to nearest
    even).  Returns the new dst."""
    import numpy as np

    a = dst.detach().cpu().numpy().astype(np.float16).astype(np.float32)
    b = src.detach().cpu().numpy().astype(np.float16).astype(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        s = (a + b).astype(np.float32).astype(np.float16)
    return torch.from_numpy(s).reshape(dst.shape)
