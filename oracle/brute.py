"""Pure-Python fp64 loop restatement of the reference kernels (TEST INFRASTRUCTURE ONLY).

An independent second restatement used only to pin ``oracle/attention.py`` on
tiny inputs.  Where ``attention.py`` writes each entry point as a closed-form
masked softmax, this module walks the reference kernels' own loop structure:
the launch grid (which rows get a thread at all), the KV tile loop, the
``-FLT_MAX`` mask sentinel, the online-softmax state ``(m_i, l_i, acc)`` and the
final ``acc / l_i`` (which is 0/0 = NaN when no key survived).  A plausible
mistake in either restatement (a wrong mask bound, a transposed GQA map, a
page-address slip, an off-by-one in the varlen grid) makes the two disagree.

Inputs are nested Python lists or torch tensors (converted with ``.tolist()``);
use only for shapes of a few thousand elements.
"""
from __future__ import annotations

import math
import struct

FLT_MAX = 3.4028234663852886e38
PAGE = 16  # PAGE_BLOCK_SIZE (flash_attn_kernel.cu:3389)


def _tolist(x):
    return x.tolist() if hasattr(x, "tolist") else x


def _online_attend(qvec, key_rows, val_rows, masked, scale, tile):
    """Reference online-softmax loop over keys in tiles of ``tile``
    (e.g. flash_attn_kernel.cu:1196-1282): per tile, masked scores are the
    ``-FLT_MAX`` sentinel and are skipped; a tile with every score masked is
    skipped entirely; output is ``acc / l`` (NaN when l == 0)."""
    d = len(qvec)
    m_i, l_i = -FLT_MAX, 0.0
    acc = [0.0] * d
    n = len(key_rows)
    for start in range(0, n, tile):
        idx = range(start, min(start + tile, n))
        scores = []
        for j in idx:
            if masked(j):
                scores.append(-FLT_MAX)
            else:
                scores.append(sum(qvec[t] * key_rows[j][t] for t in range(d)) * scale)
        m_blk = max(scores) if scores else -FLT_MAX
        if m_blk == -FLT_MAX:
            continue
        m_new = max(m_i, m_blk)
        alpha = 0.0 if m_i == -FLT_MAX else math.exp(m_i - m_new)
        w = [0.0] * d
        beta = 0.0
        for s, j in zip(scores, idx):
            if s == -FLT_MAX:
                continue
            p = math.exp(s - m_new)
            beta += p
            for t in range(d):
                w[t] += val_rows[j][t] * p
        acc = [alpha * acc[t] + w[t] for t in range(d)]
        l_i = alpha * l_i + beta
        m_i = m_new
    if l_i == 0.0:
        return [float("nan")] * d
    return [a / l_i for a in acc]


def prefill(q, k, v, causal):
    """a1/a2: grid (B*H_Q, ceil(N/32)), one query row per thread, keys 0..N-1,
    causal masks k_idx > q_idx (flash_attn_kernel.cu:1223), GQA map :2489."""
    q, k, v = _tolist(q), _tolist(k), _tolist(v)
    b_, hq, n, d = len(q), len(q[0]), len(q[0][0]), len(q[0][0][0])
    hkv = len(k[0])
    scale = 1.0 / math.sqrt(d)
    out = [[[None] * n for _ in range(hq)] for _ in range(b_)]
    for b in range(b_):
        for h in range(hq):
            g = h // (hq // hkv)
            for i in range(n):
                out[b][h][i] = _online_attend(q[b][h][i], k[b][g], v[b][g],
                                              lambda j, i=i: causal and j > i, scale, 32)
    return out


def decode(q, k, v, causal, cache_len):
    """a3/a4: one (b, h_q) per block, keys 0..N-1 in tiles of 64, causal masks
    k_idx > cache_len (flash_attn_kernel.cu:1719)."""
    q, k, v = _tolist(q), _tolist(k), _tolist(v)
    b_, hq, d = len(q), len(q[0]), len(q[0][0][0])
    hkv = len(k[0])
    scale = 1.0 / math.sqrt(d)
    out = [[None] * hq for _ in range(b_)]
    for b in range(b_):
        for h in range(hq):
            g = h // (hq // hkv)
            out[b][h] = [_online_attend(q[b][h][0], k[b][g], v[b][g],
                                        lambda j: causal and j > cache_len, scale, 64)]
    return out


def continuous_batching(q, k, v, cache_lens, causal):
    """a5: current_N = min(cache_len+1, max_N) rows read (continuous_batching_kernel.cu:66-69),
    causal masks k_idx > cache_len (:122)."""
    q, k, v, cl = _tolist(q), _tolist(k), _tolist(v), _tolist(cache_lens)
    b_, hq, d = len(q), len(q[0]), len(q[0][0][0])
    hkv, max_n = len(k[0]), len(k[0][0])
    scale = 1.0 / math.sqrt(d)
    out = [[None] * hq for _ in range(b_)]
    for b in range(b_):
        c = cl[b]
        cur = min(c + 1, max_n)
        for h in range(hq):
            g = h // (hq // hkv)
            rows_k = k[b][g][:max(cur, 0)]
            rows_v = v[b][g][:max(cur, 0)]
            out[b][h] = [_online_attend(q[b][h][0], rows_k, rows_v,
                                        lambda j, c=c: causal and j > c, scale, 64)]
    return out


def paged_decode(q, k_cache, v_cache, block_table, seq_lens, max_num_blocks):
    """a7: page loop with physical = block_table[b*max_num_blocks + i]
    (flash_attn_kernel.cu:3438), element ((phys*H_KV + h_kv)*16 + row)*D + col
    computed on the flattened cache (:3418, :3446)."""
    q = _tolist(q)
    bt = [x for row in _tolist(block_table) for x in row]
    sl = _tolist(seq_lens)
    kc, vc = k_cache.reshape(-1).tolist(), v_cache.reshape(-1).tolist()
    hkv, d = k_cache.shape[1], k_cache.shape[3]
    b_, hq = len(q), len(q[0])
    scale = 1.0 / math.sqrt(d)
    out = [[None] * hq for _ in range(b_)]
    for b in range(b_):
        n = sl[b]
        for h in range(hq):
            g = h // (hq // hkv)
            rows_k, rows_v = [], []
            for t in range(max(n, 0)):
                phys = bt[b * max_num_blocks + t // PAGE]
                base = ((phys * hkv + g) * PAGE + t % PAGE) * d
                rows_k.append(kc[base:base + d])
                rows_v.append(vc[base:base + d])
            out[b][h] = [_online_attend(q[b][h][0], rows_k, rows_v, lambda j: False, scale, PAGE)]
    return out


def varlen_prefill(q, k, v, cu_seqlens, max_seqlen, causal):
    """a6: grid (ceil(max_seqlen/T), H, batch) with T = 32 (D<=128) or 8 (D>128)
    (flash_attn_kernel.cu:3319-3338); thread rows q_start+tid inside [cu[b], cu[b+1]);
    keys of the same sequence; causal k_idx > q_idx in packed coordinates (:3087).
    Rows never visited keep the output's initial zeros (:3382)."""
    q, k, v, cu = _tolist(q), _tolist(k), _tolist(v), _tolist(cu_seqlens)
    total, h_, d = len(q), len(q[0]), len(q[0][0])
    tile = 32 if d <= 128 else 8
    scale = 1.0 / math.sqrt(d)
    out = [[[0.0] * d for _ in range(h_)] for _ in range(total)]
    n_tiles = (max_seqlen + tile - 1) // tile
    for b in range(len(cu) - 1):
        s, e = cu[b], cu[b + 1]
        if e - s == 0:
            continue
        for h in range(h_):
            keys = [k[r][h] for r in range(s, e)] if e > s else []
            vals = [v[r][h] for r in range(s, e)] if e > s else []
            for t in range(n_tiles):
                for tid in range(tile):
                    qi = s + t * tile + tid
                    if qi >= e:
                        continue
                    out[qi][h] = _online_attend(q[qi][h], keys, vals,
                                                lambda j, qi=qi: causal and (s + j) > qi, scale, 32)
    return out


def _roundf(x):
    """C roundf (half away from zero)."""
    return math.copysign(math.floor(abs(x) + 0.5), x)


def _quant(x, inv):
    y = x * inv
    if y != y:  # NaN: fminf(127, NaN) = 127, fmaxf(-127, 127) = 127
        return 127
    return int(max(-127.0, min(127.0, _roundf(y))))


def decode_int8(q, k, v, q_scale, k_scale, cache_len):
    """a8 (flash_attn_kernel.cu:2796-2939): integer dot of clamp(roundf(x*inv_s))
    codes, score = dot*q_s*k_s*scale (:2888), k_s = k_scale.flat[b*H_KV+h_kv]
    (:2825), keys k_idx > cache_len always masked (:2866), V in fp16.
    ``inv_s`` is the float32 reciprocal of the scale (see oracle.attention.quantize_int8)."""
    import numpy as np

    q, k, v = _tolist(q), _tolist(k), _tolist(v)
    qs = q_scale.reshape(-1).tolist()
    ks_flat = k_scale.reshape(-1).tolist()
    b_, hq, d = len(q), len(q[0]), len(q[0][0][0])
    hkv = len(k[0])
    f32 = np.float32
    scale = f32(1.0) / np.sqrt(f32(d))  # 1.0f / std::sqrt((float)D) (flash_attn_kernel.cu:2983)
    out = [[None] * hq for _ in range(b_)]
    for b in range(b_):
        for h in range(hq):
            g = h // (hq // hkv)
            q_s = f32(qs[b * hq + h])
            k_s = f32(ks_flat[b * hkv + g])
            inv_q = float(f32(1.0) / q_s)
            inv_k = float(f32(1.0) / k_s)
            qi = [_quant(float(f32(x) * f32(inv_q)), 1.0) for x in q[b][h][0]]
            n = len(k[b][g])
            rows = []
            for j in range(n):
                kj = [_quant(float(f32(x) * f32(inv_k)), 1.0) for x in k[b][g][j]]
                rows.append(kj)
            # scores in float32 in the reference's multiplication order
            sc = []
            for j in range(n):
                dot = sum(a * c for a, c in zip(qi, rows[j]))
                sc.append(float(f32(dot) * q_s * k_s * scale))
            m = max(sc[j] for j in range(n) if j <= cache_len)
            p = [math.exp(sc[j] - m) if j <= cache_len else 0.0 for j in range(n)]
            l_ = sum(p)
            out[b][h] = [[sum(p[j] * v[b][g][j][t] for j in range(n)) / l_ for t in range(d)]]
    return out


def decode_sliding_window(q, k, v, cache_len, window_size, sink_size):
    """forward_decode_sliding_window_gqa kernel (flash_attn_kernel.cu:4346-4482): keys
    0..N-1 in tiles of 64; key j kept iff j < sink_size or window_start <= j <= cache_len,
    window_start = max(0, min(cache_len + 1, N) - window_size) (:4386-4387, :4413-4416)."""
    q, k, v = _tolist(q), _tolist(k), _tolist(v)
    b_, hq, d = len(q), len(q[0]), len(q[0][0][0])
    hkv, n = len(k[0]), len(k[0][0])
    scale = 1.0 / math.sqrt(d)
    eff_end = min(cache_len + 1, n)
    wstart = max(0, eff_end - window_size)
    out = [[None] * hq for _ in range(b_)]
    for b in range(b_):
        for h in range(hq):
            g = h // (hq // hkv)
            out[b][h] = [_online_attend(
                q[b][h][0], k[b][g], v[b][g],
                lambda j: not (j < sink_size or (wstart <= j <= cache_len)), scale, 64)]
    return out


def _to_half(x):
    """Round to the nearest fp16 value, ties to even (IEEE binary16 packing)."""
    return struct.unpack("<e", struct.pack("<e", x))[0]


def decode_int8_kv_cache(q, k_i8, v_i8, k_scale, v_scale, cache_len):
    """forward_decode_int8_kv_cache_gqa kernel (flash_attn_kernel.cu:4020-4159): each
    element dequantized to half(x * scale[token]) in the tile load (:4083-4086), keys
    j > cache_len masked (:4094), online softmax over tiles of 64."""
    q, k_i8, v_i8 = _tolist(q), _tolist(k_i8), _tolist(v_i8)
    k_scale, v_scale = _tolist(k_scale), _tolist(v_scale)
    b_, hq, d = len(q), len(q[0]), len(q[0][0][0])
    hkv, n = len(k_i8[0]), len(k_i8[0][0])
    scale = 1.0 / math.sqrt(d)
    out = [[None] * hq for _ in range(b_)]
    for b in range(b_):
        kd = [[[_to_half(float(k_i8[b][g][j][t]) * float(k_scale[b][g][j])) for t in range(d)]
               for j in range(n)] for g in range(hkv)]
        vd = [[[_to_half(float(v_i8[b][g][j][t]) * float(v_scale[b][g][j])) for t in range(d)]
               for j in range(n)] for g in range(hkv)]
        for h in range(hq):
            g = h // (hq // hkv)
            out[b][h] = [_online_attend(q[b][h][0], kd[g], vd[g], lambda j: j > cache_len, scale, 64)]
    return out


def prefill_lse(q, k, v, causal):
    """forward_with_lse / forward_fp16_with_lse: the fp32 kernel's loop
    (flash_attn_kernel.cu:421-504, tiles of TILE_K=32) keeping ``m_i`` and
    ``l_i``; LSE = m_i + log(l_i) (:502-504).  Returns (out, lse) as nested lists
    [B][H][N][D] and [B][H][N]."""
    q, k, v = _tolist(q), _tolist(k), _tolist(v)
    B, H, N, D = len(q), len(q[0]), len(q[0][0]), len(q[0][0][0])
    scale = 1.0 / math.sqrt(D)
    out, lse = [], []
    for b in range(B):
        ob, lb = [], []
        for h in range(H):
            oh, lh = [], []
            for i in range(N):
                m_i, l_i = -FLT_MAX, 0.0
                acc = [0.0] * D
                for start in range(0, N, 32):
                    js = [j for j in range(start, min(start + 32, N)) if not (causal and j > i)]
                    if not js:
                        continue
                    sc = {j: sum(q[b][h][i][t] * k[b][h][j][t] for t in range(D)) * scale for j in js}
                    m_new = max(m_i, max(sc.values()))
                    alpha = 0.0 if m_i == -FLT_MAX else math.exp(m_i - m_new)
                    acc = [alpha * a for a in acc]
                    l_i *= alpha
                    for j in js:
                        p = math.exp(sc[j] - m_new)
                        l_i += p
                        for t in range(D):
                            acc[t] += p * v[b][h][j][t]
                    m_i = m_new
                oh.append([a / l_i for a in acc])
                lh.append(m_i + math.log(l_i))
            ob.append(oh)
            lb.append(lh)
        out.append(ob)
        lse.append(lb)
    return out, lse


def backward(dout, q, k, v, out, lse, causal):
    """backward: the reference's one-thread-per-(query, key) kernel
    (flash_attn_kernel.cu:2056-2111) as a loop over (b, h, i, j) with the
    atomicAdd accumulations as +=.  Returns (dq, dk, dv) nested lists."""
    dout, q, k, v, out, lse = (_tolist(x) for x in (dout, q, k, v, out, lse))
    B, H, N, D = len(q), len(q[0]), len(q[0][0]), len(q[0][0][0])
    scale = 1.0 / math.sqrt(D)
    zeros = lambda: [[[[0.0] * D for _ in range(N)] for _ in range(H)] for _ in range(B)]
    dq, dk, dv = zeros(), zeros(), zeros()
    for b in range(B):
        for h in range(H):
            for i in range(N):
                for j in range(N):
                    if causal and j > i:
                        continue
                    qi, kj, vj = q[b][h][i], k[b][h][j], v[b][h][j]
                    doi, oi = dout[b][h][i], out[b][h][i]
                    score = sum(qi[t] * kj[t] for t in range(D))
                    do_dot_v = sum(doi[t] * vj[t] for t in range(D))
                    delta = sum(doi[t] * oi[t] for t in range(D))
                    p = math.exp(score * scale - lse[b][h][i])
                    ds = p * (do_dot_v - delta) * scale
                    for t in range(D):
                        dq[b][h][i][t] += ds * kj[t]
                        dk[b][h][j][t] += ds * qi[t]
                        dv[b][h][j][t] += p * doi[t]
    return dq, dk, dv


def token_eviction(k, v, attn_scores, num_evict):
    """token_eviction_kernel (flash_attn_kernel.cu:4223-4294) as written: the
    one-thread bubble sort (swap on s[j] > s[j+1]), the mask of the first
    num_evict sorted indices, and the in-order copy of kept rows.  Returns
    nested lists (k_out, v_out, mask)."""
    k, v, sc = _tolist(k), _tolist(v), _tolist(attn_scores)
    B, H, N, D = len(k), len(k[0]), len(k[0][0]), len(k[0][0][0])
    k_out = [[[[0.0] * D for _ in range(N)] for _ in range(H)] for _ in range(B)]
    v_out = [[[[0.0] * D for _ in range(N)] for _ in range(H)] for _ in range(B)]
    masks = []
    for b in range(B):
        s = list(sc[b])
        idx = list(range(N))
        for i in range(N - 1):
            for j in range(N - 1 - i):
                if s[j] > s[j + 1]:
                    s[j], s[j + 1] = s[j + 1], s[j]
                    idx[j], idx[j + 1] = idx[j + 1], idx[j]
        mask = [1] * N
        i = 0
        while i < num_evict and i < N:
            mask[idx[i]] = 0
            i += 1
        masks.append(mask)
        for h in range(H):
            w = 0
            for i in range(N):
                if mask[i]:
                    k_out[b][h][w] = list(k[b][h][i])
                    v_out[b][h][w] = list(v[b][h][i])
                    w += 1
    return k_out, v_out, masks


def speculative_verify(target_probs, draft_probs, draft_tokens, random_vals, K):
    """speculative_verify_kernel (flash_attn_kernel.cu:3853-3970) as written, on
    one thread, with numpy float32 scalars for every fp32 operation.  Returns
    (accepted list, tokens nested list)."""
    import numpy as np

    f = np.float32
    tp = np.asarray(target_probs, dtype=np.float32)
    dp = np.asarray(draft_probs, dtype=np.float32)
    tok = np.asarray(draft_tokens, dtype=np.int64)
    rv = np.asarray(random_vals, dtype=np.float32)
    B, V = tp.shape[0], tp.shape[2]
    accepted, outs = [], []
    for b in range(B):
        out = [-1] * (K + 1)
        s_acc, s_rej = 0, False
        for i in range(K):
            if s_rej:
                break
            t = int(tok[b, i])
            p_tok, q_tok = tp[b, i, t], dp[b, i, t]
            accept_prob = min(f(1.0), f(p_tok / f(q_tok + f(1e-10))))
            r = rv[b, i]
            if r < accept_prob:
                out[i] = t
                s_acc += 1
            else:
                s_rej = True
                Z = f(0.0)
                for v in range(V):
                    diff = f(tp[b, i, v] - dp[b, i, v])
                    if diff > f(0.0):
                        Z = f(Z + diff)
                if Z > f(0.0):
                    r2, cumsum, sampled = rv[b, i], f(0.0), 0
                    for v in range(V):
                        diff = f(tp[b, i, v] - dp[b, i, v])
                        if diff > f(0.0):
                            cumsum = f(cumsum + f(diff / Z))
                            if r2 < cumsum and sampled == 0:
                                sampled = v
                    out[i] = sampled
                else:
                    r2, cum, sampled = rv[b, i], f(0.0), 0
                    for v in range(V):
                        cum = f(cum + tp[b, i, v])
                        if r2 < cum and sampled == 0:
                            sampled = v
                    out[i] = sampled
                for j in range(i + 1, K):
                    out[j] = -1
                bonus_r, cum, bonus = rv[b, min(i, K - 1)], f(0.0), 0
                for v in range(V):
                    cum = f(cum + tp[b, i + 1, v])
                    if cum >= bonus_r and bonus == 0:
                        bonus = v
                out[i + 1] = bonus
                break
        if not s_rej:
            bonus_r, cum, bonus = rv[b, K - 1], f(0.0), 0
            for v in range(V):
                cum = f(cum + tp[b, K, v])
                if cum >= bonus_r and bonus == 0:
                    bonus = v
            out[K] = bonus
        accepted.append(s_acc)
        outs.append(out)
    return accepted, outs
