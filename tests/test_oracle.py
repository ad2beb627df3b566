"""Pins the CPU oracle (oracle/attention.py) before it is trusted as the checker.

Each oracle function is checked against
  * the independent fp64 loop restatement of the reference kernels (oracle/brute.py),
  * closed forms that the mathematics fixes (cache_len=0, identical keys,
    a dominant key, exactly representable INT8 codes, roundf ties),
  * invariants between entry points (GQA == expanded MHA, paged == gathered
    contiguous decode, varlen == per-segment prefill, continuous batching ==
    per-row decode on the truncated cache),
  * the committed fixtures in tests/golden/ (written by tests/golden/make_golden.py
    from the brute-force restatement).
The reference ships no golden vectors of its own (its tests compare against
torch on the same GPU), so these are the pins.
"""
import os
import math

import pytest
import torch

from oracle import attention as A
from oracle import brute as Bt
from tests.helpers import randn

F64 = torch.float64
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def t64(x):
    return torch.tensor(x, dtype=F64)


def close(a, b, tol=1e-9):
    a, b = torch.as_tensor(a, dtype=F64), torch.as_tensor(b, dtype=F64)
    assert a.shape == b.shape, (a.shape, b.shape)
    assert torch.equal(torch.isnan(a), torch.isnan(b))
    m = ~torch.isnan(a)
    if m.any():
        assert (a[m] - b[m]).abs().max().item() < tol


# ---------------------------------------------------------------- vs brute force

@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("hq,hkv,n,d", [(2, 2, 7, 8), (4, 2, 5, 8), (4, 1, 33, 4)])
def test_prefill_vs_brute(causal, hq, hkv, n, d):
    g = torch.Generator().manual_seed(1)
    q, k, v = randn(g, 2, hq, n, d), randn(g, 2, hkv, n, d), randn(g, 2, hkv, n, d)
    close(A.prefill(q, k, v, causal, F64), t64(Bt.prefill(q.double(), k.double(), v.double(), causal)))


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("cache_len", [0, 5, 69])
def test_decode_vs_brute(causal, cache_len):
    g = torch.Generator().manual_seed(2)
    q, k, v = randn(g, 2, 4, 1, 8), randn(g, 2, 2, 70, 8), randn(g, 2, 2, 70, 8)
    close(A.decode(q, k, v, causal, cache_len, F64),
          t64(Bt.decode(q.double(), k.double(), v.double(), causal, cache_len)))


@pytest.mark.parametrize("causal", [True, False])
def test_continuous_batching_vs_brute(causal):
    g = torch.Generator().manual_seed(3)
    q, k, v = randn(g, 5, 4, 1, 8), randn(g, 5, 2, 17, 8), randn(g, 5, 2, 17, 8)
    cl = torch.tensor([0, 3, 15, 40, -1], dtype=torch.int32)  # last: empty range -> NaN
    ref = t64(Bt.continuous_batching(q.double(), k.double(), v.double(), cl, causal))
    out = A.continuous_batching(q, k, v, cl, causal, F64)
    close(out, ref)
    assert torch.isnan(out[4]).all() and not torch.isnan(out[:4]).any()


def _paged_case(seed=2025, seq_lens=(16, 23, 33), order=(5, 2, 7, 1, 9, 3), hq=8, hkv=4, d=16):
    """The reference's paged test layout (test_decode.py:22-44, :269-297)."""
    g = torch.Generator().manual_seed(seed)
    b = len(seq_lens)
    lmax = max(seq_lens)
    q, k, v = randn(g, b, hq, 1, d), randn(g, b, hkv, lmax, d), randn(g, b, hkv, lmax, d)
    mnb = max((s + 15) // 16 for s in seq_lens)
    npages = max(order) + 1
    kc = torch.zeros(npages, hkv, 16, d, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    bt = torch.full((b, mnb), -1, dtype=torch.int32)
    cur = 0
    for i, s in enumerate(seq_lens):
        for blk in range((s + 15) // 16):
            p = order[cur]
            cur += 1
            bt[i, blk] = p
            st, en = blk * 16, min(blk * 16 + 16, s)
            kc[p, :, : en - st] = k[i, :, st:en]
            vc[p, :, : en - st] = v[i, :, st:en]
    return q, k, v, kc, vc, bt, torch.tensor(seq_lens, dtype=torch.int32), mnb


def test_paged_vs_brute_and_contiguous():
    q, k, v, kc, vc, bt, sl, mnb = _paged_case()
    out = A.paged_decode(q, kc, vc, bt, sl, mnb, F64)
    close(out, t64(Bt.paged_decode(q.double(), kc.double(), vc.double(), bt, sl, mnb)))
    # invariant: paged == contiguous decode on each sequence's first seq_len keys
    for i, s in enumerate(sl.tolist()):
        ref = A.decode(q[i:i + 1], k[i:i + 1, :, :s], v[i:i + 1, :, :s], False, 0, F64)
        close(out[i:i + 1], ref)


def test_paged_empty_sequence_is_nan():
    q, k, v, kc, vc, bt, sl, mnb = _paged_case()
    sl = torch.tensor([16, 0, 33], dtype=torch.int32)
    out = A.paged_decode(q, kc, vc, bt, sl, mnb, F64)
    assert torch.isnan(out[1]).all() and not torch.isnan(out[0]).any()
    close(out, t64(Bt.paged_decode(q.double(), kc.double(), vc.double(), bt, sl, mnb)))


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("d,max_seqlen", [(8, 40), (8, 20), (136, 20)])
def test_varlen_vs_brute(causal, d, max_seqlen):
    """max_seqlen below the longest sequence exercises the rows-never-written rule:
    D<=128 covers 32*ceil(max_seqlen/32) rows, D>128 covers 8*ceil(max_seqlen/8)."""
    g = torch.Generator().manual_seed(4)
    lens = [5, 0, 37, 12]
    cu = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0).tolist()), dtype=torch.int32)
    tot = int(cu[-1])
    q, k, v = randn(g, tot, 2, d), randn(g, tot, 2, d), randn(g, tot, 2, d)
    out = A.varlen_prefill(q, k, v, cu, max_seqlen, causal, F64)
    close(out, t64(Bt.varlen_prefill(q.double(), k.double(), v.double(), cu, max_seqlen, causal)))
    limit = A.varlen_row_limit(max_seqlen, d)
    assert limit == (32 * ((max_seqlen + 31) // 32) if d <= 128 else 8 * ((max_seqlen + 7) // 8))
    s37 = int(cu[2])
    if limit < 37:
        assert (out[s37 + limit:s37 + 37] == 0).all()
    # rows that are written equal per-segment prefill
    for i, n in enumerate(lens):
        if n == 0:
            continue
        s = int(cu[i])
        r = min(n, limit)
        seg = A.prefill(q[s:s + n].permute(1, 0, 2)[None], k[s:s + n].permute(1, 0, 2)[None],
                        v[s:s + n].permute(1, 0, 2)[None], causal, F64)[0].permute(1, 0, 2)
        close(out[s:s + r], seg[:r])


def _int8_inputs(seed=5, b=2, hq=4, hkv=2, n=9, d=16):
    g = torch.Generator().manual_seed(seed)
    q, k, v = randn(g, b, hq, 1, d), randn(g, b, hkv, n, d), randn(g, b, hkv, n, d)
    qs = q.float().abs().amax(-1).squeeze(-1) / 127
    ks = (k.float().abs().amax((-1, -2)) / 127).unsqueeze(-1).expand(b, hkv, n).contiguous()
    return q, k, v, qs, ks


@pytest.mark.parametrize("cache_len", [0, 4, 8])
def test_int8_vs_brute_and_dequant(cache_len):
    q, k, v, qs, ks = _int8_inputs()
    out = A.decode_int8(q, k, v, qs, ks, cache_len, F64)
    close(out, t64(Bt.decode_int8(q, k.float(), v.double(), qs, ks, cache_len)), tol=1e-6)
    close(out, A.decode_int8_dequant_reference(q, k, v, qs, ks, cache_len), tol=1e-5)


def test_int8_k_scale_flat_read_quirk():
    """The kernel reads k_scale.flat[b*H_KV + h_kv] (flash_attn_kernel.cu:2825), not
    k_scale[b, h_kv, 0]: a per-(b,h) scale laid out along N changes the result."""
    q, k, v, qs, _ = _int8_inputs(n=9)
    b, hkv, n = 2, 2, 9
    ks = torch.rand(b, hkv, n, generator=torch.Generator().manual_seed(9)) * 0.05 + 0.01
    used = A.int8_k_scale_per_head(ks, b, hkv)
    assert torch.equal(used, ks.reshape(-1)[: b * hkv].view(b, hkv))
    out = A.decode_int8(q, k, v, qs, ks, 8, F64)
    close(out, t64(Bt.decode_int8(q, k.float(), v.double(), qs, ks, 8)), tol=1e-6)


# ---------------------------------------------------------------- closed forms

def test_decode_cache_len_zero_returns_first_value_row():
    g = torch.Generator().manual_seed(6)
    q, k, v = randn(g, 2, 4, 1, 16), randn(g, 2, 2, 9, 16), randn(g, 2, 2, 9, 16)
    out = A.decode(q, k, v, True, 0, F64)
    close(out, A.expand_kv(v, 4)[:, :, :1].double())


def test_identical_keys_give_mean_value():
    g = torch.Generator().manual_seed(7)
    q, v = randn(g, 1, 2, 6, 8), randn(g, 1, 2, 6, 8)
    k = randn(g, 1, 2, 1, 8).expand(1, 2, 6, 8).contiguous()
    out = A.prefill(q, k, v, False, F64)
    close(out, v.double().mean(2, keepdim=True).expand_as(out))
    out_c = A.prefill(q, k, v, True, F64)  # causal: running means
    close(out_c, v.double().cumsum(2) / torch.arange(1, 7, dtype=F64).view(1, 1, 6, 1))


def test_dominant_key_selects_its_value_row():
    d = 16
    q = torch.zeros(1, 1, 1, d, dtype=torch.float16)
    q[..., 0] = 8.0
    k = torch.zeros(1, 1, 10, d, dtype=torch.float16)
    k[0, 0, 6, 0] = 8.0  # score 64/4 = 16 vs 0 elsewhere
    v = torch.arange(10 * d, dtype=torch.float32).view(1, 1, 10, d).half() / 100
    out = A.decode(q, k, v, False, 9, F64)
    w = torch.exp(torch.tensor(16.0, dtype=F64))
    expect = (w * v[0, 0, 6].double() + v[0, 0].double().sum(0) - v[0, 0, 6].double()) / (w + 9)
    close(out[0, 0, 0], expect)


def test_prefill_causal_first_row_is_first_value():
    g = torch.Generator().manual_seed(8)
    q, k, v = randn(g, 1, 3, 5, 8), randn(g, 1, 3, 5, 8), randn(g, 1, 3, 5, 8)
    close(A.prefill(q, k, v, True, F64)[:, :, 0], v[:, :, 0].double())


def test_int8_exact_codes_reduce_to_float_decode():
    """With q = qi*q_s and k = ki*k_s exactly representable, quantization is
    lossless and the INT8 path must equal plain decode (no dropped term/scale)."""
    g = torch.Generator().manual_seed(10)
    b, hq, hkv, n, d = 2, 4, 2, 7, 16
    qi = torch.randint(-127, 128, (b, hq, 1, d), generator=g).float()
    ki = torch.randint(-127, 128, (b, hkv, n, d), generator=g).float()
    qs = torch.full((b, hq), 2.0 ** -7)
    ks = torch.full((b, hkv, n), 2.0 ** -6)
    q, k = (qi * 2.0 ** -7).half(), (ki * 2.0 ** -6).half()
    v = randn(g, b, hkv, n, d)
    out = A.decode_int8(q, k, v, qs, ks, 5, F64)
    ref = A.decode(q, k, v, True, 5, F64)
    close(out, ref, tol=1e-5)


def test_roundf_ties_away_from_zero():
    s = torch.tensor([1.0])
    x = torch.tensor([2.5, -2.5, 0.5, -0.5, 1.4990234375, 126.5, 300.0, -300.0]).half()  # all exact in fp16
    got = A.quantize_int8(x, s).tolist()
    assert got == [3, -3, 1, -1, 1, 127, 127, -127]


def test_gqa_equals_expanded_mha():
    g = torch.Generator().manual_seed(11)
    q, k, v = randn(g, 2, 8, 12, 8), randn(g, 2, 2, 12, 8), randn(g, 2, 2, 12, 8)
    close(A.prefill(q, k, v, True, F64),
          A.prefill(q, k.repeat_interleave(4, 1), v.repeat_interleave(4, 1), True, F64))
    # head h uses kv head h // 4 (not h % 2)
    alt = A.prefill(q, k.repeat(1, 4, 1, 1), v.repeat(1, 4, 1, 1), True, F64)
    assert not torch.allclose(alt, A.prefill(q, k, v, True, F64))


def test_continuous_batching_equals_per_row_decode():
    g = torch.Generator().manual_seed(12)
    q, k, v = randn(g, 3, 4, 1, 8), randn(g, 3, 2, 20, 8), randn(g, 3, 2, 20, 8)
    cl = torch.tensor([0, 7, 30], dtype=torch.int32)
    out = A.continuous_batching(q, k, v, cl, True, F64)
    for i, c in enumerate(cl.tolist()):
        n = min(c + 1, 20)
        close(out[i:i + 1], A.decode(q[i:i + 1], k[i:i + 1, :, :n], v[i:i + 1, :, :n], True, n - 1, F64))


# ---------------------------------------------------------------- golden fixtures

def _golden_files():
    return sorted(f for f in os.listdir(GOLDEN) if f.endswith(".pt")) if os.path.isdir(GOLDEN) else []


def test_golden_fixtures_present():
    assert len(_golden_files()) >= 13


@pytest.mark.parametrize("fname", _golden_files())
def test_oracle_matches_golden(fname):
    fx = torch.load(os.path.join(GOLDEN, fname), weights_only=True)
    kind = fx["kind"]
    a = fx["args"]
    if kind == "prefill":
        out = A.prefill(a["q"], a["k"], a["v"], bool(a["causal"]), F64)
    elif kind == "decode":
        out = A.decode(a["q"], a["k"], a["v"], bool(a["causal"]), int(a["cache_len"]), F64)
    elif kind == "continuous_batching":
        out = A.continuous_batching(a["q"], a["k"], a["v"], a["cache_lens"], bool(a["causal"]), F64)
    elif kind == "paged":
        out = A.paged_decode(a["q"], a["k_cache"], a["v_cache"], a["block_table"], a["seq_lens"],
                             int(a["max_num_blocks"]), F64)
    elif kind == "varlen":
        out = A.varlen_prefill(a["q"], a["k"], a["v"], a["cu_seqlens"], int(a["max_seqlen"]),
                               bool(a["causal"]), F64)
    elif kind == "int8":
        out = A.decode_int8(a["q"], a["k"], a["v"], a["q_scale"], a["k_scale"], int(a["cache_len"]), F64)
    elif kind == "prefill_lse":
        for got, exp in zip(A.prefill_lse(a["q"], a["k"], a["v"], bool(a["causal"]), F64), fx["outs"]):
            close(got, exp, tol=1e-9)
        return
    elif kind == "backward":
        got = A.backward(a["dout"], a["q"], a["k"], a["v"], a["out"], a["lse"], bool(a["causal"]))
        for g_, exp in zip(got, fx["outs"]):
            close(g_, exp, tol=1e-9)
        return
    elif kind == "sliding_window":
        out = A.decode_sliding_window(a["q"], a["k"], a["v"], int(a["cache_len"]), int(a["window"]),
                                      int(a["sink"]), F64)
        close(out, fx["outs"][0], tol=1e-6)
        return
    elif kind == "int8_kv_cache":
        out = A.decode_int8_kv_cache(a["q"], a["k_i8"], a["v_i8"], a["k_scale"], a["v_scale"],
                                     int(a["cache_len"]), F64)
        close(out, fx["outs"][0], tol=1e-6)
        return
    elif kind == "token_eviction":
        got = A.token_eviction(a["k"], a["v"], a["attn_scores"], int(a["num_evict"]))
        for g_, exp in zip(got, fx["outs"]):
            assert torch.equal(g_, exp)
        return
    elif kind == "speculative_verify":
        acc, toks = A.speculative_verify(a["target_probs"], a["draft_probs"], a["draft_tokens"],
                                         a["random_vals"], int(a["K"]))
        assert torch.equal(acc, fx["outs"][0]) and torch.equal(toks, fx["outs"][1])
        return
    else:
        raise AssertionError(kind)
    close(out, fx["out"], tol=1e-6)


# ---------------------------------------------------------------- next-row decode variants

@pytest.mark.parametrize("cache_len,window,sink", [
    (69, 16, 4), (69, 16, 0), (69, 200, 0), (30, 8, 40), (69, 0, 5), (5, 3, 5),
    (100, 10, 2), (-1, 4, 0), (-1, 4, 3), (40, -3, 2), (0, 1, 0),
])
def test_sliding_window_vs_brute(cache_len, window, sink):
    """Window/sink index rules (flash_attn_kernel.cu:4386-4387, :4413-4416) against the
    kernel-loop restatement, including sinks past cache_len, windows past N, an
    empty key set (NaN) and cache_len >= N."""
    g = torch.Generator().manual_seed(11)
    q, k, v = randn(g, 2, 4, 1, 8), randn(g, 2, 2, 70, 8), randn(g, 2, 2, 70, 8)
    close(A.decode_sliding_window(q, k, v, cache_len, window, sink, F64),
          t64(Bt.decode_sliding_window(q.double(), k.double(), v.double(), cache_len, window, sink)))


def test_sliding_window_reductions():
    """A window covering every key is causal decode; a sink covering every key is the
    non-causal decode; a zero window keeps exactly the sink keys."""
    g = torch.Generator().manual_seed(12)
    q, k, v = randn(g, 1, 4, 1, 8), randn(g, 1, 2, 50, 8), randn(g, 1, 2, 50, 8)
    close(A.decode_sliding_window(q, k, v, 30, 1000, 0, F64), A.decode(q, k, v, True, 30, F64))
    close(A.decode_sliding_window(q, k, v, 30, 1, 50, F64), A.decode(q, k, v, False, 30, F64))
    close(A.decode_sliding_window(q, k, v, 30, 0, 7, F64), A.decode(q, k[:, :, :7], v[:, :, :7], False, 0, F64))


@pytest.mark.parametrize("cache_len", [0, 40, 69, 200, -1])
def test_int8_kv_cache_vs_brute(cache_len):
    """Per-token fp16-scale dequantization to half (flash_attn_kernel.cu:4083-4086) and
    the always-on k > cache_len mask (:4094) against the kernel-loop restatement."""
    g = torch.Generator().manual_seed(13)
    q = randn(g, 2, 4, 1, 8)
    k_i8 = torch.randint(-127, 128, (2, 2, 70, 8), generator=g, dtype=torch.int8)
    v_i8 = torch.randint(-127, 128, (2, 2, 70, 8), generator=g, dtype=torch.int8)
    ks = (torch.rand(2, 2, 70, generator=g) * 0.05 + 1e-3).half()
    vs = (torch.rand(2, 2, 70, generator=g) * 0.05 + 1e-3).half()
    close(A.decode_int8_kv_cache(q, k_i8, v_i8, ks, vs, cache_len, F64),
          t64(Bt.decode_int8_kv_cache(q.double(), k_i8, v_i8, ks, vs, cache_len)))


def test_int8_kv_cache_exact_scales_reduce_to_decode():
    """With power-of-two scales the dequantized cache is exact, so the result is the
    plain causal decode on int8 * scale."""
    g = torch.Generator().manual_seed(14)
    q = randn(g, 1, 8, 1, 16)
    k_i8 = torch.randint(-127, 128, (1, 2, 33, 16), generator=g, dtype=torch.int8)
    v_i8 = torch.randint(-127, 128, (1, 2, 33, 16), generator=g, dtype=torch.int8)
    ks = torch.full((1, 2, 33), 2.0 ** -6).half()
    vs = torch.full((1, 2, 33), 2.0 ** -5).half()
    kd, vd = k_i8.double() * 2.0 ** -6, v_i8.double() * 2.0 ** -5
    close(A.decode_int8_kv_cache(q, k_i8, v_i8, ks, vs, 20, F64), A.decode(q, kd, vd, True, 20, F64))


# ---------------------------------------------------------------- training path (LSE forward, backward)

@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("n,d", [(5, 4), (33, 8), (40, 3)])
def test_prefill_lse_vs_brute(causal, n, d):
    g = torch.Generator().manual_seed(100 + n + d)
    q, k, v = (randn(g, 1, 2, n, d, dtype=F64) for _ in range(3))
    out, lse = A.prefill_lse(q, k, v, causal, compute_dtype=F64)
    bo, bl = Bt.prefill_lse(q, k, v, causal)
    close(out, bo)
    close(lse, bl)
    # out equals the plain prefill restatement
    close(out, A.prefill(q, k, v, causal, compute_dtype=F64))


def test_prefill_lse_closed_forms():
    g = torch.Generator().manual_seed(7)
    d = 8
    q = randn(g, 1, 1, 6, d, dtype=F64)
    k1 = randn(g, 1, 1, 1, d, dtype=F64)
    kk = k1.expand(1, 1, 6, d).contiguous()
    v = randn(g, 1, 1, 6, d, dtype=F64)
    _, lse = A.prefill_lse(q, kk, v, causal=False, compute_dtype=F64)
    # identical keys: LSE_i = s_i + log(N)
    s = (q * k1).sum(-1) / d ** 0.5
    close(lse, s + torch.log(torch.tensor(6.0, dtype=F64)))
    # causal row 0 sees only key 0: LSE_0 = s_00
    _, lse_c = A.prefill_lse(q, v, v, causal=True, compute_dtype=F64)
    close(lse_c[..., 0], (q[..., 0, :] * v[..., 0, :]).sum(-1) / d ** 0.5)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("n,d", [(5, 4), (17, 8), (9, 3)])
def test_backward_vs_brute(causal, n, d):
    g = torch.Generator().manual_seed(200 + n * d)
    q, k, v, do = (randn(g, 1, 2, n, d, dtype=F64) for _ in range(4))
    out, lse = A.prefill_lse(q, k, v, causal, compute_dtype=F64)
    got = A.backward(do, q, k, v, out, lse, causal)
    ref = Bt.backward(do, q, k, v, out, lse, causal)
    for a, b in zip(got, ref):
        close(a, b)


@pytest.mark.parametrize("causal", [True, False])
def test_backward_equals_autograd(causal):
    """Independent derivation: torch autograd of the math attention
    (the reference test_backward.py:7-18 reference) gives the same gradients."""
    g = torch.Generator().manual_seed(7)
    B, H, N, D = 2, 3, 17, 32  # test_backward.py:35-36
    q, k, v, do = (randn(g, B, H, N, D, dtype=F64) for _ in range(4))
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    s = torch.matmul(qa, ka.transpose(-1, -2)) / D ** 0.5
    if causal:
        s = s.masked_fill(torch.triu(torch.ones(N, N, dtype=torch.bool), 1), float("-inf"))
    o = torch.matmul(torch.softmax(s, -1), va)
    o.backward(do)
    out, lse = A.prefill_lse(q, k, v, causal, compute_dtype=F64)
    close(out, o.detach(), 1e-12)
    dq, dk, dv = A.backward(do, q, k, v, out, lse, causal)
    close(dq, qa.grad, 1e-10)
    close(dk, ka.grad, 1e-10)
    close(dv, va.grad, 1e-10)


def test_backward_finite_differences():
    """dL/dx for L = sum(dO * O) by central differences on a tiny fp64 case."""
    g = torch.Generator().manual_seed(3)
    q, k, v, do = (randn(g, 1, 1, 4, 3, dtype=F64) for _ in range(4))

    def loss(q_, k_, v_):
        return (A.prefill(q_, k_, v_, True, compute_dtype=F64) * do).sum()

    out, lse = A.prefill_lse(q, k, v, True, compute_dtype=F64)
    grads = A.backward(do, q, k, v, out, lse, True)
    eps = 1e-6
    for which, grad in enumerate(grads):
        args = [q, k, v]
        for idx in [(0, 0, 0, 0), (0, 0, 2, 1), (0, 0, 3, 2)]:
            plus = [a.clone() for a in args]
            minus = [a.clone() for a in args]
            plus[which][idx] += eps
            minus[which][idx] -= eps
            fd = (loss(*plus) - loss(*minus)) / (2 * eps)
            assert abs(fd.item() - grad[idx].item()) < 1e-7, (which, idx)


# ---------------------------------------------------------------- token eviction

@pytest.mark.parametrize("n,num_evict", [(1, 0), (1, 1), (7, 3), (16, 0), (16, 16), (16, 20), (33, -2), (40, 11)])
def test_token_eviction_vs_brute(n, num_evict):
    g = torch.Generator().manual_seed(n * 31 + num_evict)
    k = randn(g, 2, 3, n, 4)
    v = randn(g, 2, 3, n, 4)
    # few distinct values: many ties, so the stable tie order is exercised
    sc = torch.randint(0, 5, (2, n), generator=g).float() * 0.5
    ko, vo, m = A.token_eviction(k, v, sc, num_evict)
    bk, bv, bm = Bt.token_eviction(k, v, sc, num_evict)
    assert torch.equal(m, torch.tensor(bm, dtype=torch.int32))
    assert torch.equal(ko, torch.tensor(bk, dtype=torch.float16))
    assert torch.equal(vo, torch.tensor(bv, dtype=torch.float16))


def test_token_eviction_closed_forms():
    g = torch.Generator().manual_seed(9)
    k, v = randn(g, 1, 2, 10, 8), randn(g, 1, 2, 10, 8)
    sc = torch.arange(10, dtype=torch.float32).flip(0).unsqueeze(0)  # token 9 lowest
    ko, vo, m = A.token_eviction(k, v, sc, 3)
    assert m.tolist() == [[1] * 7 + [0] * 3]  # the three lowest scores are tokens 7, 8, 9
    assert torch.equal(ko[:, :, :7], k[:, :, :7]) and not ko[:, :, 7:].any()
    ko, vo, m = A.token_eviction(k, v, sc, 0)
    assert torch.equal(ko, k) and torch.equal(vo, v) and bool(m.all())


# ---------------------------------------------------------------- speculative verify

def _spec_inputs(seed, B, K, V, mode="random"):
    g = torch.Generator().manual_seed(seed)
    tp = torch.softmax(torch.randn(B, K + 1, V, generator=g), -1)
    if mode == "same":
        dp = tp[:, :K].clone()
    else:
        dp = torch.softmax(torch.randn(B, K, V, generator=g), -1)
    tok = torch.randint(0, V, (B, K), generator=g)
    rv = torch.rand(B, K, generator=g)
    return tp, dp, tok, rv


@pytest.mark.parametrize("seed,B,K,V,mode", [(0, 2, 4, 256, "random"), (1, 4, 5, 128, "same"),
                                             (2, 3, 8, 64, "random"), (3, 2, 1, 100, "random")])
def test_speculative_verify_vs_brute(seed, B, K, V, mode):
    tp, dp, tok, rv = _spec_inputs(seed, B, K, V, mode)
    if mode == "same":
        rv = torch.zeros(B, K)  # test_speculative.py:152: everything accepted
    acc, out = A.speculative_verify(tp, dp, tok, rv, K)
    bacc, bout = Bt.speculative_verify(tp, dp, tok, rv, K)
    assert acc.tolist() == bacc and out.tolist() == bout


def test_speculative_verify_orthogonal_and_quirks():
    """test_speculative.py:167-200 (one-hot, disjoint supports): rejection at 0;
    plus the index-0 quirk: a hit at v = 0 is overwritten by the next hit."""
    B, K, V = 2, 4, 64
    tp = torch.zeros(B, K + 1, V)
    dp = torch.zeros(B, K, V)
    for i in range(K + 1):
        tp[:, i, (i * 10) % V] = 1.0
    for i in range(K):
        dp[:, i, (i * 10 + 1) % V] = 1.0
    tok = torch.full((B, K), 1)
    rv = torch.full((B, K), 0.5)
    acc, out = A.speculative_verify(tp, dp, tok, rv, K)
    bacc, bout = Bt.speculative_verify(tp, dp, tok, rv, K)
    assert acc.tolist() == bacc == [0, 0]
    assert out.tolist() == bout
    # row 0: residual sampled at v=0 (only hit); bonus from target row 1 (one-hot at 10)
    assert out[0].tolist() == [0, 10, -1, -1, -1]
    # quirk: the first hit is v=0 and a later hit exists -> the later one
    assert A._first_index_quirk([True, False, True, True]) == 2
    assert A._first_index_quirk([False, True, True]) == 1
    assert A._first_index_quirk([True]) == 0
    assert A._first_index_quirk([False, False]) == 0


# ---- tensor-parallel helpers (same-device copies and the fp16 accumulate) ----

@pytest.mark.parametrize("total,start,count", [(16, 0, 4), (16, 0, 8), (16, 5, 3), (16, 0, 16), (16, 15, 1),
                                               (16, 7, 0), (3, 1, 2)])
def test_scatter_gather_heads_equal_slicing(total, start, count):
    """The reference's per-element index map (three divisions per element) is a
    head-range slice: scatter == full[:, start:start+count]; gather writes that
    slice and leaves every other head untouched; gather(scatter(x)) == x there."""
    g = torch.Generator().manual_seed(total * 100 + start * 10 + count)
    B, N, D = 2, 5, 6
    full = torch.randn(B, total, N, D, generator=g).half()
    local0 = torch.randn(B, count, N, D, generator=g).half()
    loc = A.scatter_heads(full, local0, total, start, count)
    assert torch.equal(loc, full[:, start:start + count])
    base = torch.randn(B, total, N, D, generator=g).half()
    got = A.gather_heads(base, local0, total, start, count)
    ref = base.clone()
    ref[:, start:start + count] = local0
    assert torch.equal(got, ref)
    assert torch.equal(A.gather_heads(torch.zeros_like(full), loc, total, start, count)[:, start:start + count],
                       full[:, start:start + count])


def test_scatter_gather_reference_case():
    """test_multi_gpu.py:44-70: seed 42, B=2, H=16, N=128, D=64, counts 4 and 8
    from head 0; scatter equals the leading heads, gather reconstructs them."""
    torch.manual_seed(42)
    B, H, N, D = 2, 16, 128, 64
    full = torch.randn(B, H, N, D).half()
    for c in (4, 8):
        loc = A.scatter_heads(full, torch.zeros(B, c, N, D).half(), H, 0, c)
        assert (loc.float() - full[:, :c].float()).abs().max().item() < 1e-6
        rec = A.gather_heads(torch.zeros_like(full), loc, H, 0, c)
        assert torch.equal(rec[:, :c], full[:, :c]) and not rec[:, c:].any()


def test_allreduce_fp16_is_correctly_rounded_sum():
    """fp16 + fp16 widened to fp32, added (RNE) and narrowed (RNE) equals the
    exact sum rounded once to fp16: fp32 carries 24 >= 2*11 + 2 significand
    bits, so the double rounding is innocuous (Figueroa, 1995).  Checked for
    every fp16 bit pattern against a set of partners that produce ties, carries,
    cancellation, subnormals and overflow; the exact sum is computed in fp64,
    where the sum of two fp16 values is exact."""
    import numpy as np

    a = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    partners = np.array([0.0, -0.0, 1.0, -1.0, 2.0 ** -24, -(2.0 ** -24), 2.0 ** -14, 0.5, 3.0, 1024.5,
                         2049.0, 65504.0, -65504.0, 16.0, 0.333, 1e-3, 7.0e4, np.inf, -np.inf], dtype=np.float64)
    partners = partners.astype(np.float16)
    for p in partners:
        b = np.full_like(a, p)
        got = A.allreduce_fp16(torch.from_numpy(a.copy()), torch.from_numpy(b)).numpy()
        with np.errstate(over="ignore", invalid="ignore"):
            exact = (a.astype(np.float64) + b.astype(np.float64)).astype(np.float16)
        nan = np.isnan(exact)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan].view(np.uint16), exact[~nan].view(np.uint16)), float(p)


def test_allreduce_fp16_known_answers():
    """Ties to even (2048 + 1 -> 2048, 2050 + 1 -> 2052), overflow past the
    rounding midpoint (65504 + 16 -> inf), exact cancellation (+0), NaN."""
    import numpy as np

    d = torch.tensor([2048.0, 2050.0, 65504.0, 1.5, float("nan"), 65504.0]).half()
    s = torch.tensor([1.0, 1.0, 16.0, -1.5, 1.0, 8.0]).half()
    r = A.allreduce_fp16(d, s)
    assert r[:4].tolist() == [2048.0, 2052.0, float("inf"), 0.0]
    assert math.isnan(r[4].item()) and r[5].item() == 65504.0
    assert not np.signbit(r[3].numpy())
