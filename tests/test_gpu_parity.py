"""GPU parity: every hot-path entry point of ``flash_attn_v100`` against the CPU oracle.

Shapes, seeds and cases follow the reference's own test scripts (test.py,
test_decode.py, test_gqa.py, test_wmma.py, test_prefill_gqa.py,
test_continuous_batching.py, test_async.py) plus the BASELINE configs, edge
cases (cache_len 0 and N-1, ragged tails, D not a multiple of 8/16, empty
ranges -> NaN) and full-size configs checked on sampled sequences.
Tolerance: max-abs 2e-3 + rtol 1e-2 (fp16 paths), rel-L2 1.5e-2 (INT8).
"""
import math

import pytest
import torch

from oracle import attention as A
from tests.helpers import INT8_REL_L2, assert_close, randn, rel_l2

pytestmark = pytest.mark.gpu
DEV = "cuda"


def gen(seed):
    return torch.Generator().manual_seed(seed)


def cuda(*ts):
    return [t.to(DEV).contiguous() for t in ts]


# ---------------------------------------------------------------- prefill

@pytest.mark.parametrize("causal", [True, False])
def test_forward_fp16_config1(fa, causal):
    """BASELINE config 1 / test.py:18-57: B=2,H=8,N=256,D=64, seed 0."""
    g = gen(0)
    q, k, v = randn(g, 2, 8, 256, 64), randn(g, 2, 8, 256, 64), randn(g, 2, 8, 256, 64)
    out = fa.forward_fp16(*cuda(q, k, v), causal)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16 and out.shape == q.shape
    assert_close(out, A.prefill(q, k, v, causal), what="forward_fp16 cfg1")


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("b,h,n,d", [
    (1, 2, 1, 64), (1, 2, 5, 64), (2, 3, 33, 64), (1, 2, 127, 128), (1, 2, 129, 128),
    (1, 4, 300, 128), (1, 2, 77, 32), (1, 2, 70, 80), (1, 2, 50, 96), (1, 2, 45, 36),
    (1, 2, 130, 256), (1, 1, 65, 200), (1, 2, 64, 16),
])
def test_forward_fp16_shapes(fa, causal, b, h, n, d):
    g = gen(n * 7 + d)
    q, k, v = randn(g, b, h, n, d), randn(g, b, h, n, d), randn(g, b, h, n, d)
    out = fa.forward_fp16(*cuda(q, k, v), causal)
    assert_close(out, A.prefill(q, k, v, causal), what=f"forward_fp16 {b,h,n,d}")


@pytest.mark.parametrize("b,h,n,d", [(1, 4, 64, 64), (2, 4, 128, 64), (1, 8, 256, 64),
                                     (2, 8, 512, 64), (1, 4, 128, 128), (1, 2, 96, 32)])
def test_forward_fp16_wmma(fa, b, h, n, d):
    """test_wmma.py:25-78 (seed 42): WMMA name == forward_fp16 == oracle."""
    g = gen(42)
    q, k, v = randn(g, b, h, n, d), randn(g, b, h, n, d), randn(g, b, h, n, d)
    qc, kc, vc = cuda(q, k, v)
    out = fa.forward_fp16_wmma(qc, kc, vc, True)
    ref = fa.forward_fp16(qc, kc, vc, True)
    assert_close(out, A.prefill(q, k, v, True), what="wmma")
    assert torch.equal(out, ref)


def test_forward_fp16_wmma_rejects_unsupported_d(fa):
    x = torch.zeros(1, 1, 8, 72, dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError):
        fa.forward_fp16_wmma(x, x, x, True)
    y = torch.zeros(1, 1, 8, 144, dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError):
        fa.forward_fp16_wmma(y, y, y, True)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("b,hq,hkv,n,d", [(1, 8, 4, 64, 64), (2, 16, 4, 96, 64), (1, 32, 8, 128, 128),
                                          (1, 32, 8, 64, 256)])
def test_prefill_gqa(fa, causal, b, hq, hkv, n, d):
    """test_gqa.py:133-167 shapes (seed 1234), plus _out aliasing (test.py:108-131)."""
    g = gen(1234)
    q, k, v = randn(g, b, hq, n, d), randn(g, b, hkv, n, d), randn(g, b, hkv, n, d)
    qc, kc, vc = cuda(q, k, v)
    ref = A.prefill(q, k, v, causal)
    assert_close(fa.forward_prefill_gqa_fp16(qc, kc, vc, causal), ref, what="prefill_gqa")
    assert_close(fa.forward_prefill_gqa_fp16_warp(qc, kc, vc, causal), ref, what="prefill_gqa_warp")
    out = torch.empty_like(qc)
    ret = fa.forward_prefill_gqa_fp16_out(out, qc, kc, vc, causal)
    assert ret.data_ptr() == out.data_ptr()
    assert_close(out, ref, what="prefill_gqa_out")


def test_prefill_mha_equals_gqa_api(fa):
    """test_prefill_gqa.py:94-116: with H_Q == H_KV the GQA API equals forward_fp16."""
    g = gen(42)
    q, k, v = cuda(randn(g, 2, 4, 100, 64), randn(g, 2, 4, 100, 64), randn(g, 2, 4, 100, 64))
    a = fa.forward_fp16(q, k, v, True)
    b = fa.forward_prefill_gqa_fp16(q, k, v, True)
    assert (a.float() - b.float()).abs().max().item() <= 1e-3


# ---------------------------------------------------------------- decode

@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("b,h,n,d,cache_len", [(2, 4, 1, 64, 0), (1, 8, 65, 64, 0), (2, 8, 65, 64, 64),
                                               (1, 8, 300, 128, 200), (1, 2, 40, 256, 39),
                                               (1, 2, 33, 72, 10), (1, 1, 5000, 128, 4999)])
def test_forward_decode_fp16(fa, causal, b, h, n, d, cache_len):
    """test_decode.py:218-266: MHA decode, causal masks k > cache_len."""
    g = gen(b * 1000 + n + d)
    q, k, v = randn(g, b, h, 1, d), randn(g, b, h, n, d), randn(g, b, h, n, d)
    out = fa.forward_decode_fp16(*cuda(q, k, v), causal, cache_len)
    assert_close(out, A.decode(q, k, v, causal, cache_len), what="decode_fp16")


@pytest.mark.parametrize("b,hq,hkv,n,d", [(1, 8, 4, 65, 64), (2, 16, 4, 127, 64), (1, 32, 8, 257, 128),
                                          (1, 32, 8, 129, 256), (2, 12, 4, 70, 128), (1, 64, 2, 500, 64),
                                          (3, 6, 1, 1000, 96)])
def test_forward_decode_gqa_fp16(fa, b, hq, hkv, n, d):
    """test_gqa.py:120-153 shapes (seed 1234) plus non-power-of-two group sizes."""
    g = gen(1234)
    q, k, v = randn(g, b, hq, 1, d), randn(g, b, hkv, n, d), randn(g, b, hkv, n, d)
    qc, kc, vc = cuda(q, k, v)
    for causal, cl in ((True, n - 1), (True, n // 2), (False, n // 3)):
        out = fa.forward_decode_gqa_fp16(qc, kc, vc, causal, cl)
        assert_close(out, A.decode(q, k, v, causal, cl), what=f"decode_gqa c={causal} cl={cl}")


def test_decode_gqa_config2(fa):
    """Q [1,32,1,128], K/V [1,8,4097,128], cache_len 4096, causal."""
    g = gen(0)
    q, k, v = randn(g, 1, 32, 1, 128), randn(g, 1, 8, 4097, 128), randn(g, 1, 8, 4097, 128)
    out = fa.forward_decode_gqa_fp16(*cuda(q, k, v), True, 4096)
    assert_close(out, A.decode(q, k, v, True, 4096), what="config2")


def test_decode_split_workspace_reuse(fa):
    """The fused split combine leaves its arrival counters at zero: repeated calls,
    calls with other shapes in between, and calls on another stream all agree."""
    g = gen(21)
    q, k, v = randn(g, 2, 32, 1, 128), randn(g, 2, 8, 9000, 128), randn(g, 2, 8, 9000, 128)
    qc, kc, vc = cuda(q, k, v)
    ref = A.decode(q, k, v, True, 8000)
    first = fa.forward_decode_gqa_fp16(qc, kc, vc, True, 8000)
    assert_close(first, ref, what="split decode")
    q2, k2, v2 = cuda(randn(g, 1, 8, 1, 64), randn(g, 1, 2, 3000, 64), randn(g, 1, 2, 3000, 64))
    for i in range(5):
        fa.forward_decode_gqa_fp16(q2, k2, v2, False, 0)
        again = fa.forward_decode_gqa_fp16(qc, kc, vc, True, 8000)
        assert torch.equal(again, first), f"iteration {i}"
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        other = fa.forward_decode_gqa_fp16(qc, kc, vc, True, 8000)
    s.synchronize()
    assert torch.equal(other, first)


def test_decode_workspace_shared_across_shapes(fa):
    """Calls of different shapes share one workspace per stream: a call with few
    units and large partials (B=1, D=256, many splits) must not disturb the split
    counters of a following call with many units (B=16)."""
    g = gen(23)
    a = [randn(g, 1, 16, 1, 256), randn(g, 1, 2, 3000, 256), randn(g, 1, 2, 3000, 256)]
    b = [randn(g, 16, 32, 1, 128), randn(g, 16, 8, 1025, 128), randn(g, 16, 8, 1025, 128)]
    ac, bc = cuda(*a), cuda(*b)
    ref_b = A.decode(*b, True, 1024)
    for _ in range(3):
        fa.forward_decode_gqa_fp16(*ac, True, 2999)
        assert_close(fa.forward_decode_gqa_fp16(*bc, True, 1024), ref_b, what="after small-unit call")
        qs, ks = int8_scales(b[0], b[1])
        out = fa.forward_decode_int8_gqa(*bc, qs.cuda(), ks.cuda(), 1024)
        assert_close(out, A.decode_int8(*b, qs, ks, 1024), what="int8 after small-unit call")


def test_paged_decode_sequence_longer_than_table_row_reads_on(fa):
    """A sequence longer than 16 * max_num_blocks keeps reading the flattened
    table past its own row (flash_attn_kernel.cu:3438), as the reference does."""
    g = gen(22)
    q, kc, vc = randn(g, 2, 4, 1, 64), randn(g, 8, 2, 16, 64), randn(g, 8, 2, 16, 64)
    bt = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32)
    slt = torch.tensor([40, 20], dtype=torch.int32)  # 40 > 16 * max_num_blocks: row 0 reads page 2 too
    out = fa.forward_paged_decode_gqa_fp16(*cuda(q, kc, vc, bt, slt), 2)
    assert_close(out, A.paged_decode(q, kc, vc, bt, slt, 2), what="paged overrun")


def test_paged_decode_overrun_spanning_page_rounds(fa):
    """An overrun far past the row (17 600 tokens on a 10-block row stride) is
    walked by the last split in several rounds of staged page ids."""
    g = gen(24)
    B, Hq, Hkv, D, P = 2, 8, 2, 64, 64
    q, kc, vc = randn(g, B, Hq, 1, D), randn(g, P, Hkv, 16, D), randn(g, P, Hkv, 16, D)
    bt = torch.randint(0, P, (B, 600), generator=g, dtype=torch.int32)
    slt = torch.tensor([16 * 1100, 150], dtype=torch.int32)
    out = fa.forward_paged_decode_gqa_fp16(*cuda(q, kc, vc, bt, slt), 10)
    assert_close(out, A.paged_decode(q, kc, vc, bt, slt, 10), what="paged multi-round overrun")


def test_paged_decode_out_of_bounds_reads_are_nan(fa):
    """Only genuinely out-of-bounds reads (a flat table index past
    block_table.numel(), a page id outside [0, num_pages)) give NaN, and only
    for the sequence that makes them."""
    g = gen(25)
    q, kc, vc = randn(g, 3, 4, 1, 64), randn(g, 8, 2, 16, 64), randn(g, 8, 2, 16, 64)
    bt = torch.tensor([[0, 1], [2, 3], [4, 9]], dtype=torch.int32)  # page 9 >= num_pages
    slt = torch.tensor([20, 70, 30], dtype=torch.int32)  # row 1: 70 tokens need flat index 6 >= numel 6
    out = fa.forward_paged_decode_gqa_fp16(*cuda(q, kc, vc, bt, slt), 2)
    assert torch.isnan(out[1:].float()).all()
    assert_close(out[:1], A.paged_decode(q[:1], kc, vc, bt, slt[:1], 2), what="paged row 0")


def test_decode_gqa_out_and_stream(fa):
    """_out writes into the caller's tensor; _stream equals the default (test_async.py:37-65)."""
    g = gen(7)
    q, k, v = cuda(randn(g, 2, 8, 1, 64), randn(g, 2, 2, 600, 64), randn(g, 2, 2, 600, 64))
    ref = fa.forward_decode_gqa_fp16(q, k, v, True, 0)
    out = torch.empty_like(q)
    ret = fa.forward_decode_gqa_fp16_out(out, q, k, v, True, 0)
    assert ret.data_ptr() == out.data_ptr()
    assert torch.equal(out, ref)
    assert_close(ref, A.decode(q.cpu(), k.cpu(), v.cpu(), True, 0), what="cache_len=0")
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    got = fa.forward_decode_gqa_fp16_stream(q, k, v, True, 599, s.cuda_stream)
    s.synchronize()
    assert torch.equal(got, fa.forward_decode_gqa_fp16(q, k, v, True, 599))


def test_decode_validation_errors(fa):
    """test.py:70-102, :133-139: errors surface as RuntimeError."""
    q = torch.zeros(1, 4, 1, 64, dtype=torch.float16, device=DEV)
    k = torch.zeros(1, 2, 10, 64, dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError):
        fa.forward_decode_gqa_fp16(q, k.float(), k, True, 3)
    with pytest.raises(RuntimeError):
        fa.forward_decode_gqa_fp16(q, k, k, True, -1)
    with pytest.raises(RuntimeError):
        fa.forward_decode_gqa_fp16(q, k, k, True, 10)
    with pytest.raises(RuntimeError):
        fa.forward_decode_gqa_fp16(q, k.cpu(), k, True, 3)
    with pytest.raises(RuntimeError):
        fa.forward_decode_gqa_fp16_out(torch.empty(1, 4, 2, 64, dtype=torch.float16, device=DEV), q, k, k, True, 3)
    with pytest.raises(RuntimeError):
        fa.forward_decode_fp16(q, k, k, True, 3)  # MHA API needs equal head counts
    with pytest.raises(RuntimeError):
        fa.forward_decode_gqa_fp16(q, k[:, :, ::2], k[:, :, ::2], True, 3)  # non-contiguous


# ---------------------------------------------------------------- continuous batching

@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("b,hq,hkv,d,max_n,cls", [
    (3, 8, 2, 64, 17, [0, 3, 15]), (2, 32, 8, 256, 33, [0, 31]),      # test_continuous_batching.py:349-352
    (4, 32, 8, 128, 1025, [16, 1024, 500, 2000]), (5, 4, 4, 96, 700, [0, 699, 1, 350, 64]),
])
def test_continuous_batching(fa, causal, b, hq, hkv, d, max_n, cls):
    g = gen(0)
    q, k, v = randn(g, b, hq, 1, d), randn(g, b, hkv, max_n, d), randn(g, b, hkv, max_n, d)
    cl = torch.tensor(cls, dtype=torch.int32)
    out = fa.forward_continuous_batching_fp16(*cuda(q, k, v, cl), causal)
    assert_close(out, A.continuous_batching(q, k, v, cl, causal), what="cb")


@pytest.mark.parametrize("b,cls", [
    (12, [40, 7, 40, 40, 0, 7, 90, 40, 7, 90, 3, 40]),   # ties: the longest-first order must stay a bijection
    (600, None),                                          # more sequences than the longest-first limit (natural order)
])
def test_continuous_batching_ordering(fa, b, cls):
    g = gen(12)
    hq, hkv, d, max_n = 4, 2, 64, 96
    if cls is None:
        cls = torch.randint(-1, max_n, (b,), generator=g, dtype=torch.int32).tolist()
    q, k, v = randn(g, b, hq, 1, d), randn(g, b, hkv, max_n, d), randn(g, b, hkv, max_n, d)
    cl = torch.tensor(cls, dtype=torch.int32)
    out = fa.forward_continuous_batching_fp16(*cuda(q, k, v, cl), True)
    assert_close(out, A.continuous_batching(q, k, v, cl, True), what="cb order")


def test_continuous_batching_negative_len_is_nan(fa):
    g = gen(1)
    q, k, v = randn(g, 2, 4, 1, 64), randn(g, 2, 2, 300, 64), randn(g, 2, 2, 300, 64)
    cl = torch.tensor([-1, 100], dtype=torch.int32)
    out = fa.forward_continuous_batching_fp16(*cuda(q, k, v, cl), True)
    assert torch.isnan(out[0].float()).all()
    assert_close(out, A.continuous_batching(q, k, v, cl, True), what="cb nan")


def _sample_check_decode_like(out, ref_fn, rows):
    for b in rows:
        assert_close(out[b:b + 1], ref_fn(b), what=f"row {b}")


def test_continuous_batching_config3_full(fa):
    """BASELINE config 3 at full size (B=64, 32:8 heads, max_N=8193, D=128), cache_lens
    U[16,8192]; every sequence is checked against the oracle on that sequence."""
    g = gen(3)
    B, HQ, HKV, MAXN, D = 64, 32, 8, 8193, 128
    cl = torch.randint(16, 8193, (B,), generator=g, dtype=torch.int32)
    gg = torch.Generator(device=DEV).manual_seed(3)
    q = torch.randn(B, HQ, 1, D, generator=gg, device=DEV).half()
    k = torch.randn(B, HKV, MAXN, D, generator=gg, device=DEV).half()
    v = torch.randn(B, HKV, MAXN, D, generator=gg, device=DEV).half()
    out = fa.forward_continuous_batching_fp16(q, k, v, cl.to(DEV), True).cpu()
    for b in range(B):
        n = min(int(cl[b]) + 1, MAXN)
        ref = A.decode(q[b:b + 1].cpu(), k[b:b + 1, :, :n].cpu(), v[b:b + 1, :, :n].cpu(), True, n - 1)
        assert_close(out[b:b + 1], ref, what=f"cfg3 b={b}")


# ---------------------------------------------------------------- paged decode

def build_paged(k, v, seq_lens, order, page=16):
    """Reference layout builder (test_decode.py:22-44)."""
    B, HKV, _, D = k.shape
    mnb = max((s + page - 1) // page for s in seq_lens)
    npages = max(order[: sum((s + page - 1) // page for s in seq_lens)]) + 1
    kc = torch.zeros(npages, HKV, page, D, dtype=k.dtype)
    vc = torch.zeros_like(kc)
    bt = torch.full((B, mnb), -1, dtype=torch.int32)
    cur = 0
    for b, s in enumerate(seq_lens):
        for blk in range((s + page - 1) // page):
            p = order[cur]
            cur += 1
            bt[b, blk] = p
            st, en = blk * page, min(blk * page + page, s)
            kc[p, :, : en - st] = k[b, :, st:en]
            vc[p, :, : en - st] = v[b, :, st:en]
    return kc, vc, bt, mnb


def test_paged_decode_reference_case(fa):
    """test_decode.py:269-322: seed 2025, seq_lens [16,23,33], pages [5,2,7,1,9,3],
    then a cache update must change the output and still match."""
    g = gen(2025)
    B, HQ, HKV, D = 3, 8, 4, 64
    sl = [16, 23, 33]
    q, k, v = randn(g, B, HQ, 1, D), randn(g, B, HKV, 33, D), randn(g, B, HKV, 33, D)
    order = [5, 2, 7, 1, 9, 3]
    kc, vc, bt, mnb = build_paged(k, v, sl, order)
    slt = torch.tensor(sl, dtype=torch.int32)
    out = fa.forward_paged_decode_gqa_fp16(*cuda(q, kc, vc, bt, slt), mnb)
    ref = A.paged_decode(q, kc, vc, bt, slt, mnb)
    assert_close(out, ref, what="paged ref case")
    k2, v2 = k.clone(), v.clone()
    k2[1, :, 16:23] += 0.5
    v2[1, :, 16:23] -= 0.25
    kc2, vc2, _, _ = build_paged(k2, v2, sl, order)
    out2 = fa.forward_paged_decode_gqa_fp16(*cuda(q, kc2, vc2, bt, slt), mnb)
    assert_close(out2, A.paged_decode(q, kc2, vc2, bt, slt, mnb), what="paged updated")
    assert (out2.float() - out.float()).abs().max().item() > 1e-4


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (8, 8, 64), (16, 2, 256), (12, 4, 80)])
def test_paged_decode_random_tables(fa, hq, hkv, d):
    g = gen(hq + d)
    B = 6
    sl = [1, 15, 16, 17, 300, 1000]
    mnb = 64
    npages = 200
    perm = torch.randperm(npages, generator=g)
    bt = torch.full((B, mnb), -1, dtype=torch.int32)
    cur = 0
    for b, s in enumerate(sl):
        nb = (s + 15) // 16
        bt[b, :nb] = perm[cur:cur + nb].int()
        cur += nb
    kc, vc = randn(g, npages, hkv, 16, d), randn(g, npages, hkv, 16, d)
    q = randn(g, B, hq, 1, d)
    slt = torch.tensor(sl, dtype=torch.int32)
    out = fa.forward_paged_decode_gqa_fp16(*cuda(q, kc, vc, bt, slt), mnb)
    assert_close(out, A.paged_decode(q, kc, vc, bt, slt, mnb), what="paged random")


@pytest.mark.parametrize("b,sls", [
    (12, [40, 7, 40, 40, 1, 7, 90, 40, 7, 90, 3, 40]),   # longest first with ties: the order must stay a bijection
    (600, None),                                          # more sequences than the longest-first limit (natural order)
])
def test_paged_decode_ordering(fa, b, sls):
    """Paged decode serves sequences longest first (ties by index) for up to
    512 sequences and in index order beyond; every row against the oracle."""
    g = gen(13)
    hq, hkv, d, mnb = 4, 2, 64, 6
    if sls is None:
        sls = torch.randint(1, 16 * mnb + 1, (b,), generator=g, dtype=torch.int32).tolist()
    npages = b * mnb
    bt = torch.randperm(npages, generator=g).int().reshape(b, mnb)
    kc, vc = randn(g, npages, hkv, 16, d), randn(g, npages, hkv, 16, d)
    q = randn(g, b, hq, 1, d)
    slt = torch.tensor(sls, dtype=torch.int32)
    out = fa.forward_paged_decode_gqa_fp16(*cuda(q, kc, vc, bt, slt), mnb)
    assert_close(out, A.paged_decode(q, kc, vc, bt, slt, mnb), what=f"paged order b={b}")


def test_paged_decode_empty_sequence_is_nan(fa):
    g = gen(5)
    q, kc, vc = randn(g, 2, 4, 1, 64), randn(g, 4, 2, 16, 64), randn(g, 4, 2, 16, 64)
    bt = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32)
    slt = torch.tensor([0, 20], dtype=torch.int32)
    out = fa.forward_paged_decode_gqa_fp16(*cuda(q, kc, vc, bt, slt), 2)
    assert torch.isnan(out[0].float()).all()
    assert_close(out, A.paged_decode(q, kc, vc, bt, slt, 2), what="paged nan")


def test_paged_decode_config4_full(fa):
    """BASELINE config 4 at full size: B=128, 32:8 heads, D=128, 65536 pages,
    seq_lens U[64,4096], block_table = first 32768 entries of randperm(65536).
    Every sequence is checked against the oracle's paged formula
    (A.paged_decode) on the real block_table and the whole host copy of the
    caches, 16 sequences per oracle call."""
    g = gen(4)
    B, HQ, HKV, D, P, MNB = 128, 32, 8, 128, 65536, 256
    sl = torch.randint(64, 4097, (B,), generator=g, dtype=torch.int32)
    bt = torch.randperm(P, generator=g)[: B * MNB].view(B, MNB).int()
    gg = torch.Generator(device=DEV).manual_seed(4)
    q = torch.randn(B, HQ, 1, D, generator=gg, device=DEV).half()
    kc = torch.randn(P, HKV, 16, D, generator=gg, device=DEV).half()
    vc = torch.randn(P, HKV, 16, D, generator=gg, device=DEV).half()
    out = fa.forward_paged_decode_gqa_fp16(q, kc, vc, bt.to(DEV), sl.to(DEV), MNB).cpu()
    qh, kh, vh = q.cpu(), kc.cpu(), vc.cpu()
    del kc, vc
    for b0 in range(0, B, 16):
        # rows b0.. of the flat table: the oracle reads entry b * MNB + t / 16 of the
        # sub-table exactly as the kernel reads entry (b0 + b) * MNB + t / 16 of the whole
        ref = A.paged_decode(qh[b0:b0 + 16], kh, vh, bt[b0:b0 + 16], sl[b0:b0 + 16], MNB)
        for b in range(16):
            assert_close(out[b0 + b:b0 + b + 1], ref[b:b + 1], what=f"cfg4 b={b0 + b}")


# ---------------------------------------------------------------- varlen prefill

@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("lens,h,d,max_seqlen", [
    ([64, 128, 256], 4, 64, None), ([32, 64, 96], 8, 256, None),     # test_async.py:68-113
    ([5, 0, 200, 37, 1], 2, 128, None), ([100, 300], 2, 64, 40),    # empty seq, row limit
    ([70, 20], 2, 200, 30), ([129, 64, 3], 3, 80, None),
])
def test_varlen_prefill(fa, causal, lens, h, d, max_seqlen):
    g = gen(sum(lens) + d)
    cu = torch.tensor([0] + torch.cumsum(torch.tensor(lens), 0).tolist(), dtype=torch.int32)
    tot = int(cu[-1])
    q, k, v = randn(g, tot, h, d), randn(g, tot, h, d), randn(g, tot, h, d)
    ms = max(lens) if max_seqlen is None else max_seqlen
    out = fa.forward_varlen_prefill_fp16(*cuda(q, k, v, cu), ms, causal)
    assert_close(out, A.varlen_prefill(q, k, v, cu, ms, causal), what="varlen")


def test_varlen_unwritten_rows_are_zero(fa):
    """Rows outside [cu[0], cu[batch]) and past each sequence's row limit come back 0
    (the reference returns a zero-initialised tensor), even over reused dirty memory."""
    g = gen(77)
    total, h, d = 100, 2, 64
    cu = torch.tensor([3, 40, 40, 90], dtype=torch.int32)
    q, k, v = randn(g, total, h, d), randn(g, total, h, d), randn(g, total, h, d)
    for _ in range(2):
        junk = torch.full((total, h, d), float("nan"), dtype=torch.float16, device=DEV)
        del junk
        out = fa.forward_varlen_prefill_fp16(*cuda(q, k, v, cu), 20, True)
        ref = A.varlen_prefill(q, k, v, cu, 20, True)
        assert_close(out, ref, what="varlen gaps")
        assert torch.count_nonzero(out[:3]) == 0 and torch.count_nonzero(out[90:]) == 0


def test_varlen_equals_per_sequence_prefill_and_stream(fa):
    g = gen(11)
    lens = [300, 17, 512]
    cu = torch.tensor([0, 300, 317, 829], dtype=torch.int32)
    q, k, v = cuda(randn(g, 829, 4, 128), randn(g, 829, 4, 128), randn(g, 829, 4, 128))
    cuc = cu.to(DEV)
    out = fa.forward_varlen_prefill_fp16(q, k, v, cuc, 512, True)
    for i, n in enumerate(lens):
        s = int(cu[i])
        seg = fa.forward_fp16(*[t[s:s + n].permute(1, 0, 2).unsqueeze(0).contiguous() for t in (q, k, v)], True)
        assert (seg[0].permute(1, 0, 2).float() - out[s:s + n].float()).abs().max().item() <= 1e-3
    st = torch.cuda.Stream()
    torch.cuda.synchronize()
    got = fa.forward_varlen_prefill_fp16_stream(q, k, v, cuc, 512, True, st.cuda_stream)
    st.synchronize()
    assert torch.equal(got, out)


def test_varlen_config5a_sampled(fa):
    """BASELINE config 5a: 16 sequences with L ~ U[128,2048], H=32, D=128, causal."""
    g = gen(5)
    lens = torch.randint(128, 2049, (16,), generator=g).tolist()
    cu = torch.tensor([0] + torch.cumsum(torch.tensor(lens), 0).tolist(), dtype=torch.int32)
    tot = int(cu[-1])
    gg = torch.Generator(device=DEV).manual_seed(5)
    q, k, v = [torch.randn(tot, 32, 128, generator=gg, device=DEV).half() for _ in range(3)]
    out = fa.forward_varlen_prefill_fp16(q, k, v, cu.to(DEV), max(lens), True).cpu()
    # every sequence, all 32 heads
    for i in range(16):
        s, n = int(cu[i]), lens[i]
        ref = A.prefill(*[t[s:s + n].permute(1, 0, 2).unsqueeze(0).cpu() for t in (q, k, v)], True)
        assert_close(out[s:s + n], ref[0].permute(1, 0, 2), what=f"cfg5a seq {i}")


# ---------------------------------------------------------------- INT8 decode

def int8_scales(q, k):
    B, HKV, N = k.shape[0], k.shape[1], k.shape[2]
    qs = (q.float().abs().amax(-1).squeeze(-1) / 127).contiguous()
    ks = (k.float().abs().amax((-1, -2)) / 127).unsqueeze(-1).expand(B, HKV, N).contiguous()
    return qs, ks


@pytest.mark.parametrize("b,hq,hkv,n,d,cl", [(2, 8, 4, 65, 64, 64), (1, 32, 8, 300, 128, 150),
                                             (2, 4, 4, 100, 128, 0), (1, 16, 2, 700, 256, 699),
                                             (1, 6, 2, 90, 40, 50)])
def test_decode_int8(fa, b, hq, hkv, n, d, cl):
    g = gen(n + d)
    q, k, v = randn(g, b, hq, 1, d), randn(g, b, hkv, n, d), randn(g, b, hkv, n, d)
    qs, ks = int8_scales(q, k)
    out = fa.forward_decode_int8_gqa(*cuda(q, k, v, qs, ks), cl)
    ref = A.decode_int8(q, k, v, qs, ks, cl)
    assert rel_l2(out, ref) <= INT8_REL_L2
    assert_close(out, ref, what="int8")  # the integer codes agree exactly, so fp16 tolerance holds too


def test_decode_int8_k_scale_flat_quirk(fa):
    g = gen(9)
    q, k, v = randn(g, 2, 4, 1, 64), randn(g, 2, 2, 50, 64), randn(g, 2, 2, 50, 64)
    qs, _ = int8_scales(q, k)
    ks = (torch.rand(2, 2, 50, generator=g) * 0.03 + 0.02).contiguous()
    out = fa.forward_decode_int8_gqa(*cuda(q, k, v, qs, ks), 49)
    assert_close(out, A.decode_int8(q, k, v, qs, ks, 49), what="int8 quirk")


def test_decode_int8_config5b_sampled(fa):
    """BASELINE config 5b: Q [16,32,1,128], K/V [16,8,2049,128], per-head absmax/127 scales."""
    g = gen(55)
    q, k, v = randn(g, 16, 32, 1, 128), randn(g, 16, 8, 2049, 128), randn(g, 16, 8, 2049, 128)
    qs, ks = int8_scales(q, k)
    out = fa.forward_decode_int8_gqa(*cuda(q, k, v, qs, ks), 2048).cpu()
    ref = A.decode_int8(q, k, v, qs, ks, 2048)
    assert rel_l2(out, ref) <= INT8_REL_L2
    assert_close(out, ref, what="cfg5b")


# ---------------------------------------------------------------- transfer helpers and the overlapped decode step

def test_alloc_pinned_tensor(fa):
    """test_async.py:146-164: dtype code 5 is float16, the tensor is page-locked host memory."""
    t = fa.alloc_pinned_tensor([2, 8, 512, 64], 5)
    assert list(t.shape) == [2, 8, 512, 64] and t.dtype == torch.float16
    assert t.device.type == "cpu" and t.is_pinned()


def test_async_h2d_transfer(fa):
    """test_async.py:115-143: a pinned host tensor copied on a side stream arrives intact."""
    g = gen(5)
    src = fa.alloc_pinned_tensor([2, 8, 1, 64], 5)
    src.copy_(randn(g, 2, 8, 1, 64))
    dst = torch.empty(2, 8, 1, 64, dtype=torch.float16, device=DEV)
    st = torch.cuda.Stream()
    fa.async_h2d_transfer(dst, src, st.cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(dst.cpu(), src)
    with pytest.raises(RuntimeError):
        fa.async_h2d_transfer(dst, src.clone(), st.cuda_stream)  # not pinned
    with pytest.raises(RuntimeError):
        fa.async_h2d_transfer(dst, src.to(DEV), st.cuda_stream)  # not a host tensor


@pytest.mark.parametrize("use_out", [True, False])
def test_pipeline_decode_step(fa, use_out):
    """test_async.py:166-214: decode on the compute stream equals forward_decode_gqa_fp16, the
    three host-to-device copies on the transfer stream land, and _out returns the caller's buffer."""
    B, H_Q, H_KV, N, D = 2, 8, 2, 512, 64
    g = gen(42)
    q, k, v = randn(g, B, H_Q, 1, D), randn(g, B, H_KV, N, D), randn(g, B, H_KV, N, D)
    qc, kc, vc = cuda(q, k, v)
    host = [fa.alloc_pinned_tensor(list(s), 5) for s in ([B, H_Q, 1, D], [B, H_KV, N, D], [B, H_KV, N, D])]
    for h in host:
        h.copy_(randn(g, *h.shape))
    dst = [torch.empty(h.shape, dtype=torch.float16, device=DEV) for h in host]
    cs, ts = torch.cuda.Stream(), torch.cuda.Stream()
    if use_out:
        out_buf = torch.empty(B, H_Q, 1, D, dtype=torch.float16, device=DEV)
        out, q_dst, k_dst = fa.pipeline_decode_step_out(out_buf, qc, kc, vc, *host, *dst, True, 0,
                                                        cs.cuda_stream, ts.cuda_stream)
        assert out.data_ptr() == out_buf.data_ptr()
    else:
        out, q_dst, k_dst = fa.pipeline_decode_step(qc, kc, vc, *host, *dst, True, 0, cs.cuda_stream, ts.cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(out, fa.forward_decode_gqa_fp16(qc, kc, vc, True, 0))
    assert_close(out, A.decode(q, k, v, True, 0), what="pipeline decode")
    assert q_dst.data_ptr() == dst[0].data_ptr() and k_dst.data_ptr() == dst[1].data_ptr()
    for d_, h in zip(dst, host):
        assert torch.equal(d_.cpu(), h)
    with pytest.raises(RuntimeError):
        fa.pipeline_decode_step(qc, kc, vc, host[0].clone(), *host[1:], *dst, True, 0,
                                cs.cuda_stream, ts.cuda_stream)  # unpinned source


def test_decode_graph_capture_replays(fa):
    """Decode calls captured in a HIP graph (no memset nodes: the split workspace already exists
    on the capture stream) replay to the eager results, with eager work between replays."""
    g = gen(9)
    sets = [(randn(g, 1, 32, 1, 128), randn(g, 1, 8, 1025, 128), randn(g, 1, 8, 1025, 128)) for _ in range(3)]
    dev = [cuda(*s) for s in sets]
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        for q, k, v in dev:
            fa.forward_decode_gqa_fp16(q, k, v, True, 1024)
    st.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        outs = [fa.forward_decode_gqa_fp16(q, k, v, True, 1024) for q, k, v in dev]
    refs = [A.decode(q, k, v, True, 1024) for q, k, v in sets]
    for _ in range(3):
        eager = [fa.forward_decode_gqa_fp16(q, k, v, True, 1024) for q, k, v in dev]
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for o, e, r in zip(outs, eager, refs):
            assert torch.equal(o, e)
            assert_close(o, r, what="graph replay")


def test_decode_graph_survives_workspace_growth_on_its_stream(fa):
    """Capture on a stream, then make a larger eager decode call on that same
    stream (which grows the eager workspace) and allocate more memory: the
    captured graph keeps its own workspace, so every replay still matches the
    eager result and the new allocations keep their contents."""
    g = gen(10)
    small = (randn(g, 1, 32, 1, 128), randn(g, 1, 8, 1025, 128), randn(g, 1, 8, 1025, 128))
    big = (randn(g, 4, 32, 1, 128), randn(g, 4, 8, 16385, 128), randn(g, 4, 8, 16385, 128))
    sd, bd = cuda(*small), cuda(*big)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        fa.forward_decode_gqa_fp16(*sd, True, 1024)
    st.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        out = fa.forward_decode_gqa_fp16(*sd, True, 1024)
    ref_small = A.decode(*small, True, 1024)
    with torch.cuda.stream(st):
        big_out = fa.forward_decode_gqa_fp16(*bd, True, 16384)  # grows the eager workspace of st
        filler = [torch.full((1 << 20,), float(i), device="cuda") for i in range(8)]
    st.synchronize()
    ref_big = A.decode(*big, True, 16384)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert_close(out, ref_small, what="graph replay after growth")
        with torch.cuda.stream(st):
            again = fa.forward_decode_gqa_fp16(*bd, True, 16384)
        st.synchronize()
        assert torch.equal(again, big_out)
    assert_close(big_out, ref_big, what="grown eager call")
    for i, f in enumerate(filler):
        assert torch.equal(f, torch.full_like(f, float(i)))


def test_decode_workspace_cache_many_streams(fa):
    """More streams than the eager pool keeps (8 per device): the least recently
    used buffers are dropped and remade, results unchanged."""
    g = gen(12)
    q, k, v = randn(g, 1, 32, 1, 128), randn(g, 1, 8, 4097, 128), randn(g, 1, 8, 4097, 128)
    qc, kc, vc = cuda(q, k, v)
    ref = fa.forward_decode_gqa_fp16(qc, kc, vc, True, 4096)
    assert_close(ref, A.decode(q, k, v, True, 4096), what="decode")
    torch.cuda.synchronize()
    for rnd in range(2):
        streams = [torch.cuda.Stream() for _ in range(20)]
        outs = []
        for s in streams:
            with torch.cuda.stream(s):
                outs.append(fa.forward_decode_gqa_fp16(qc, kc, vc, True, 4096))
        torch.cuda.synchronize()
        for o in outs:
            assert torch.equal(o, ref)


# ---------------------------------------------------------------- sliding-window decode

@pytest.mark.parametrize("b,hq,hkv,n,d,cache_len,window,sink", [
    (2, 8, 2, 512, 64, 300, 64, 4),        # sink + window, far apart
    (1, 32, 8, 4097, 128, 4096, 1024, 16),  # config-2-like shape, long window
    (2, 4, 4, 300, 128, 100, 200, 150),    # sink overlaps the window
    (1, 8, 2, 200, 64, 50, 8, 100),        # sink past cache_len (still attended)
    (1, 4, 1, 128, 256, 127, 1000, 0),     # window covers everything
    (1, 4, 2, 96, 80, 40, 0, 3),           # zero window: sink only, odd D
    (2, 4, 2, 64, 64, -1, 4, 0),           # nothing attended -> NaN
    (1, 4, 2, 64, 64, 500, 16, 2),         # cache_len >= N: window ends at N-1
])
def test_decode_sliding_window(fa, b, hq, hkv, n, d, cache_len, window, sink):
    g = gen(n + d + window)
    q, k, v = randn(g, b, hq, 1, d), randn(g, b, hkv, n, d), randn(g, b, hkv, n, d)
    out = fa.forward_decode_sliding_window_gqa(*cuda(q, k, v), True, cache_len, window, sink)
    assert_close(out, A.decode_sliding_window(q, k, v, cache_len, window, sink), what="sliding window")


def test_decode_sliding_window_validation(fa):
    x = torch.zeros(1, 4, 1, 64, dtype=torch.float16, device=DEV)
    kv = torch.zeros(1, 3, 32, 64, dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError):
        fa.forward_decode_sliding_window_gqa(x, kv, kv, True, 10, 4, 0)  # H_Q % H_KV != 0
    with pytest.raises(RuntimeError):
        fa.forward_decode_sliding_window_gqa(x.float(), kv, kv, True, 10, 4, 0)
    q2 = torch.zeros(1, 4, 2, 64, dtype=torch.float16, device=DEV)
    kv2 = torch.zeros(1, 2, 32, 64, dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError):
        fa.forward_decode_sliding_window_gqa(q2, kv2, kv2, True, 10, 4, 0)  # q_len != 1


# ---------------------------------------------------------------- INT8 KV-cache decode

def _int8_cache(g, b, hkv, n, d):
    """Per-token absmax/127 quantization of N(0,1) K/V (test_kv_compress.py:7-18 convention),
    with the extreme code -128 planted in a few places."""
    k, v = randn(g, b, hkv, n, d).float(), randn(g, b, hkv, n, d).float()
    ks, vs = k.abs().amax(-1) / 127, v.abs().amax(-1) / 127
    k8 = torch.clamp(torch.round(k / ks.unsqueeze(-1)), -127, 127).to(torch.int8)
    v8 = torch.clamp(torch.round(v / vs.unsqueeze(-1)), -127, 127).to(torch.int8)
    k8.view(-1)[::97] = -128
    v8.view(-1)[::89] = -128
    return k8, v8, ks.half(), vs.half()


@pytest.mark.parametrize("b,hq,hkv,n,d,cache_len", [
    (2, 8, 2, 512, 64, 300), (1, 32, 8, 4097, 128, 4096), (2, 4, 4, 300, 256, 299),
    (1, 8, 2, 200, 80, 150),      # odd D: element-wise path
    (1, 4, 1, 64, 128, 500),      # cache_len >= N: every key
    (2, 4, 2, 64, 64, -1),        # no key -> NaN
])
def test_decode_int8_kv_cache(fa, b, hq, hkv, n, d, cache_len):
    g = gen(n + d)
    q = randn(g, b, hq, 1, d)
    k8, v8, ks, vs = _int8_cache(g, b, hkv, n, d)
    out = fa.forward_decode_int8_kv_cache_gqa(*cuda(q, k8, v8, ks, vs), cache_len)
    assert_close(out, A.decode_int8_kv_cache(q, k8, v8, ks, vs, cache_len), what="int8 kv cache")


def test_decode_int8_kv_cache_unaligned_codes(fa):
    """K codes 8 bytes past a 16-byte boundary: the per-slice load path (the
    16-byte paired-slice loads need 16-byte-aligned rows)."""
    g = gen(4242)
    b, hq, hkv, n, d = 2, 8, 2, 333, 128
    q = randn(g, b, hq, 1, d)
    k8, v8, ks, vs = _int8_cache(g, b, hkv, n, d)
    buf = torch.empty(k8.numel() + 8, dtype=torch.int8, device="cuda")
    k8u = buf[8:].view(k8.shape)
    k8u.copy_(k8.cuda())
    assert k8u.data_ptr() % 16 == 8
    out = fa.forward_decode_int8_kv_cache_gqa(q.cuda(), k8u, v8.cuda(), ks.cuda(), vs.cuda(), 300)
    assert_close(out, A.decode_int8_kv_cache(q, k8, v8, ks, vs, 300), what="int8 kv cache, unaligned codes")


def test_decode_int8_kv_cache_validation(fa):
    q = torch.zeros(1, 4, 1, 64, dtype=torch.float16, device=DEV)
    k8 = torch.zeros(1, 2, 32, 64, dtype=torch.int8, device=DEV)
    s = torch.zeros(1, 2, 32, dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError):
        fa.forward_decode_int8_kv_cache_gqa(q, k8.half(), k8, s, s, 3)   # k not int8
    with pytest.raises(RuntimeError):
        fa.forward_decode_int8_kv_cache_gqa(q, k8, k8, s.float(), s, 3)  # scale not fp16
    with pytest.raises(RuntimeError):
        fa.forward_decode_int8_kv_cache_gqa(q, k8, k8, s[:, :, :16].contiguous(), s, 3)  # scale length


@pytest.mark.parametrize("b,hq,hkv,n,d", [(1, 8, 8, 128, 64), (2, 8, 2, 256, 64), (4, 16, 4, 512, 128)])
def test_int8_kv_cache_reference_case(fa, b, hq, hkv, n, d):
    """test_kv_compress.py:21-60: its quantizer (per-token absmax/127, scale >= 1e-8, codes
    clamped to [-128, 127]); the output matches the oracle on the int8 cache and stays within
    the reference's 0.1 of the fp16 decode on the unquantized cache."""
    g = gen(42)
    q, k, v = randn(g, b, hq, 1, d), randn(g, b, hkv, n, d), randn(g, b, hkv, n, d)

    def quant(x):
        s = (x.float().abs().amax(-1, keepdim=True) / 127.0).clamp(min=1e-8)
        return (x.float() / s).round().clamp(-128, 127).to(torch.int8), s.squeeze(-1).half()

    k8, ks = quant(k)
    v8, vs = quant(v)
    out = fa.forward_decode_int8_kv_cache_gqa(*cuda(q, k8, v8, ks, vs), n - 1)
    assert_close(out, A.decode_int8_kv_cache(q, k8, v8, ks, vs, n - 1), what="int8 kv reference case")
    assert (out.float().cpu() - A.decode(q, k, v, True, n - 1)).abs().max().item() < 0.1


def test_sliding_window_reference_case(fa):
    """test_kv_compress.py:231-290: B=2, 8:2 heads, N=256, D=64, cache_len=N-1, window 64, sink 4."""
    g = gen(42)
    q, k, v = randn(g, 2, 8, 1, 64), randn(g, 2, 2, 256, 64), randn(g, 2, 2, 256, 64)
    out = fa.forward_decode_sliding_window_gqa(*cuda(q, k, v), True, 255, 64, 4)
    assert_close(out, A.decode_sliding_window(q, k, v, 255, 64, 4), what="sliding reference case")


@pytest.mark.parametrize("n", [1025, 1087, 1088, 1089, 2049, 4097, 4160, 4161])
def test_decode_split_tail_boundaries(fa, n):
    """Fixed-length decode folds a key remainder of at most a quarter chunk into
    split 0 (256-key chunks here: remainders 1, 63, 64 folded; 65 not)."""
    g = gen(n)
    q, k, v = randn(g, 1, 32, 1, 128), randn(g, 1, 8, n, 128), randn(g, 1, 8, n, 128)
    out = fa.forward_decode_gqa_fp16(*cuda(q, k, v), True, n - 1)
    assert_close(out, A.decode(q, k, v, True, n - 1), what=f"decode tail n={n}")
    # the same sequence length through the INT8 path (same split plan)
    qs = (q.float().abs().amax(-1).squeeze(-1) / 127).contiguous()
    ks = (k.float().abs().amax((-1, -2)) / 127).unsqueeze(-1).expand(1, 8, n).contiguous()
    o8 = fa.forward_decode_int8_gqa(*cuda(q, k, v, qs, ks), n - 1)
    r8 = A.decode_int8(q, k, v, qs, ks, n - 1)
    assert rel_l2(o8, r8) <= INT8_REL_L2


@pytest.mark.parametrize("d", [64, 80, 128, 256])
@pytest.mark.parametrize("n", [129, 257, 300, 513])
def test_decode_small_grid_two_tile_waves(fa, d, n):
    """Small contiguous decode grids (no LDS staging) split at 128 keys; a wave
    with exactly two tiles (every wave at D = 256, whose tiles are 16 keys; the
    waves of split 0 that take the folded remainder) loads both tiles before
    computing either.  Against the oracle at several head dims (80: rows not
    16-byte multiples) and group sizes, and through the sliding-window entry."""
    for hq, hkv in ((8, 2), (4, 4), (16, 2)):
        g = gen(7000 + 13 * d + n + hq)
        q, k, v = randn(g, 1, hq, 1, d), randn(g, 1, hkv, n, d), randn(g, 1, hkv, n, d)
        out = fa.forward_decode_gqa_fp16(*cuda(q, k, v), True, n - 1)
        assert_close(out, A.decode(q, k, v, True, n - 1), what=f"two-tile decode d={d} n={n} {hq}:{hkv}")
    sw = fa.forward_decode_sliding_window_gqa(*cuda(q, k, v), True, n - 1, n // 2, 4)
    assert_close(sw, A.decode_sliding_window(q, k, v, n - 1, n // 2, 4), what=f"two-tile window d={d} n={n}")


@pytest.mark.parametrize("mode", ["decode", "window", "int8", "cb"])
def test_decode_long_context(fa, mode):
    """One sequence of 300001 keys (8:2 heads): the split length is capped by
    the 128-split limit rather than the workgroup target, against the oracle."""
    n, d = 300001, 128
    g = gen(31000 + len(mode))
    q, k, v = randn(g, 1, 8, 1, d), randn(g, 1, 2, n, d), randn(g, 1, 2, n, d)
    if mode == "decode":
        out = fa.forward_decode_gqa_fp16(*cuda(q, k, v), True, n - 1)
        assert_close(out, A.decode(q, k, v, True, n - 1), what="long-context decode")
    elif mode == "window":
        out = fa.forward_decode_sliding_window_gqa(*cuda(q, k, v), True, n - 1, 70000, 64)
        assert_close(out, A.decode_sliding_window(q, k, v, n - 1, 70000, 64), what="long-context window")
    elif mode == "int8":
        qs = (q.float().abs().amax(-1).squeeze(-1) / 127).contiguous()
        ks = (k.float().abs().amax((-1, -2)) / 127).unsqueeze(-1).expand(1, 2, n).contiguous()
        o8 = fa.forward_decode_int8_gqa(*cuda(q, k, v, qs, ks), n - 1)
        assert rel_l2(o8, A.decode_int8(q, k, v, qs, ks, n - 1)) <= INT8_REL_L2
    else:
        # continuous batching: two sequences of the same cache, 300000 and 150000 cached keys
        q2, k2, v2 = torch.cat([q, q.flip(1)]), torch.cat([k, k.flip(1)]), torch.cat([v, v.flip(1)])
        cl = torch.tensor([n - 1, 150000], dtype=torch.int32)
        out = fa.forward_continuous_batching_fp16(*cuda(q2, k2, v2, cl), True)
        assert_close(out, A.continuous_batching(q2, k2, v2, cl, True), what="long-context continuous batching")


# ---------------------------------------------------------------- many-unit fixed-length launches

@pytest.mark.parametrize("mode", ["decode", "window", "int8_cache"])
def test_fixed_length_many_units(fa, mode):
    """B=16 with 8 KV heads: 128 (batch, KV head) units, so fixed-length decode
    deals its splits split-major (every split index of every unit before the
    next split index); each mode against the oracle on every output row."""
    b, hq, hkv, n, d, cl = 16, 32, 8, 1537, 128, 1536
    g = gen(1600 + len(mode))
    q = randn(g, b, hq, 1, d)
    if mode == "int8_cache":
        k8, v8, ks, vs = _int8_cache(g, b, hkv, n, d)
        out = fa.forward_decode_int8_kv_cache_gqa(*cuda(q, k8, v8, ks, vs), cl)
        ref = A.decode_int8_kv_cache(q, k8, v8, ks, vs, cl)
    else:
        k, v = randn(g, b, hkv, n, d), randn(g, b, hkv, n, d)
        if mode == "decode":
            out = fa.forward_decode_gqa_fp16(*cuda(q, k, v), True, cl)
            ref = A.decode(q, k, v, True, cl)
        else:
            out = fa.forward_decode_sliding_window_gqa(*cuda(q, k, v), True, cl, 1024, 64)
            ref = A.decode_sliding_window(q, k, v, cl, 1024, 64)
    assert_close(out, ref, what=f"{mode} many units")


def test_decode_more_units_than_counter_slots(fa):
    """65537 (batch, head) units with two splits each: more units than the
    workspace's 65536 arrival counters, so the call is issued as two launches
    over unit ranges (the second reusing the counters the first left at zero).
    Each half of the batch run as a call of its own (one launch, same split
    plan) gives the same rows bit for bit; rows at the launch boundary and the
    ends against the oracle.  D=8 keeps the 8256-key cache at 17 GB."""
    b, n, d = 65537, 8256, 8
    cl = n - 1
    g = torch.Generator(device="cuda").manual_seed(65537)
    q = torch.randn(b, 1, 1, d, generator=g, device="cuda", dtype=torch.float16)
    k = torch.randn(b, 1, n, d, generator=g, device="cuda", dtype=torch.float16)
    v = torch.randn(b, 1, n, d, generator=g, device="cuda", dtype=torch.float16)
    out = fa.forward_decode_gqa_fp16(q, k, v, True, cl)
    h = 32768
    lo = fa.forward_decode_gqa_fp16(q[:h], k[:h], v[:h], True, cl)
    hi = fa.forward_decode_gqa_fp16(q[h:], k[h:], v[h:], True, cl)
    torch.cuda.synchronize()
    assert torch.equal(out[:h], lo)
    assert torch.equal(out[h:], hi)
    for row in (0, h - 1, h, 65535, 65536):
        sl = slice(row, row + 1)
        ref = A.decode(q[sl].cpu(), k[sl].cpu(), v[sl].cpu(), True, cl)
        assert_close(out[sl], ref, what=f"decode row {row} of 65537 units")
    del k, v


@pytest.mark.parametrize("mode", ["decode", "window", "int8"])
@pytest.mark.parametrize("d,n", [(64, 2049), (256, 2049), (64, 3329), (256, 3329), (128, 3329)])
def test_fixed_length_lds_k_head_dims(fa, mode, d, n):
    """B=16, 32:8 heads: 128 units in 4 (n=2049) or 5 (n=3329, an odd split
    count) splits, i.e. 512-640 workgroups, the launches that stage K in LDS by
    row-coalesced copies; D=64 (two rows per swizzle) and D=256 (two copies per
    row) take other copy shapes than D=128.  Every output row against the oracle."""
    b, hq, hkv = 16, 32, 8
    cl = n - 1
    g = gen(7000 + d + n + len(mode))
    q, k, v = randn(g, b, hq, 1, d), randn(g, b, hkv, n, d), randn(g, b, hkv, n, d)
    if mode == "decode":
        out = fa.forward_decode_gqa_fp16(*cuda(q, k, v), True, cl)
        assert_close(out, A.decode(q, k, v, True, cl), what=f"decode d={d} n={n}")
    elif mode == "window":
        out = fa.forward_decode_sliding_window_gqa(*cuda(q, k, v), True, cl, n - 100, 64)
        assert_close(out, A.decode_sliding_window(q, k, v, cl, n - 100, 64), what=f"window d={d} n={n}")
    else:
        qs = (q.float().abs().amax(-1).squeeze(-1) / 127).contiguous()
        ks = (k.float().abs().amax((-1, -2)) / 127).unsqueeze(-1).expand(b, hkv, n).contiguous()
        out = fa.forward_decode_int8_gqa(*cuda(q, k, v, qs, ks), cl)
        ref = A.decode_int8(q, k, v, qs, ks, cl)
        assert rel_l2(out, ref) <= INT8_REL_L2
        # per row as well: a wrong row cannot hide in the global norm
        for bb in range(b):
            assert rel_l2(out[bb:bb + 1], ref[bb:bb + 1]) <= INT8_REL_L2, f"int8 d={d} n={n} row {bb}"


@pytest.mark.parametrize("d", [64, 256])
def test_continuous_batching_many_splits_head_dims(fa, d):
    """Continuous batching (K staged in LDS) at D=64 and D=256 with sequences long
    enough for several splits each, plus an empty and a one-key sequence;
    every output row against the oracle."""
    g = gen(900 + d)
    b, hq, hkv, max_n = 6, 16, 4, 3001
    cls = torch.tensor([3000, 1, 2047, -1, 1500, 2999], dtype=torch.int32)
    q, k, v = randn(g, b, hq, 1, d), randn(g, b, hkv, max_n, d), randn(g, b, hkv, max_n, d)
    out = fa.forward_continuous_batching_fp16(*cuda(q, k, v, cls), True)
    assert_close(out, A.continuous_batching(q, k, v, cls, True), what=f"cb d={d}")


@pytest.mark.parametrize("d", [64, 256])
def test_paged_decode_many_splits_head_dims(fa, d):
    """Paged decode at D=64 and D=256 over a random page permutation with
    sequences of several splits (up to 3000 tokens)."""
    g = gen(950 + d)
    b, hq, hkv, mnb, npages = 5, 16, 4, 200, 1000
    sl = torch.tensor([3000, 17, 1999, 16, 2500], dtype=torch.int32)
    bt = torch.randperm(npages, generator=g)[: b * mnb].view(b, mnb).int()
    kc, vc = randn(g, npages, hkv, 16, d), randn(g, npages, hkv, 16, d)
    q = randn(g, b, hq, 1, d)
    out = fa.forward_paged_decode_gqa_fp16(*cuda(q, kc, vc, bt, sl), mnb)
    assert_close(out, A.paged_decode(q, kc, vc, bt, sl, mnb), what=f"paged d={d}")
