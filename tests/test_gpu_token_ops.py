"""GPU parity of token_eviction against the CPU oracle: bit-exact outputs and
mask (pure index and copy work), including ties (stable order), num_evict at
0, N and beyond, N up to the 1024 limit, and D not a multiple of 8."""
import pytest
import numpy as np
import torch

from oracle import attention as A
from tests.helpers import randn

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("b,h,n,d,num_evict,ties", [
    (1, 1, 1, 64, 0, False), (1, 1, 1, 64, 1, False), (2, 3, 7, 64, 3, True), (2, 8, 33, 128, 10, True),
    (3, 2, 255, 128, 100, False), (2, 2, 256, 64, 256, False), (2, 4, 1000, 128, 250, True),
    (1, 8, 1024, 128, 512, False), (2, 2, 300, 36, 77, True), (2, 2, 64, 128, -5, False),
    (1, 2, 50, 128, 80, True),
    (16, 8, 1024, 128, 256, False),  # 512 output rows per workgroup (the bench shape)
    (8, 8, 1024, 128, 300, True),    # 256 rows per workgroup
    (16, 16, 700, 64, 123, True),    # 512 rows per workgroup, ragged last block
])
def test_token_eviction(fa, b, h, n, d, num_evict, ties):
    g = torch.Generator().manual_seed(n + d + num_evict)
    k, v = randn(g, b, h, n, d), randn(g, b, h, n, d)
    if ties:
        sc = torch.randint(0, 7, (b, n), generator=g).float() * 0.25
    else:
        sc = torch.randn(b, n, generator=g)
    ko, vo, m = fa.token_eviction(k.cuda(), v.cuda(), sc.cuda(), num_evict)
    rk, rv, rm = A.token_eviction(k, v, sc, num_evict)
    assert m.dtype == torch.int32 and ko.dtype == torch.float16
    assert torch.equal(m.cpu(), rm)
    assert torch.equal(ko.cpu(), rk)
    assert torch.equal(vo.cpu(), rv)


@pytest.mark.parametrize("pattern", ["signed_zeros", "all_equal", "extremes", "few_distinct"])
@pytest.mark.parametrize("n,num_evict", [(1024, 1), (1024, 1023), (700, 350), (129, 64)])
def test_token_eviction_score_patterns(fa, pattern, n, num_evict):
    """The keep mask comes from a radix select over order-preserving keys:
    -0.0 and +0.0 tie (stable order decides), equal scores, infinities and
    values straddling the sign."""
    g = torch.Generator().manual_seed(n * 7 + num_evict)
    b, h, d = 2, 3, 64
    k, v = randn(g, b, h, n, d), randn(g, b, h, n, d)
    if pattern == "signed_zeros":
        sc = torch.tensor([0.0, -0.0, 1.0, -1.0])[torch.randint(0, 4, (b, n), generator=g)]
    elif pattern == "all_equal":
        sc = torch.full((b, n), -2.5)
    elif pattern == "extremes":
        vals = torch.tensor([float("-inf"), -3.4e38, -1e-45, 0.0, 1e-45, 3.4e38, float("inf")])
        sc = vals[torch.randint(0, vals.numel(), (b, n), generator=g)]
    else:
        sc = torch.randint(-2, 3, (b, n), generator=g).float() * 1e-3
    ko, vo, m = fa.token_eviction(k.cuda(), v.cuda(), sc.cuda(), num_evict)
    rk, rv, rm = A.token_eviction(k, v, sc, num_evict)
    assert torch.equal(m.cpu(), rm)
    assert torch.equal(ko.cpu(), rk)
    assert torch.equal(vo.cpu(), rv)


def test_token_eviction_validation(fa):
    k = torch.zeros(1, 2, 8, 64, dtype=torch.float16, device="cuda")
    sc = torch.zeros(1, 8, device="cuda")
    with pytest.raises(RuntimeError):
        fa.token_eviction(k, k, sc[:, :4].contiguous(), 1)  # length mismatch
    with pytest.raises(RuntimeError):
        fa.token_eviction(k, k, sc.double(), 1)  # dtype
    big = torch.zeros(1, 1, 1025, 64, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError):
        fa.token_eviction(big, big, torch.zeros(1, 1025, device="cuda"), 1)  # N > 1024


# ---------------------------------------------------------------- speculative verify

def _spec(seed, B, K, V, same=False, zero_rand=False):
    g = torch.Generator().manual_seed(seed)
    tp = torch.softmax(torch.randn(B, K + 1, V, generator=g), -1)
    dp = tp[:, :K].clone() if same else torch.softmax(torch.randn(B, K, V, generator=g), -1)
    tok = torch.randint(0, V, (B, K), generator=g)
    rv = torch.zeros(B, K) if zero_rand else torch.rand(B, K, generator=g)
    return tp, dp, tok, rv


def _check_spec(fa, tp, dp, tok, rv, K):
    acc, out = fa.speculative_verify(tp.cuda(), dp.cuda(), tok.cuda(), rv.cuda(), K)
    racc, rout = A.speculative_verify(tp, dp, tok, rv, K)
    assert acc.dtype == torch.int32 and out.dtype == torch.int64
    assert torch.equal(acc.cpu(), racc), (acc.cpu(), racc)
    assert torch.equal(out.cpu(), rout), (out.cpu(), rout)


@pytest.mark.parametrize("seed,B,K,V,same,zero_rand", [
    (42, 2, 4, 256, False, False),    # test_speculative.py:115-157
    (42, 4, 5, 128, True, True),      # :160-196 all accepted
    (7, 2, 3, 32000, False, False),   # :240- large vocabulary
    (3, 16, 8, 1000, False, False), (4, 3, 1, 257, False, False), (5, 8, 4, 4099, False, False),
    (6, 4, 2, 1, False, False),       # one-word vocabulary
    (8, 4, 3, 63, False, False),      # less than one 64-term batch
    (9, 6, 2, 2049, False, False),    # one element into a second staged chunk
    (10, 3, 2, 4096, False, False),   # exactly two chunks
])
def test_speculative_verify(fa, seed, B, K, V, same, zero_rand):
    _check_spec(fa, *_spec(seed, B, K, V, same, zero_rand), K)


def test_speculative_verify_orthogonal(fa):
    """test_speculative.py:199-236: disjoint one-hot supports, r = 0.5: rejection at 0."""
    B, K, V = 2, 4, 64
    tp = torch.zeros(B, K + 1, V)
    dp = torch.zeros(B, K, V)
    for i in range(K + 1):
        tp[:, i, (i * 10) % V] = 1.0
    for i in range(K):
        dp[:, i, (i * 10 + 1) % V] = 1.0
    _check_spec(fa, tp, dp, torch.full((B, K), 1), torch.full((B, K), 0.5), K)


def test_speculative_verify_residual_zero(fa):
    """Draft dominates target everywhere it differs (Z == 0 path: sample from target)."""
    B, K, V = 2, 2, 300
    g = torch.Generator().manual_seed(11)
    tp = torch.softmax(torch.randn(B, K + 1, V, generator=g), -1)
    dp = tp[:, :K].clone()
    tok = torch.randint(0, V, (B, K), generator=g)
    rv = torch.ones(B, K)  # r = 1 is never < accept_prob <= 1: reject at step 0 with Z == 0
    _check_spec(fa, tp, dp, tok, rv, K)


def test_speculative_verify_zero_hit_across_chunks(fa):
    """A residual hit at index 0 defers to the next contributing index, 1500
    elements (more than one 1024-element scan chunk) later."""
    V = 3000
    g = torch.Generator().manual_seed(12)
    tp = torch.zeros(1, 2, V)
    tp[0, 0, 0] = tp[0, 0, 1500] = 0.5
    tp[0, 1] = torch.softmax(torch.randn(V, generator=g), -1)
    dp = torch.full((1, 1, V), 1.0 / (V - 2))
    dp[0, 0, 0] = dp[0, 0, 1500] = 0.0
    tok = torch.tensor([[7]])  # target mass 0: rejected at step 0
    rv = torch.tensor([[0.3]])
    _check_spec(fa, tp, dp, tok, rv, 1)
    _, rout = A.speculative_verify(tp, dp, tok, rv, 1)
    assert int(rout[0, 0]) == 1500


def test_speculative_verify_residual_at_a_running_sum(fa):
    """r equal to one of the residual scan's own fp32 running sums, so the
    sampled index depends on every rounding of the serial sum over the
    contributing terms (about half of a row, spread over several scan chunks
    and a ragged tail)."""
    V = 5003
    g = torch.Generator().manual_seed(13)
    tp = torch.softmax(torch.randn(1, 2, V, generator=g), -1)
    dp = torch.softmax(torch.randn(1, 1, V, generator=g), -1)
    d = (tp[0, 0] - dp[0, 0]).numpy().astype(np.float32)
    z = np.float32(0.0)
    for x in d:
        if x > 0:
            z = np.float32(z + x)
    cs, sums = np.float32(0.0), []
    for v, x in enumerate(d):
        if x > 0:
            cs = np.float32(cs + np.float32(x / z))
            sums.append((v, cs))
    ratio = (tp[0, 0] / (dp[0, 0] + 1e-10)).numpy()
    tok = int(np.argmin(ratio))  # least acceptable draft token: rejected once r >= its ratio
    j = next(i for i, (_, c) in enumerate(sums) if c > max(0.6, float(ratio[tok])))
    r = float(sums[j][1])
    tokt, rv = torch.tensor([[tok]]), torch.tensor([[r]], dtype=torch.float32)
    _check_spec(fa, tp, dp, tokt, rv, 1)
    _, rout = A.speculative_verify(tp, dp, tokt, rv, 1)
    assert int(rout[0, 0]) > sums[j][0]  # the first index whose running sum exceeds r


def _adversarial_rows(g, shape, kind):
    """Non-negative float32 rows that stress the exact fp32 running sums: few
    mantissa bits (round-half-to-even ties and exact binade ends), a dynamic
    range down to subnormals, mostly zeros, or typical softmax values."""
    if kind == "ties":
        m = torch.randint(0, 16, shape, generator=g).float()
        e = torch.randint(8, 24, shape, generator=g).float()
        return (m * torch.exp2(-e)).float()
    if kind == "range":
        e = torch.randint(0, 140, shape, generator=g).float()
        return (torch.rand(shape, generator=g) * torch.exp2(-e)).float()
    if kind == "sparse":
        x = torch.rand(shape, generator=g) * 1e-3
        return torch.where(torch.rand(shape, generator=g) < 0.8, torch.zeros(shape), x).float()
    return torch.softmax(torch.randn(shape, generator=g), -1)


@pytest.mark.parametrize("kind", ["ties", "range", "sparse", "softmax"])
@pytest.mark.parametrize("V", [700, 5000, 32000])
def test_speculative_verify_exact_sums(fa, kind, V):
    """Every scan (Z, the residual sample, the sample from the target, the
    bonus) against the oracle's serial float32 loops on rows built to make the
    sums' rounding matter, with r set to one of the bonus scan's own running
    sums (hit exactly at the boundary) on half of the rows."""
    B, K = 8, 2
    g = torch.Generator().manual_seed(900 + V + len(kind))
    tp = _adversarial_rows(g, (B, K + 1, V), kind)
    dp = _adversarial_rows(g, (B, K, V), kind)
    dp[1] = tp[1, :K]  # Z == 0 rows: sample from the target itself
    tok = torch.randint(0, V, (B, K), generator=g)
    rv = torch.rand(B, K, generator=g)
    for b in range(0, B, 2):
        # every step accepted (a token the target gives at least the draft's
        # mass, r < 1), so the bonus scan of row K runs with r = r_{K-1}, set
        # to one of that scan's own running sums
        tok[b] = (tp[b, :K] - dp[b, :K]).argmax(-1)
        cs = np.cumsum(tp[b, K].numpy().astype(np.float32), dtype=np.float32)
        j = int(torch.randint(0, V, (1,), generator=g))
        rv[b] = 0.0
        if 0 < cs[j] < 1:
            rv[b, K - 1] = float(cs[j])
    _check_spec(fa, tp, dp, tok, rv, K)


def test_speculative_verify_non_monotone_rows(fa):
    """Rows with negative and non-finite entries (outside the probability
    contract) take the plain serial loop and still match the serial oracle."""
    B, K, V = 4, 2, 3000
    g = torch.Generator().manual_seed(77)
    tp = torch.softmax(torch.randn(B, K + 1, V, generator=g), -1)
    dp = torch.softmax(torch.randn(B, K, V, generator=g), -1)
    tp[0, K, 100:110] = -1e-3
    tp[1, :, 2500] = float("inf")
    tp[2, K, 5] = float("nan")
    tok = torch.randint(0, V, (B, K), generator=g)
    rv = torch.rand(B, K, generator=g)
    _check_spec(fa, tp, dp, tok, rv, K)


def test_speculative_verify_validation(fa):
    tp = torch.rand(1, 3, 10, device="cuda")
    dp = torch.rand(1, 2, 10, device="cuda")
    tok = torch.zeros(1, 2, dtype=torch.int64, device="cuda")
    rv = torch.rand(1, 2, device="cuda")
    with pytest.raises(RuntimeError):
        fa.speculative_verify(tp, dp, tok, rv, 3)  # positions mismatch
    with pytest.raises(RuntimeError):
        fa.speculative_verify(tp, dp, tok.int(), rv, 2)  # token dtype
    with pytest.raises(RuntimeError):
        fa.speculative_verify(torch.rand(1, 10, 10, device="cuda"), dp, tok, rv, 9)  # K > 8
