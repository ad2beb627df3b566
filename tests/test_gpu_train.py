"""GPU parity of the training path: forward with log-sum-exp (fp32 and fp16),
fp32 forward, and the backward (dq, dk, dv), against the CPU oracle.

Cases follow the reference's test_backward.py (B=2, H=3, N=17, D=32; seeds 11
for the LSE forwards, 7 for the backward, through the autograd wrapper) plus
ragged lengths, D not a multiple of 8, D in {16..128} and longer sequences.
Tolerances: fp32 max-abs 2e-4 + rtol 2e-4 (the reference's fp32 bound);
fp16 forward max-abs 2e-3 + rtol 1e-2; fp16 LSE max-abs 2e-3; fp16 gradients
max-abs 3e-2 + rtol 3e-2 (the reference's fp16 bound) and rel-L2 <= 1e-2.
"""
import pytest
import torch

from oracle import attention as A
from tests.helpers import assert_close, randn, rel_l2

pytestmark = pytest.mark.gpu
F64 = torch.float64


def gen(seed):
    return torch.Generator().manual_seed(seed)


def cuda(*ts):
    return [t.cuda().contiguous() for t in ts]


SHAPES = [(2, 3, 17, 32), (1, 2, 1, 64), (1, 2, 33, 64), (1, 2, 129, 128), (2, 2, 200, 80),
          (1, 1, 70, 36), (1, 2, 45, 16), (1, 3, 300, 128), (1, 2, 96, 100)]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("b,h,n,d", SHAPES)
def test_forward_with_lse_fp32(fa, causal, b, h, n, d):
    g = gen(11 + n + d)
    q, k, v = (randn(g, b, h, n, d, dtype=torch.float32) for _ in range(3))
    out, lse = fa.forward_with_lse(*cuda(q, k, v), causal)
    ro, rl = A.prefill_lse(q, k, v, causal, compute_dtype=F64)
    assert out.dtype == torch.float32 and lse.dtype == torch.float32 and lse.shape == (b, h, n)
    assert_close(out, ro, atol=2e-4, rtol=2e-4, what="forward_with_lse out")
    assert_close(lse, rl, atol=2e-4, rtol=2e-4, what="forward_with_lse lse")
    out2 = fa.forward(*cuda(q, k, v), causal)
    assert torch.equal(out2, out)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("b,h,n,d", SHAPES)
def test_forward_fp16_with_lse(fa, causal, b, h, n, d):
    g = gen(11 + n + d)
    q, k, v = (randn(g, b, h, n, d) for _ in range(3))
    qc, kc, vc = cuda(q, k, v)
    out, lse = fa.forward_fp16_with_lse(qc, kc, vc, causal)
    ro, rl = A.prefill_lse(q, k, v, causal, compute_dtype=F64)
    assert out.dtype == torch.float16 and lse.dtype == torch.float32 and lse.shape == (b, h, n)
    assert_close(out, ro, what="forward_fp16_with_lse out")
    assert_close(lse, rl, atol=2e-3, rtol=0, what="forward_fp16_with_lse lse")
    # same kernel as forward_fp16: identical output
    assert torch.equal(out, fa.forward_fp16(qc, kc, vc, causal))


def _check_grads(got, ref, fp16, what):
    for name, a, r in zip(("dq", "dk", "dv"), got, ref):
        if fp16:
            assert_close(a, r, atol=3e-2, rtol=3e-2, what=f"{what} {name}")
            if r.double().norm() > 1e-3:  # rel-L2 is undefined for an all-zero gradient (N=1 dq)
                assert rel_l2(a, r) <= 1e-2, (what, name, rel_l2(a, r))
        else:
            assert_close(a, r, atol=2e-4, rtol=2e-4, what=f"{what} {name}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("causal", [True, False])
def test_backward_reference_case(fa, dtype, causal):
    """test_backward.py:33-71 through the autograd wrapper (flash_attn_autograd.flash_attn)."""
    from flash_attn_autograd import flash_attn

    g = gen(7)
    B, H, N, D = 2, 3, 17, 32
    q, k, v, do = (randn(g, B, H, N, D, dtype=dtype) for _ in range(4))
    qg, kg, vg = (t.cuda().requires_grad_(True) for t in (q, k, v))
    out = flash_attn(qg, kg, vg, causal=causal)
    out.backward(do.cuda())
    ro, rl = A.prefill_lse(q, k, v, causal, compute_dtype=F64)
    ref = A.backward(do, q, k, v, ro, rl, causal)
    assert qg.grad.dtype == dtype
    _check_grads((qg.grad, kg.grad, vg.grad), ref, dtype == torch.float16, "autograd")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("causal", [True, False])
# (3, 4, 333, 128) and (2, 5, 150, 64): at least 8 (batch, head) units (the
# XCD-grouped block order) with a partial last tile
@pytest.mark.parametrize("b,h,n,d", SHAPES[1:] + [(1, 2, 512, 128), (2, 2, 257, 64), (3, 4, 333, 128), (2, 5, 150, 64)])
def test_backward_shapes(fa, dtype, causal, b, h, n, d):
    g = gen(300 + n * 3 + d)
    q, k, v, do = (randn(g, b, h, n, d, dtype=dtype) for _ in range(4))
    qc, kc, vc, dc = cuda(q, k, v, do)
    fwd = fa.forward_fp16_with_lse if dtype == torch.float16 else fa.forward_with_lse
    out, lse = fwd(qc, kc, vc, causal)
    dq, dk, dv = fa.backward(dc, qc, kc, vc, out, lse, causal)
    # the oracle takes the same out/lse the kernels were given
    ref = A.backward(do, q, k, v, out.cpu(), lse.cpu(), causal)
    _check_grads((dq, dk, dv), ref, dtype == torch.float16, f"backward {b,h,n,d}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_backward_grouped_units_with_padding(fa, dtype):
    """Causal calls deal each XCD's (batch, head) units in groups of 4, the
    blocks of a group heaviest first: 40 units (5 per XCD, so a full group
    and a group of one unit plus three padding slots) over 3 blocks of 128
    rows with a partial last block; every gradient against the oracle."""
    b, h, n, d = 5, 8, 300, 128
    g = gen(4141)
    q, k, v, do = (randn(g, b, h, n, d, dtype=dtype) for _ in range(4))
    qc, kc, vc, dc = cuda(q, k, v, do)
    fwd = fa.forward_fp16_with_lse if dtype == torch.float16 else fa.forward_with_lse
    out, lse = fwd(qc, kc, vc, True)
    dq, dk, dv = fa.backward(dc, qc, kc, vc, out, lse, True)
    ref = A.backward(do, q, k, v, out.cpu(), lse.cpu(), True)
    _check_grads((dq, dk, dv), ref, dtype == torch.float16, "grouped units")
    # the fp32 forward's causal grid is dealt the same way
    if dtype == torch.float32:
        ro, rl = A.prefill_lse(q, k, v, True, compute_dtype=F64)
        assert_close(out, ro, atol=2e-4, rtol=2e-4, what="grouped fp32 forward")
        assert_close(lse, rl, atol=2e-4, rtol=2e-4, what="grouped fp32 lse")


def test_backward_deterministic(fa):
    g = gen(5)
    q, k, v, do = (randn(g, 1, 4, 333, 64) for _ in range(4))
    qc, kc, vc, dc = cuda(q, k, v, do)
    out, lse = fa.forward_fp16_with_lse(qc, kc, vc, True)
    a = fa.backward(dc, qc, kc, vc, out, lse, True)
    b = fa.backward(dc, qc, kc, vc, out, lse, True)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_training_validation_errors(fa):
    q = torch.randn(1, 2, 8, 256, device="cuda", dtype=torch.float16)
    with pytest.raises(RuntimeError):
        fa.forward_fp16_with_lse(q, q, q, True)  # D > 128
    q32 = torch.randn(1, 2, 8, 64, device="cuda")
    with pytest.raises(RuntimeError):
        fa.forward_with_lse(q32.half(), q32.half(), q32.half(), True)  # dtype
    with pytest.raises(RuntimeError):
        fa.forward(q32, q32[:, :1].contiguous(), q32, True)  # shapes
    out, lse = fa.forward_with_lse(q32, q32, q32, True)
    with pytest.raises(RuntimeError):
        fa.backward(q32, q32, q32, q32, out, lse[:, :1].contiguous(), True)  # lse shape
    with pytest.raises(RuntimeError):
        fa.backward(q32, q32, q32, q32, out, lse.double(), True)  # lse dtype
    with pytest.raises(RuntimeError):
        fa.backward(q32.half(), q32, q32, q32, out, lse, True)  # dout dtype


def test_backward_bench_shape_sampled(fa):
    """Config 7's full shape (B=4 H=16 N=2048 D=128 causal, fp16): every gradient
    computed on the GPU, three (batch, head) slices checked against the oracle."""
    g = gen(70)
    B, H, N, D = 4, 16, 2048, 128
    q, k, v, do = (randn(g, B, H, N, D) for _ in range(4))
    qc, kc, vc, dc = cuda(q, k, v, do)
    out, lse = fa.forward_fp16_with_lse(qc, kc, vc, True)
    dq, dk, dv = fa.backward(dc, qc, kc, vc, out, lse, True)
    oc, lc = out.cpu(), lse.cpu()
    for b, h in ((0, 0), (2, 7), (3, 15)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        ref = A.backward(do[sl], q[sl], k[sl], v[sl], oc[sl], lc[sl], True)
        _check_grads((dq.cpu()[sl], dk.cpu()[sl], dv.cpu()[sl]), ref, True, f"bench shape b={b} h={h}")


def test_forward_fp32_bench_shape_sampled(fa):
    """Config 7b's forward (fp32, B=4 H=16 N=2048 D=128 causal) on sampled slices."""
    g = gen(71)
    B, H, N, D = 4, 16, 2048, 128
    q, k, v = (randn(g, B, H, N, D, dtype=torch.float32) for _ in range(3))
    out, lse = fa.forward_with_lse(*cuda(q, k, v), True)
    for b, h in ((1, 3), (3, 12)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        ro, rl = A.prefill_lse(q[sl], k[sl], v[sl], True, compute_dtype=F64)
        assert_close(out.cpu()[sl], ro, atol=2e-4, rtol=2e-4, what="fp32 forward bench shape")
        assert_close(lse.cpu()[sl], rl, atol=2e-4, rtol=2e-4, what="fp32 lse bench shape")


@pytest.mark.parametrize("dtype,d", [(torch.float16, 128), (torch.float16, 64), (torch.float32, 128),
                                     (torch.float32, 32)])
def test_backward_concurrent_streams_and_graph_capture(fa, dtype, d):
    """The backward's kernels run on side streams forked from the caller's
    stream (delta kernel, dQ, dK/dV passes).  Results equal the in-order run
    under graph capture (where the launches stay on the captured stream) bit
    for bit on every replay, and a backward on a non-default stream is
    ordered with that stream's later work."""
    g = gen(72 + d)
    q, k, v, do = (randn(g, 2, 8, 300, d, dtype=dtype) for _ in range(4))
    qc, kc, vc, dc = cuda(q, k, v, do)
    fwd = fa.forward_fp16_with_lse if dtype == torch.float16 else fa.forward_with_lse
    out, lse = fwd(qc, kc, vc, True)
    eager = fa.backward(dc, qc, kc, vc, out, lse, True)
    ref = A.backward(do, q, k, v, out.cpu(), lse.cpu(), True)
    _check_grads(eager, ref, dtype == torch.float16, "concurrent backward")

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        on_s = fa.backward(dc, qc, kc, vc, out, lse, True)
        sums = [t.float().sum() for t in on_s]  # consumes the results on the same stream
    torch.cuda.current_stream().wait_stream(s)
    for x, y, t in zip(on_s, eager, sums):
        assert torch.equal(x, y)
        assert t.item() == y.float().sum().item()

    graph = torch.cuda.CUDAGraph()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fa.backward(dc, qc, kc, vc, out, lse, True)  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(graph):
        captured = fa.backward(dc, qc, kc, vc, out, lse, True)
    for _ in range(3):
        for t in captured:
            t.zero_()
        fa.backward(dc, qc, kc, vc, out, lse, True)  # eager work between the replays
        graph.replay()
        torch.cuda.synchronize()
        for x, y in zip(captured, eager):
            assert torch.equal(x, y)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_backward_on_several_caller_streams(fa, dtype):
    """Backward calls issued on different caller streams at once (each with its
    own pair of side streams for the concurrent passes) give exactly the
    results of the same calls run one after another on the default stream."""
    b, h, n, d = 1, 4, 384, 128
    g = gen(4040)
    cases = []
    for i in range(4):
        q, k, v, do = (randn(g, b, h, n, d, dtype=dtype).cuda() for _ in range(4))
        fwd = fa.forward_fp16_with_lse if dtype == torch.float16 else fa.forward_with_lse
        out, lse = fwd(q, k, v, True)
        cases.append((do, q, k, v, out, lse))
    torch.cuda.synchronize()
    ref = [fa.backward(*c, True) for c in cases]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in cases]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    got = []
    for s, c in zip(streams, cases):
        with torch.cuda.stream(s):
            got.append(fa.backward(*c, True))
    torch.cuda.synchronize()
    for r, x in zip(ref, got):
        for a, e in zip(x, r):
            assert torch.equal(a, e)
