"""GPU parity of the tensor-parallel helpers (scatter_heads, gather_heads,
cross_gpu_allreduce_fp16) against the CPU oracle: bit-exact (pure copies and
one correctly rounded fp16 add per element), on the reference test's case,
partial and empty head ranges, shapes that take the 2-byte path, and the
validation errors of the reference wrappers."""
import pytest
import torch

from oracle import attention as A

pytestmark = pytest.mark.gpu


def test_scatter_gather_reference_case(fa):
    """test_multi_gpu.py:44-70, seed 42, B=2 H=16 N=128 D=64, counts 4 and 8."""
    torch.manual_seed(42)
    B, H, N, D = 2, 16, 128, 64
    full = torch.randn(B, H, N, D).half()
    for c in (4, 8):
        loc = torch.zeros(B, c, N, D, dtype=torch.float16, device="cuda")
        fa.scatter_heads(full.cuda(), loc, H, 0, c)
        assert torch.equal(loc.cpu(), A.scatter_heads(full, torch.zeros(B, c, N, D).half(), H, 0, c))
        rec = torch.zeros(B, H, N, D, dtype=torch.float16, device="cuda")
        fa.gather_heads(rec, loc, H, 0, c)
        assert torch.equal(rec.cpu(), A.gather_heads(torch.zeros_like(full), loc.cpu(), H, 0, c))


@pytest.mark.parametrize("B,H,start,count,N,D", [
    (2, 16, 5, 3, 128, 64), (1, 32, 31, 1, 1, 128), (3, 8, 0, 8, 17, 128), (2, 16, 7, 0, 64, 64),
    (2, 8, 2, 4, 9, 7), (4, 6, 1, 3, 33, 36), (1, 64, 16, 16, 4097, 128), (0, 4, 0, 2, 8, 64),
    (70000, 2, 1, 1, 1, 8),
])
def test_scatter_gather_heads(fa, B, H, start, count, N, D):
    g = torch.Generator().manual_seed(B * 1000 + H * 10 + start + count + N + D)
    full = torch.randn(B, H, N, D, generator=g).half()
    local0 = torch.randn(B, count, N, D, generator=g).half()
    loc = local0.cuda()
    fa.scatter_heads(full.cuda(), loc, H, start, count)
    assert torch.equal(loc.cpu(), A.scatter_heads(full, local0, H, start, count))
    base = torch.randn(B, H, N, D, generator=g).half()
    fg = base.cuda()
    fa.gather_heads(fg, local0.cuda(), H, start, count)
    assert torch.equal(fg.cpu(), A.gather_heads(base, local0, H, start, count))


def test_scatter_gather_unaligned_views(fa):
    """Storage offsets that break 16-byte alignment take the 2-byte path."""
    g = torch.Generator().manual_seed(3)
    B, H, N, D = 2, 8, 16, 64
    raw = torch.randn(B * H * N * D + 1, generator=g).half()
    full = raw[1:].view(B, H, N, D)
    rawl = torch.zeros(B * 3 * N * D + 1).half()
    loc = rawl.cuda()[1:].view(B, 3, N, D)
    fa.scatter_heads(raw.cuda()[1:].view(B, H, N, D), loc, H, 2, 3)
    assert torch.equal(loc.cpu(), full[:, 2:5])


@pytest.mark.parametrize("n", [0, 1, 7, 8, 9, 1000, 4096 * 33 + 5, 64 * 1024 * 1024])
def test_allreduce_fp16(fa, n):
    g = torch.Generator().manual_seed(n % 1000 + 1)
    d = (torch.randn(n, generator=g) * 300).half()
    s = (torch.randn(n, generator=g) * 300).half()
    if n >= 8:
        d[:6] = torch.tensor([2048.0, 2050.0, 65504.0, 1.5, float("nan"), float("inf")]).half()
        s[:6] = torch.tensor([1.0, 1.0, 16.0, -1.5, 1.0, 1.0]).half()
    dg = d.cuda()
    fa.cross_gpu_allreduce_fp16(dg, s.cuda())
    ref = A.allreduce_fp16(d, s)
    got = dg.cpu()
    nan = torch.isnan(ref)
    assert torch.equal(torch.isnan(got), nan)
    assert torch.equal(got[~nan].view(torch.int16), ref[~nan].view(torch.int16))


def test_allreduce_fp16_shapes_alias_and_offsets(fa):
    g = torch.Generator().manual_seed(11)
    d = torch.randn(3, 5, 7, generator=g).half()
    dg = d.cuda()
    fa.cross_gpu_allreduce_fp16(dg, dg)  # src == dst doubles
    assert torch.equal(dg.cpu(), A.allreduce_fp16(d, d))
    raw_d = torch.randn(1001, generator=g).half()
    raw_s = torch.randn(1003, generator=g).half()
    dgr = raw_d.cuda()
    fa.cross_gpu_allreduce_fp16(dgr[1:], raw_s.cuda()[3:])  # misaligned views: scalar path
    ref = raw_d.clone()
    ref[1:] = A.allreduce_fp16(raw_d[1:], raw_s[3:])
    assert torch.equal(dgr.cpu(), ref)


def test_tp_validation_errors(fa):
    f = torch.zeros(2, 8, 4, 64, dtype=torch.float16, device="cuda")
    loc = torch.zeros(2, 4, 4, 64, dtype=torch.float16, device="cuda")
    for fn in (fa.scatter_heads, fa.gather_heads):
        with pytest.raises(RuntimeError):
            fn(f, loc, 7, 0, 4)  # total_heads mismatch
        with pytest.raises(RuntimeError):
            fn(f, loc, 8, 0, 3)  # local head count mismatch
        with pytest.raises(RuntimeError):
            fn(f, loc, 8, 5, 4)  # range exceeds total
        with pytest.raises(RuntimeError):
            fn(f, loc, 8, -1, 4)
        with pytest.raises(RuntimeError):
            fn(f.float(), loc, 8, 0, 4)
        with pytest.raises(RuntimeError):
            fn(f, torch.zeros(2, 4, 5, 64, dtype=torch.float16, device="cuda"), 8, 0, 4)
        with pytest.raises(RuntimeError):
            fn(f, loc.cpu(), 8, 0, 4)
        with pytest.raises(RuntimeError):
            fn(f[:, :, :, :32], torch.zeros(2, 4, 4, 32, dtype=torch.float16, device="cuda"), 8, 0, 4)
    with pytest.raises(RuntimeError):
        fa.cross_gpu_allreduce_fp16(f, loc)  # size mismatch
    with pytest.raises(RuntimeError):
        fa.cross_gpu_allreduce_fp16(f, f.float())
    with pytest.raises(RuntimeError):
        fa.cross_gpu_allreduce_fp16(f, f.cpu())
