"""GPU parity of token_eviction against the CPU oracle: bit-exact outputs and
mask (pure index and copy work), including ties (stable order), num_evict at
0, N and beyond, N up to the 1024 limit, and D not a multiple of 8."""
import pytest
import torch

from oracle import attention as A
from tests.helpers import randn

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("b,h,n,d,num_evict,ties", [
    (1, 1, 1, 64, 0, False), (1, 1, 1, 64, 1, False), (2, 3, 7, 64, 3, True), (2, 8, 33, 128, 10, True),
    (3, 2, 255, 128, 100, False), (2, 2, 256, 64, 256, False), (2, 4, 1000, 128, 250, True),
    (1, 8, 1024, 128, 512, False), (2, 2, 300, 36, 77, True), (2, 2, 64, 128, -5, False),
    (1, 2, 50, 128, 80, True),
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
