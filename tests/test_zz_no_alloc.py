"""The allocation-free decode entry point (fa_decode_fp16_noalloc) against
fa_decode_fp16 with a caller workspace, through the C ABI: bit-identical
outputs, each case called twice in a row, cases of decreasing size (the
refusal of an oversized call is a CPU test in test_capi.py)."""
import ctypes
import os

import pytest
import torch

from tests.helpers import randn

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "flash_attn_v100_amd", "libflash_attn_mi355x.so")
FA_OK, FA_ERR_UNSUPPORTED = 0, 3


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    L = ctypes.CDLL(LIB)
    L.fa_last_error.restype = ctypes.c_char_p
    L.fa_decode_workspace_size.restype = ctypes.c_size_t
    L.fa_decode_workspace_size.argtypes = [ctypes.c_int] * 5
    return L


def _p(t):
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _reference(lib, q, k, v, causal, cache_len):
    B, H_Q, _, D = q.shape
    H_KV, N = k.shape[1], k.shape[2]
    o = torch.empty_like(q)
    nbytes = lib.fa_decode_workspace_size(B, H_Q, H_KV, N, D)
    ws = torch.zeros(max(nbytes, 1), dtype=torch.uint8, device="cuda")
    rc = lib.fa_decode_fp16(_p(q), _p(k), _p(v), _p(o), B, H_Q, H_KV, N, D, int(causal), cache_len,
                            _p(ws), ctypes.c_size_t(nbytes), _stream())
    assert rc == FA_OK, lib.fa_last_error()
    return o


def _noalloc(lib, q, k, v, causal, cache_len):
    B, H_Q, _, D = q.shape
    H_KV, N = k.shape[1], k.shape[2]
    o = torch.empty_like(q)
    rc = lib.fa_decode_fp16_noalloc(_p(q), _p(k), _p(v), _p(o), B, H_Q, H_KV, N, D, int(causal), cache_len,
                                    _stream())
    assert rc == FA_OK, lib.fa_last_error()
    return o


def test_noalloc_matches_workspace_entry_point(lib):
    g = torch.Generator().manual_seed(77)
    cases = [(1, 32, 8, 4097, 128, True, 4096),   # config 2: 32 splits per head, early merge
             (1, 32, 8, 1000, 128, False, 999),   # smaller: fewer splits, same static array
             (2, 16, 4, 3000, 64, True, 2500),
             (1, 8, 8, 64, 128, True, 10)]        # one split: no workspace at all
    for B, H_Q, H_KV, N, D, causal, cl in cases:
        print(f"noalloc case B={B} H_Q={H_Q} H_KV={H_KV} N={N} D={D} causal={causal} cache_len={cl}", flush=True)
        q = randn(g, B, H_Q, 1, D).cuda()
        k = randn(g, B, H_KV, N, D).cuda()
        v = randn(g, B, H_KV, N, D).cuda()
        ref = _reference(lib, q, k, v, causal, cl)
        for _ in range(2):
            got = _noalloc(lib, q, k, v, causal, cl)
            torch.cuda.synchronize()
            assert torch.equal(got, ref)


def test_noalloc_replays_from_a_captured_graph(lib):
    """The entry point's callers capture it: a captured config-2 call replays to
    the workspace entry point's result, with eager calls of another shape
    (sharing the same static array, in order) between the replays."""
    g = torch.Generator().manual_seed(78)
    q, k, v = (randn(g, 1, 32, 1, 128).cuda(), randn(g, 1, 8, 4097, 128).cuda(), randn(g, 1, 8, 4097, 128).cuda())
    q2, k2, v2 = (randn(g, 2, 16, 1, 64).cuda(), randn(g, 2, 4, 3000, 64).cuda(), randn(g, 2, 4, 3000, 64).cuda())
    ref = _reference(lib, q, k, v, True, 4096)
    ref2 = _reference(lib, q2, k2, v2, True, 2999)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    out = torch.empty_like(q)
    with torch.cuda.stream(st):
        _noalloc(lib, q, k, v, True, 4096)  # set-up outside the capture
    st.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        rc = lib.fa_decode_fp16_noalloc(_p(q), _p(k), _p(v), _p(out), 1, 32, 8, 4097, 128, 1, 4096,
                                        ctypes.c_void_p(st.cuda_stream))
    assert rc == FA_OK, lib.fa_last_error()
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        assert torch.equal(_noalloc(lib, q2, k2, v2, True, 2999), ref2)
        torch.cuda.synchronize()
