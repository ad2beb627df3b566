"""The C-ABI library: loads, exports every symbol include/*.h declares, and rejects
bad arguments before touching the GPU (CPU tests); plus GPU parity through ctypes."""
import ctypes
import glob
import os
import re

import pytest
import torch

from oracle import attention as A
from tests.helpers import assert_close, randn

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "flash_attn_v100_amd", "libflash_attn_mi355x.so")

FA_OK, FA_ERR_INVALID_ARG, FA_ERR_WORKSPACE, FA_ERR_UNSUPPORTED = 0, 1, 2, 3


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(REPO, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(fa_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


@pytest.fixture(scope="module")
def lib():
    import torch  # noqa: F401  (shares torch's HIP runtime)

    assert os.path.exists(LIB), "C-ABI library not built"
    L = ctypes.CDLL(LIB)
    L.fa_last_error.restype = ctypes.c_char_p
    L.fa_version.restype = ctypes.c_char_p
    L.fa_decode_workspace_size.restype = ctypes.c_size_t
    L.fa_decode_workspace_size.argtypes = [ctypes.c_int] * 5
    return L


def test_header_declares_the_eight_paths():
    syms = declared_symbols()
    for s in ("fa_prefill_fp16", "fa_varlen_prefill_fp16", "fa_decode_fp16", "fa_continuous_batching_fp16",
              "fa_paged_decode_gqa_fp16", "fa_decode_int8_gqa", "fa_decode_workspace_size"):
        assert s in syms


def test_library_exports_every_declared_symbol(lib):
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_version(lib):
    assert b"gfx950" in lib.fa_version()


def test_workspace_size_plan(lib):
    assert lib.fa_decode_workspace_size(1, 32, 8, 4097, 128) > 0          # config 2 splits
    assert lib.fa_decode_workspace_size(1, 8, 4, 65, 64) == 0              # one split, no workspace
    assert lib.fa_decode_workspace_size(0, 8, 4, 65, 64) == 0
    assert lib.fa_decode_workspace_size(1, 6, 4, 65, 64) == 0              # invalid group -> 0


def _vp(x=0):
    return ctypes.c_void_p(x)


def test_noalloc_decode_refuses_calls_beyond_its_static_scratch(lib):
    """fa_decode_fp16_noalloc checks the plan's workspace against its 16 MiB
    static array before touching any pointer or the GPU."""
    null = _vp()
    # B=64, 64:1 heads, 65536 keys, D=256: 8 splits x 4096 query rows of fp32 partials (33.5 MB)
    rc = lib.fa_decode_fp16_noalloc(null, null, null, null, 64, 64, 1, 65536, 256, 1, 65535, null)
    assert rc == FA_ERR_UNSUPPORTED and b"static scratch" in lib.fa_last_error()
    rc = lib.fa_decode_fp16_noalloc(null, null, null, null, 1, 6, 4, 10, 64, 1, 3, null)
    assert rc == FA_ERR_INVALID_ARG


def test_argument_errors_are_reported_without_a_gpu(lib):
    null = _vp()
    # decode: cache_len out of range
    rc = lib.fa_decode_fp16(null, null, null, null, 1, 8, 4, 10, 64, 1, 10, null, ctypes.c_size_t(0), null)
    assert rc == FA_ERR_INVALID_ARG and b"cache_len" in lib.fa_last_error()
    # decode: H_Q not a multiple of H_KV
    rc = lib.fa_decode_fp16(null, null, null, null, 1, 6, 4, 10, 64, 1, 3, null, ctypes.c_size_t(0), null)
    assert rc == FA_ERR_INVALID_ARG
    # decode: D too large
    rc = lib.fa_decode_fp16(null, null, null, null, 1, 8, 4, 10, 512, 1, 3, null, ctypes.c_size_t(0), null)
    assert rc == FA_ERR_UNSUPPORTED
    # decode: missing workspace when splits are needed
    rc = lib.fa_decode_fp16(_vp(16), _vp(16), _vp(16), _vp(16), 1, 32, 8, 4097, 128, 1, 4096, null,
                            ctypes.c_size_t(0), null)
    assert rc == FA_ERR_WORKSPACE
    # prefill: null pointers
    rc = lib.fa_prefill_fp16(null, null, null, null, 1, 2, 2, 16, 64, 1, null)
    assert rc == FA_ERR_INVALID_ARG
    # empty problems are no-ops
    assert lib.fa_prefill_fp16(null, null, null, null, 0, 2, 2, 16, 64, 1, null) == FA_OK
    rc = lib.fa_varlen_prefill_fp16(null, null, null, null, null, 0, 0, 2, 64, 1, 32, 1, null)
    assert rc == FA_OK
    # int8 and paged argument checks
    rc = lib.fa_decode_int8_gqa(null, null, null, null, null, null, 1, 8, 4, 10, 64, -1, null,
                                ctypes.c_size_t(0), null)
    assert rc == FA_ERR_INVALID_ARG
    rc = lib.fa_paged_decode_gqa_fp16(null, null, null, null, null, ctypes.c_int64(0), null, 1, 8, 4, 64, 4, -1,
                                      null, ctypes.c_size_t(0), null)
    assert rc == FA_ERR_INVALID_ARG
    rc = lib.fa_continuous_batching_fp16(null, null, null, null, null, 1, 8, 4, 0, 64, 1, null,
                                         ctypes.c_size_t(0), null)
    assert rc == FA_ERR_INVALID_ARG


# ---------------------------------------------------------------- GPU, through the C ABI

def _p(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.gpu
def test_capi_decode_prefill_on_gpu(lib):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    g = torch.Generator().manual_seed(0)
    # decode with splits: workspace from fa_decode_workspace_size
    q, k, v = randn(g, 1, 32, 1, 128), randn(g, 1, 8, 4097, 128), randn(g, 1, 8, 4097, 128)
    qc, kc, vc = q.cuda(), k.cuda(), v.cuda()
    o = torch.empty_like(qc)
    ws_bytes = lib.fa_decode_workspace_size(1, 32, 8, 4097, 128)
    ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")  # zero-filled before first use
    rc = lib.fa_decode_fp16(_p(qc), _p(kc), _p(vc), _p(o), 1, 32, 8, 4097, 128, 1, 4096, _p(ws),
                            ctypes.c_size_t(ws_bytes), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == FA_OK, lib.fa_last_error()
    torch.cuda.synchronize()
    ref = A.decode(q, k, v, True, 4096)
    assert_close(o, ref, what="capi decode")
    # the call left the workspace's arrival counters at zero: reuse it twice more
    for _ in range(2):
        o2 = torch.empty_like(qc)
        rc = lib.fa_decode_fp16(_p(qc), _p(kc), _p(vc), _p(o2), 1, 32, 8, 4097, 128, 1, 4096, _p(ws),
                                ctypes.c_size_t(ws_bytes), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert rc == FA_OK
        torch.cuda.synchronize()
        assert torch.equal(o2, o)
    counters = ws[:256].cpu()
    assert int(counters.sum()) == 0
    # prefill
    q, k, v = randn(g, 2, 8, 256, 64), randn(g, 2, 8, 256, 64), randn(g, 2, 8, 256, 64)
    qc, kc, vc = q.cuda(), k.cuda(), v.cuda()
    o = torch.empty_like(qc)
    rc = lib.fa_prefill_fp16(_p(qc), _p(kc), _p(vc), _p(o), 2, 8, 8, 256, 64, 1,
                             ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == FA_OK, lib.fa_last_error()
    torch.cuda.synchronize()
    assert_close(o, A.prefill(q, k, v, True), what="capi prefill")


def test_training_argument_errors_without_a_gpu(lib):
    null = _vp()
    lib.fa_backward_workspace_size.restype = ctypes.c_size_t
    lib.fa_backward_workspace_size.argtypes = [ctypes.c_int] * 3
    assert lib.fa_backward_workspace_size(2, 3, 17) == 2 * 3 * 17 * 4
    assert lib.fa_backward_workspace_size(0, 3, 17) == 0
    # D above 128
    rc = lib.fa_prefill_fp32(null, null, null, null, null, 1, 2, 16, 160, 1, null)
    assert rc == FA_ERR_UNSUPPORTED
    rc = lib.fa_backward_fp16(null, null, null, null, null, null, null, null, null, 1, 2, 16, 160, 1, null,
                              ctypes.c_size_t(0), null)
    assert rc == FA_ERR_UNSUPPORTED
    # null pointers / missing workspace
    rc = lib.fa_prefill_fp16_lse(_vp(16), _vp(16), _vp(16), _vp(16), null, 1, 2, 16, 64, 1, null)
    assert rc == FA_ERR_INVALID_ARG
    p = _vp(16)
    rc = lib.fa_backward_fp32(p, p, p, p, p, p, p, p, p, 1, 2, 16, 64, 1, null, ctypes.c_size_t(0), null)
    assert rc == FA_ERR_WORKSPACE
    # empty problems are no-ops
    assert lib.fa_backward_fp16(null, null, null, null, null, null, null, null, null, 0, 2, 16, 64, 1, null,
                                ctypes.c_size_t(0), null) == FA_OK


@pytest.mark.gpu
def test_capi_training_on_gpu(lib):
    """fa_prefill_fp32 (with LSE), fa_prefill_fp16_lse and fa_backward_fp16 through ctypes."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    g = torch.Generator().manual_seed(1)
    B, H, N, D = 1, 2, 100, 64
    q, k, v, do = (randn(g, B, H, N, D) for _ in range(4))
    qc, kc, vc, dc = (t.cuda() for t in (q, k, v, do))
    # fp32 forward + LSE
    q32, k32, v32 = (t.float().contiguous() for t in (qc, kc, vc))
    o32 = torch.empty_like(q32)
    l32 = torch.empty(B, H, N, device="cuda")
    rc = lib.fa_prefill_fp32(_p(q32), _p(k32), _p(v32), _p(o32), _p(l32), B, H, N, D, 1, st)
    assert rc == FA_OK, lib.fa_last_error()
    ro, rl = A.prefill_lse(q.float(), k.float(), v.float(), True, compute_dtype=torch.float64)
    torch.cuda.synchronize()
    assert_close(o32, ro, atol=2e-4, rtol=2e-4, what="capi fp32 forward")
    assert_close(l32, rl, atol=2e-4, rtol=2e-4, what="capi fp32 lse")
    # fp16 forward + LSE, then backward
    o = torch.empty_like(qc)
    lse = torch.empty(B, H, N, device="cuda")
    rc = lib.fa_prefill_fp16_lse(_p(qc), _p(kc), _p(vc), _p(o), _p(lse), B, H, N, D, 1, st)
    assert rc == FA_OK, lib.fa_last_error()
    nbytes = lib.fa_backward_workspace_size(B, H, N)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    dq, dk, dv = (torch.empty_like(qc) for _ in range(3))
    rc = lib.fa_backward_fp16(_p(dc), _p(qc), _p(kc), _p(vc), _p(o), _p(lse), _p(dq), _p(dk), _p(dv),
                              B, H, N, D, 1, _p(ws), ctypes.c_size_t(nbytes), st)
    assert rc == FA_OK, lib.fa_last_error()
    torch.cuda.synchronize()
    ref = A.backward(do, q, k, v, o.cpu(), lse.cpu(), True)
    for name, a, r in zip(("dq", "dk", "dv"), (dq, dk, dv), ref):
        assert_close(a, r, atol=3e-2, rtol=3e-2, what=f"capi backward {name}")
