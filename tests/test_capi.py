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


def test_workspace_size_bounds_every_shorter_key_count(lib):
    """The split count is not monotonic in the key count (the split length rounds
    up to a quantum), while the bindings size the workspace by N and a call may
    attend fewer keys (sliding window, cache_len < N - 1).  The size for N must
    cover every key count up to N."""
    for b, hq, hkv, d in ((16, 32, 8, 128), (16, 32, 8, 64), (16, 32, 8, 256), (1, 32, 8, 128), (64, 32, 8, 128),
                          (128, 32, 8, 128), (4, 64, 2, 128)):
        sizes = [lib.fa_decode_workspace_size(b, hq, hkv, n, d) for n in range(1, 4200, 7)]
        for i in range(1, len(sizes)):
            assert sizes[i] >= max(sizes[:i]), (b, hq, hkv, d, 1 + 7 * i)


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


def _st():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


@pytest.mark.gpu
def test_capi_every_decode_entry_point_shares_one_workspace(lib):
    """Continuous batching, paged, INT8, INT8 KV cache and sliding-window decode
    through ctypes, all on ONE caller-owned workspace (sized for the largest of
    them, zero-filled once), interleaved with the contiguous decode: each
    matches the oracle and the workspace's counters end at zero."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    g = torch.Generator().manual_seed(31)
    B, HQ, HKV, D = 3, 16, 4, 128
    nbytes = max(lib.fa_decode_workspace_size(B, HQ, HKV, n, D) for n in (2000, 4096))
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    wsp, wsn = _p(ws), ctypes.c_size_t(nbytes)
    # continuous batching
    N = 2000
    q, k, v = randn(g, B, HQ, 1, D), randn(g, B, HKV, N, D), randn(g, B, HKV, N, D)
    cl = torch.tensor([1999, 5, 1000], dtype=torch.int32)
    qc, kc, vc, clc = q.cuda(), k.cuda(), v.cuda(), cl.cuda()
    o = torch.empty_like(qc)
    rc = lib.fa_continuous_batching_fp16(_p(qc), _p(kc), _p(vc), _p(o), _p(clc), B, HQ, HKV, N, D, 1, wsp, wsn, _st())
    assert rc == FA_OK, lib.fa_last_error()
    torch.cuda.synchronize()
    assert_close(o, A.continuous_batching(q, k, v, cl, True), what="capi continuous batching")
    # contiguous decode on the same workspace
    o = torch.empty_like(qc)
    rc = lib.fa_decode_fp16(_p(qc), _p(kc), _p(vc), _p(o), B, HQ, HKV, N, D, 1, 1500, wsp, wsn, _st())
    assert rc == FA_OK, lib.fa_last_error()
    torch.cuda.synchronize()
    assert_close(o, A.decode(q, k, v, True, 1500), what="capi decode")
    # paged: 16-token pages, a permuted table, row stride 256
    P, MNB = 300, 256
    kp, vp = randn(g, P, HKV, 16, D), randn(g, P, HKV, 16, D)
    bt = torch.randint(0, P, (B, MNB), generator=g, dtype=torch.int32)
    sl = torch.tensor([4096, 17, 700], dtype=torch.int32)
    kpc, vpc, btc, slc = kp.cuda(), vp.cuda(), bt.cuda(), sl.cuda()
    o = torch.empty_like(qc)
    rc = lib.fa_paged_decode_gqa_fp16(_p(qc), _p(kpc), _p(vpc), _p(o), _p(btc), ctypes.c_int64(bt.numel()), _p(slc),
                                      B, HQ, HKV, D, P, MNB, wsp, wsn, _st())
    assert rc == FA_OK, lib.fa_last_error()
    torch.cuda.synchronize()
    assert_close(o, A.paged_decode(q, kp, vp, bt, sl, MNB), what="capi paged")
    # INT8 decode (per-head absmax/127 scales)
    qs = (q.float().abs().amax(-1).squeeze(-1) / 127).contiguous()
    ks = (k.float().abs().amax((-1, -2)) / 127).unsqueeze(-1).expand(B, HKV, N).contiguous()
    qsc, ksc = qs.cuda(), ks.cuda()
    o = torch.empty_like(qc)
    rc = lib.fa_decode_int8_gqa(_p(qc), _p(kc), _p(vc), _p(o), _p(qsc), _p(ksc), B, HQ, HKV, N, D, 1999,
                                wsp, wsn, _st())
    assert rc == FA_OK, lib.fa_last_error()
    torch.cuda.synchronize()
    ref = A.decode_int8(q, k, v, qs, ks, 1999)
    assert_close(o, ref, what="capi int8")
    # INT8 KV cache (per-token fp16 scales)
    def quant(x):
        s = (x.float().abs().amax(-1, keepdim=True) / 127.0).clamp(min=1e-8)
        return (x.float() / s).round().clamp(-128, 127).to(torch.int8), s.squeeze(-1).half()
    k8, k8s = quant(k)
    v8, v8s = quant(v)
    k8c, v8c, k8sc, v8sc = k8.cuda(), v8.cuda(), k8s.cuda(), v8s.cuda()
    o = torch.empty_like(qc)
    rc = lib.fa_decode_int8_kv_cache_gqa(_p(qc), _p(k8c), _p(v8c), _p(k8sc), _p(v8sc), _p(o), B, HQ, HKV, N, D,
                                         1999, wsp, wsn, _st())
    assert rc == FA_OK, lib.fa_last_error()
    torch.cuda.synchronize()
    assert_close(o, A.decode_int8_kv_cache(q, k8, v8, k8s, v8s, 1999), what="capi int8 kv cache")
    # sliding window + sink
    o = torch.empty_like(qc)
    rc = lib.fa_decode_sliding_window_gqa(_p(qc), _p(kc), _p(vc), _p(o), B, HQ, HKV, N, D, 1800, 512, 16,
                                          wsp, wsn, _st())
    assert rc == FA_OK, lib.fa_last_error()
    torch.cuda.synchronize()
    assert_close(o, A.decode_sliding_window(q, k, v, 1800, 512, 16), what="capi sliding window")
    # the arrival counters are back at zero
    torch.cuda.synchronize()
    assert int(ws[: 65536 * 4].cpu().sum()) == 0


@pytest.mark.gpu
def test_capi_varlen_token_ops_and_tp_helpers(lib):
    """fa_varlen_prefill_fp16, fa_token_eviction, fa_speculative_verify and the
    tensor-parallel copies / accumulate through ctypes."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    g = torch.Generator().manual_seed(32)
    # varlen prefill: 3 sequences, one empty
    lens = [130, 0, 77]
    cu = torch.tensor([0, 130, 130, 207], dtype=torch.int32)
    H, D = 4, 64
    q, k, v = (randn(g, 207, H, D) for _ in range(3))
    qc, kc, vc, cuc = q.cuda(), k.cuda(), v.cuda(), cu.cuda()
    o = torch.empty_like(qc)
    row_limit = A.varlen_row_limit(max(lens), D)
    rc = lib.fa_varlen_prefill_fp16(_p(qc), _p(kc), _p(vc), _p(o), _p(cuc), 3, 207, H, D, max(lens), row_limit, 1,
                                    _st())
    assert rc == FA_OK, lib.fa_last_error()
    torch.cuda.synchronize()
    assert_close(o, A.varlen_prefill(q, k, v, cu, max(lens), True), what="capi varlen")
    # token eviction
    Bt, Ht, Nt, Dt = 2, 3, 100, 64
    kt, vt = randn(g, Bt, Ht, Nt, Dt), randn(g, Bt, Ht, Nt, Dt)
    sc = torch.randn(Bt, Nt, generator=g)
    ktc, vtc, scc = kt.cuda(), vt.cuda(), sc.cuda()
    ko, vo = torch.empty_like(ktc), torch.empty_like(vtc)
    mask = torch.empty(Bt, Nt, dtype=torch.int32, device="cuda")
    rc = lib.fa_token_eviction(_p(ktc), _p(vtc), _p(scc), _p(ko), _p(vo), _p(mask), Bt, Ht, Nt, Dt, 30, _st())
    assert rc == FA_OK, lib.fa_last_error()
    torch.cuda.synchronize()
    rk, rv, rm = A.token_eviction(kt, vt, sc, 30)
    assert torch.equal(mask.cpu(), rm) and torch.equal(ko.cpu(), rk) and torch.equal(vo.cpu(), rv)
    # speculative verify
    Bs, K, V = 3, 4, 1000
    tp = torch.softmax(torch.randn(Bs, K + 1, V, generator=g), -1)
    dp = torch.softmax(torch.randn(Bs, K, V, generator=g), -1)
    tok = torch.randint(0, V, (Bs, K), generator=g)
    rv_ = torch.rand(Bs, K, generator=g)
    tpc, dpc, tokc, rvc = tp.cuda(), dp.cuda(), tok.cuda(), rv_.cuda()
    acc = torch.empty(Bs, dtype=torch.int32, device="cuda")
    out = torch.empty(Bs, K + 1, dtype=torch.int64, device="cuda")
    rc = lib.fa_speculative_verify(_p(tpc), _p(dpc), _p(tokc), _p(rvc), _p(acc), _p(out), Bs, K, V, _st())
    assert rc == FA_OK, lib.fa_last_error()
    torch.cuda.synchronize()
    racc, rout = A.speculative_verify(tp, dp, tok, rv_, K)
    assert torch.equal(acc.cpu(), racc) and torch.equal(out.cpu(), rout)
    # tensor-parallel helpers
    full = randn(g, 2, 8, 33, 64)
    fc = full.cuda()
    loc = torch.empty(2, 3, 33, 64, dtype=torch.float16, device="cuda")
    assert lib.fa_scatter_heads(_p(fc), _p(loc), 2, 8, 4, 3, 33, 64, _st()) == FA_OK
    back = torch.zeros_like(fc)
    assert lib.fa_gather_heads(_p(back), _p(loc), 2, 8, 4, 3, 33, 64, _st()) == FA_OK
    d0 = randn(g, 5000)
    dd, ss = d0.cuda(), randn(g, 5000).cuda()
    s_cpu = ss.cpu()
    assert lib.fa_cross_gpu_allreduce_fp16(_p(dd), _p(ss), ctypes.c_size_t(5000), _st()) == FA_OK
    torch.cuda.synchronize()
    assert torch.equal(loc.cpu(), full[:, 4:7])
    assert torch.equal(back.cpu(), A.gather_heads(torch.zeros_like(full), loc.cpu(), 8, 4, 3))
    assert torch.equal(dd.cpu(), A.allreduce_fp16(d0, s_cpu))
    # argument errors of the TP helpers
    assert lib.fa_scatter_heads(_p(fc), _p(loc), 2, 8, 6, 3, 33, 64, _st()) == FA_ERR_INVALID_ARG
