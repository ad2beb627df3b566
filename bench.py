"""Benchmark of the MI355X attention hot path on the BASELINE configs.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs 1,2,3,4,5a,5b,6a,6b,7,7b,8,9] [--no-cpu]

Prints ONE JSON line.  The headline ``value`` is BASELINE configs[1]: GQA decode
via forward_decode_gqa_fp16, Q [1,32,1,128], K/V [1,8,4097,128] fp16,
cache_len 4096, causal -- reported as algorithmic HBM GB/s (K and V rows the
attention must read, plus Q and O), with inputs resident in HBM.  Its 16.8 MB
working set fits in the 256 MB Infinity Cache, so every step uses the next of
40 distinct K/V buffer sets (672 MB) and the timed loop cannot be served from
cache.  A "step" is one call of the hot path over one batch.

The line also carries, per config, the GPU time, throughput, roofline fraction
and tokens/s (decode) or TFLOP/s (prefill), the ``roofline`` object for the
headline kernel (timed with HIP events on the stream the kernel runs on), and
``cpu_baseline``: the CPU oracle (PyTorch eager fp32 math attention with the
reference's masking, oracle/attention.py) timed on this host on a bounded
sample of the same workload.  Configs 6a/6b (INT8 KV-cache and sliding-window
decode) measure the next-row entry points at bandwidth-relevant shapes, and
configs 7/7b the attention backward (fp16 / fp32) at a training shape, and
config 8 KV-cache token eviction, config 9 speculative verification; they
are not BASELINE configs.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
MFMA_FP16_PEAK_TFS = 2500.0  # MI355X dense fp16 MFMA
MFMA_FP32_PEAK_TFS = 157.3   # MI355X dense fp32 MFMA
HEADLINE_KERNEL = "decode_splitkv_kernel<128, 4, 0, true, false>"


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--configs", default="1,2,3,4,5a,5b,6a,6b,7,7b,8,9")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only-headline", action="store_true", help="time config 2 only (for profilers)")
    ap.add_argument("--ceilings", action="store_true",
                    help="measure the streaming-read and MFMA-chain ceilings (libfa_ceilings.so; the default)")
    ap.add_argument("--no-ceilings", action="store_true", help="skip the ceilings (about a second of GPU time)")
    ap.add_argument("--record-traffic", nargs=2, type=float, metavar=("FETCH_KIB", "WRITE_KIB"),
                    help="write profiles/traffic.json for the headline kernel from the FETCH_SIZE and "
                         "WRITE_SIZE per-dispatch means (KiB) of two rocprofv3 --pmc passes, stamped "
                         "with the hash of the sources that build it, and exit")
    return ap.parse_args()


# Sources the headline kernel is built from: roofline.traffic is reported only
# while profiles/traffic.json carries the hash of these files as they are now.
TRAFFIC_SOURCES = ("flash_attn_v100_amd/csrc/decode.hip", "flash_attn_v100_amd/csrc/common.h",
                   "flash_attn_v100_amd/csrc/capi_internal.h")
FETCH_SCALE, WRITE_SCALE = 2.0, 1.0  # counter calibration against a 1 GiB copy


def traffic_source_hash():
    import hashlib

    h = hashlib.sha256()
    for rel in TRAFFIC_SOURCES:
        with open(os.path.join(REPO, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def record_traffic(fetch_kib, write_kib):
    entry = {"workload": "config 2", "fetch_kib_per_dispatch": fetch_kib, "write_kib_per_dispatch": write_kib,
             "fetch_scale": FETCH_SCALE, "write_scale": WRITE_SCALE,
             "hbm_bytes_per_launch": round((fetch_kib * FETCH_SCALE + write_kib * WRITE_SCALE) * 1024),
             "source_sha256": traffic_source_hash(), "sources": list(TRAFFIC_SOURCES)}
    with open(os.path.join(REPO, "profiles", "traffic.json"), "w") as f:
        json.dump({HEADLINE_KERNEL: entry}, f, indent=2)
        f.write("\n")
    print(json.dumps(entry))


def load_traffic():
    """(bytes per launch, stale flag) for the headline kernel; bytes is None when
    the file is missing or was measured on other sources than the ones built now."""
    tpath = os.path.join(REPO, "profiles", "traffic.json")
    if not os.path.exists(tpath):
        return None, True
    with open(tpath) as f:
        entry = json.load(f).get(HEADLINE_KERNEL, {})
    if entry.get("source_sha256") != traffic_source_hash():
        return None, True
    return entry.get("hbm_bytes_per_launch"), False


def time_gpu(fn, steps, warmup):
    """Average ms per call of fn(i), timed with HIP events on the current stream."""
    import torch

    # Untimed warmup: at least `warmup` calls and at least ~0.2 s of GPU work, so
    # the timed calls run at steady clocks (a cold GPU runs the first few
    # hundred microseconds of work measurably slower).
    t_end = time.perf_counter() + 0.2
    i = 0
    while i < warmup or time.perf_counter() < t_end:
        fn(i)
        i += 1
        if i % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    warmup = i
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for i in range(steps):
        fn(warmup + i)
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def time_cpu(fn, budget_s, min_reps=1):
    """Median seconds per call of fn(), repeating until ~budget_s is spent."""
    times = []
    t_start = time.perf_counter()
    while len(times) < min_reps or (time.perf_counter() - t_start) < budget_s:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if len(times) >= 50:
            break
    times.sort()
    return times[len(times) // 2], len(times)


# ----------------------------------------------------------------------------- configs

def cfg1_prefill(fa, torch, steps, warmup):
    B, H, N, D = 2, 8, 256, 64
    g = torch.Generator().manual_seed(0)
    q, k, v = [torch.randn(B, H, N, D, generator=g).half() for _ in range(3)]
    qc, kc, vc = q.cuda(), k.cuda(), v.cuda()
    ms = time_gpu(lambda i: fa.forward_fp16(qc, kc, vc, True), steps, warmup)
    flops = 4.0 * B * H * D * N * (N + 1) / 2
    tfs = flops / (ms * 1e-3) / 1e12
    return dict(workload="forward_fp16 causal B=2 H=8 N=256 D=64", ms=ms, tflops=tfs,
                roofline_frac=tfs / MFMA_FP16_PEAK_TFS, flops=flops,
                ref_flops_2BHN2D=2.0 * B * H * N * N * D), (q, k, v)


def cfg2_decode(fa, torch, steps, warmup, nsets=40):
    B, HQ, HKV, N, D, CL = 1, 32, 8, 4097, 128, 4096
    g = torch.Generator(device="cuda").manual_seed(0)
    qs = [torch.randn(B, HQ, 1, D, generator=g, device="cuda").half() for _ in range(nsets)]
    ks = [torch.randn(B, HKV, N, D, generator=g, device="cuda").half() for _ in range(nsets)]
    vs = [torch.randn(B, HKV, N, D, generator=g, device="cuda").half() for _ in range(nsets)]

    def step(i):
        j = i % nsets
        fa.forward_decode_gqa_fp16(qs[j], ks[j], vs[j], True, CL)

    ms = time_gpu(step, steps, warmup)
    kv_bytes = 2.0 * B * HKV * (CL + 1) * D * 2
    total = kv_bytes + 2.0 * B * HQ * D * 2
    gbs = total / (ms * 1e-3) / 1e9
    graph_us = graph_replay_us(fa, torch, qs, ks, vs, CL)
    return dict(workload="forward_decode_gqa_fp16 B=1 Hq=32 Hkv=8 N=4097 D=128 cache_len=4096 causal",
                ms=ms, gbs=gbs, roofline_frac=gbs / HBM_PEAK_GBS, bytes=total, tokens_per_s=B / (ms * 1e-3),
                rotating_sets=nsets, graph_replay_us_per_call=graph_us,
                graph_replay_gbs=total / (graph_us * 1e-6) / 1e9), (qs[0].cpu(), ks[0].cpu(), vs[0].cpu(), CL)


def graph_replay_us(fa, torch, qs, ks, vs, cl, calls=200, reps=5):
    """Config 2 captured as one HIP graph of `calls` back-to-back decode calls over the
    rotating buffer sets and replayed: the per-call time without host launch overhead.
    Every replay's last output is checked against the eager call on the same inputs."""
    n = len(qs)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):  # the capture stream's split-KV workspace exists before capture
        for i in range(3):
            fa.forward_decode_gqa_fp16(qs[i % n], ks[i % n], vs[i % n], True, cl)
    st.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        for i in range(calls):
            last = fa.forward_decode_gqa_fp16(qs[i % n], ks[i % n], vs[i % n], True, cl)
    j = (calls - 1) % n
    for _ in range(3):
        ref = fa.forward_decode_gqa_fp16(qs[j], ks[j], vs[j], True, cl)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        if not torch.equal(last, ref):
            raise RuntimeError("graph replay differs from the eager decode")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * calls)


def cfg3_cb(fa, torch, steps, warmup):
    B, HQ, HKV, MAXN, D = 64, 32, 8, 8193, 128
    g = torch.Generator().manual_seed(3)
    cl = torch.randint(16, 8193, (B,), generator=g, dtype=torch.int32)
    gg = torch.Generator(device="cuda").manual_seed(3)
    q = torch.randn(B, HQ, 1, D, generator=gg, device="cuda").half()
    k = torch.randn(B, HKV, MAXN, D, generator=gg, device="cuda").half()
    v = torch.randn(B, HKV, MAXN, D, generator=gg, device="cuda").half()
    clc = cl.cuda()
    ms = time_gpu(lambda i: fa.forward_continuous_batching_fp16(q, k, v, clc, True), steps, warmup)
    rows = torch.clamp(cl.long() + 1, max=MAXN).sum().item()
    total = rows * HKV * D * 2 * 2 + 2.0 * B * HQ * D * 2 + 4 * B
    gbs = total / (ms * 1e-3) / 1e9
    return dict(workload="forward_continuous_batching_fp16 B=64 Hq=32 Hkv=8 max_N=8193 D=128 cache_lens~U[16,8192]",
                ms=ms, gbs=gbs, roofline_frac=gbs / HBM_PEAK_GBS, bytes=total,
                tokens_per_s=B / (ms * 1e-3)), (q, k, v, cl)


def cfg4_paged(fa, torch, steps, warmup):
    B, HQ, HKV, D, P, MNB = 128, 32, 8, 128, 65536, 256
    g = torch.Generator().manual_seed(4)
    sl = torch.randint(64, 4097, (B,), generator=g, dtype=torch.int32)
    bt = torch.randperm(P, generator=g)[: B * MNB].view(B, MNB).int()
    gg = torch.Generator(device="cuda").manual_seed(4)
    q = torch.randn(B, HQ, 1, D, generator=gg, device="cuda").half()
    kc = torch.randn(P, HKV, 16, D, generator=gg, device="cuda").half()
    vc = torch.randn(P, HKV, 16, D, generator=gg, device="cuda").half()
    btc, slc = bt.cuda(), sl.cuda()
    ms = time_gpu(lambda i: fa.forward_paged_decode_gqa_fp16(q, kc, vc, btc, slc, MNB), steps, warmup)
    tok = sl.long().sum().item()
    pages = ((sl.long() + 15) // 16).sum().item()
    total = tok * HKV * D * 2 * 2 + pages * 4 + 2.0 * B * HQ * D * 2 + 4 * B
    gbs = total / (ms * 1e-3) / 1e9
    return dict(workload="forward_paged_decode_gqa_fp16 B=128 Hq=32 Hkv=8 D=128 pages=65536x16 seq_lens~U[64,4096]",
                ms=ms, gbs=gbs, roofline_frac=gbs / HBM_PEAK_GBS, bytes=total,
                tokens_per_s=B / (ms * 1e-3)), (q, kc, vc, bt, sl, MNB)


def cfg5a_varlen(fa, torch, steps, warmup):
    H, D = 32, 128
    g = torch.Generator().manual_seed(5)
    lens = torch.randint(128, 2049, (16,), generator=g).tolist()
    cu = torch.tensor([0] + torch.cumsum(torch.tensor(lens), 0).tolist(), dtype=torch.int32)
    tot = int(cu[-1])
    gg = torch.Generator(device="cuda").manual_seed(5)
    q, k, v = [torch.randn(tot, H, D, generator=gg, device="cuda").half() for _ in range(3)]
    cuc = cu.cuda()
    ms = time_gpu(lambda i: fa.forward_varlen_prefill_fp16(q, k, v, cuc, max(lens), True), steps, warmup)
    flops = sum(4.0 * H * D * L * (L + 1) / 2 for L in lens)
    tfs = flops / (ms * 1e-3) / 1e12
    return dict(workload="forward_varlen_prefill_fp16 16 seqs L~U[128,2048] H=32 D=128 causal",
                ms=ms, tflops=tfs, roofline_frac=tfs / MFMA_FP16_PEAK_TFS, flops=flops, total_tokens=tot,
                tokens_per_s=tot / (ms * 1e-3)), (q, k, v, cu, lens)


def cfg5b_int8(fa, torch, steps, warmup, nsets=5):
    B, HQ, HKV, N, D, CL = 16, 32, 8, 2049, 128, 2048
    gg = torch.Generator(device="cuda").manual_seed(55)
    sets = []
    for _ in range(nsets):
        q = torch.randn(B, HQ, 1, D, generator=gg, device="cuda").half()
        k = torch.randn(B, HKV, N, D, generator=gg, device="cuda").half()
        v = torch.randn(B, HKV, N, D, generator=gg, device="cuda").half()
        qs = (q.float().abs().amax(-1).squeeze(-1) / 127).contiguous()
        ks = (k.float().abs().amax((-1, -2)) / 127).unsqueeze(-1).expand(B, HKV, N).contiguous()
        sets.append((q, k, v, qs, ks))

    def step(i):
        q, k, v, qs, ks = sets[i % nsets]
        fa.forward_decode_int8_gqa(q, k, v, qs, ks, CL)

    ms = time_gpu(step, steps, warmup)
    total = 2.0 * B * HKV * (CL + 1) * D * 2 + 2.0 * B * HQ * D * 2 + 4.0 * B * HQ + 4.0 * B * HKV
    gbs = total / (ms * 1e-3) / 1e9
    return dict(workload="forward_decode_int8_gqa B=16 Hq=32 Hkv=8 N=2049 D=128 cache_len=2048",
                ms=ms, gbs=gbs, roofline_frac=gbs / HBM_PEAK_GBS, bytes=total, tokens_per_s=B / (ms * 1e-3),
                rotating_sets=nsets), sets[0]


def cfg6a_int8_kv_cache(fa, torch, steps, warmup, nsets=4):
    """forward_decode_int8_kv_cache_gqa on config 5b's shape with an int8 cache (per-token
    absmax/127 fp16 scales): half the K/V bytes of the fp16 cache."""
    B, HQ, HKV, N, D, CL = 16, 32, 8, 2049, 128, 2048
    gg = torch.Generator(device="cuda").manual_seed(61)
    sets = []
    for _ in range(nsets):
        q = torch.randn(B, HQ, 1, D, generator=gg, device="cuda").half()
        kv = []
        for _ in range(2):
            x = torch.randn(B, HKV, N, D, generator=gg, device="cuda")
            sc = (x.abs().amax(-1, keepdim=True) / 127.0).clamp(min=1e-8)
            kv += [(x / sc).round().clamp(-128, 127).to(torch.int8).contiguous(), sc.squeeze(-1).half().contiguous()]
        sets.append((q, kv[0], kv[2], kv[1], kv[3]))

    def step(i):
        q, k8, v8, ks, vs = sets[i % nsets]
        fa.forward_decode_int8_kv_cache_gqa(q, k8, v8, ks, vs, CL)

    ms = time_gpu(step, steps, warmup)
    total = 2.0 * B * HKV * (CL + 1) * (D + 2) + 2.0 * B * HQ * D * 2
    gbs = total / (ms * 1e-3) / 1e9
    return dict(workload="forward_decode_int8_kv_cache_gqa B=16 Hq=32 Hkv=8 N=2049 D=128 cache_len=2048 int8 K/V + fp16 per-token scales",
                ms=ms, gbs=gbs, roofline_frac=gbs / HBM_PEAK_GBS, bytes=total, tokens_per_s=B / (ms * 1e-3),
                rotating_sets=nsets), sets[0]


def cfg6b_sliding_window(fa, torch, steps, warmup, nsets=3):
    """forward_decode_sliding_window_gqa: B=16, 32:8 heads, N=8193, D=128, cache_len=8192,
    window 2048 + 64 sink tokens (only those keys are read)."""
    B, HQ, HKV, N, D, CL, W, S = 16, 32, 8, 8193, 128, 8192, 2048, 64
    gg = torch.Generator(device="cuda").manual_seed(62)
    sets = [tuple(torch.randn(*shape, generator=gg, device="cuda").half()
                  for shape in ((B, HQ, 1, D), (B, HKV, N, D), (B, HKV, N, D))) for _ in range(nsets)]

    def step(i):
        q, k, v = sets[i % nsets]
        fa.forward_decode_sliding_window_gqa(q, k, v, True, CL, W, S)

    ms = time_gpu(step, steps, warmup)
    total = 2.0 * B * HKV * (W + S) * D * 2 + 2.0 * B * HQ * D * 2
    gbs = total / (ms * 1e-3) / 1e9
    return dict(workload="forward_decode_sliding_window_gqa B=16 Hq=32 Hkv=8 N=8193 D=128 cache_len=8192 window=2048 sink=64",
                ms=ms, gbs=gbs, roofline_frac=gbs / HBM_PEAK_GBS, bytes=total, tokens_per_s=B / (ms * 1e-3),
                rotating_sets=nsets), (sets[0], CL, W, S)


def cfg7_backward(fa, torch, steps, warmup, dtype="fp16"):
    """Attention backward (dq, dk, dv) of causal MHA, B=4 H=16 N=2048 D=128, given the
    forward's out and log-sum-exp.  Algorithmic FLOPs: the five N x N x D products of
    the backward (S, dP, dV, dK, dQ) over the causal triangle, 2.5x the forward's."""
    B, H, N, D = 4, 16, 2048, 128
    dt = torch.float16 if dtype == "fp16" else torch.float32
    gg = torch.Generator(device="cuda").manual_seed(70)
    q, k, v, do = [torch.randn(B, H, N, D, generator=gg, device="cuda").to(dt) for _ in range(4)]
    fwd = fa.forward_fp16_with_lse if dtype == "fp16" else fa.forward_with_lse
    out, lse = fwd(q, k, v, True)
    ms = time_gpu(lambda i: fa.backward(do, q, k, v, out, lse, True), steps, warmup)
    fwd_ms = time_gpu(lambda i: fwd(q, k, v, True), steps, warmup)
    fwd_flops = 4.0 * B * H * D * N * (N + 1) / 2
    flops = 2.5 * fwd_flops
    tfs = flops / (ms * 1e-3) / 1e12
    peak = MFMA_FP16_PEAK_TFS if dtype == "fp16" else MFMA_FP32_PEAK_TFS
    return dict(workload=f"backward {dtype} causal B=4 H=16 N=2048 D=128 (dq, dk, dv from out + lse)",
                ms=ms, tflops=tfs, roofline_frac=tfs / peak, peak_tflops=peak, flops=flops,
                tokens_per_s=B * N / (ms * 1e-3),
                forward_with_lse_ms=fwd_ms, forward_with_lse_tflops=fwd_flops / (fwd_ms * 1e-3) / 1e12), \
        tuple(t[:1, :1].cpu() for t in (do, q, k, v, out, lse))


def cfg8_token_eviction(fa, torch, steps, warmup, nsets=3):
    """token_eviction: B=16, 8 KV heads, N=1024 (the reference's limit), D=128,
    evicting 256 tokens per row.  Algorithmic bytes: kept K/V rows read once,
    every K/V output row written once, scores read, mask written."""
    B, H, N, D, E = 16, 8, 1024, 128, 256
    gg = torch.Generator(device="cuda").manual_seed(80)
    sets = [(torch.randn(B, H, N, D, generator=gg, device="cuda").half(),
             torch.randn(B, H, N, D, generator=gg, device="cuda").half(),
             torch.randn(B, N, generator=gg, device="cuda")) for _ in range(nsets)]

    def step(i):
        k, v, sc = sets[i % nsets]
        fa.token_eviction(k, v, sc, E)

    ms = time_gpu(step, steps, warmup)
    total = 2.0 * B * H * (N - E) * D * 2 + 2.0 * B * H * N * D * 2 + 4.0 * B * N * 2
    gbs = total / (ms * 1e-3) / 1e9
    return dict(workload="token_eviction B=16 H_KV=8 N=1024 D=128 num_evict=256",
                ms=ms, gbs=gbs, roofline_frac=gbs / HBM_PEAK_GBS, bytes=total, rotating_sets=nsets,
                tokens_per_s=B * N / (ms * 1e-3)), tuple(t[:2].cpu() for t in sets[0]) + (E,)


def cfg9_speculative_verify(fa, torch, steps, warmup):
    """speculative_verify: B=16 rows, K=4 draft tokens, vocabulary 32000 (the
    reference test's large case).  Independent random target/draft
    distributions, so most rows reject early and run the full residual scans.
    Latency-bound: each sampled index comes from a serial fp32 running sum."""
    B, K, V = 16, 4, 32000
    gg = torch.Generator(device="cuda").manual_seed(90)
    tp = torch.softmax(torch.randn(B, K + 1, V, generator=gg, device="cuda"), -1)
    dp = torch.softmax(torch.randn(B, K, V, generator=gg, device="cuda"), -1)
    tok = torch.randint(0, V, (B, K), generator=gg, device="cuda")
    rv = torch.rand(B, K, generator=gg, device="cuda")
    ms = time_gpu(lambda i: fa.speculative_verify(tp, dp, tok, rv, K), steps, warmup)
    acc, _ = fa.speculative_verify(tp, dp, tok, rv, K)
    return dict(workload="speculative_verify B=16 K=4 vocab=32000", ms=ms, us_per_call=ms * 1e3,
                rows_per_s=B / (ms * 1e-3), mean_accepted=float(acc.float().mean().item()),
                bound="serial fp32 running sums (latency)"), (tp[:2].cpu(), dp[:2].cpu(), tok[:2].cpu(), rv[:2].cpu(), K)


# ----------------------------------------------------------------------------- ceilings

def measure_ceilings(torch):
    """Streaming-read and MFMA-chain ceilings from libfa_ceilings.so (csrc/ceilings.hip):
    the rates the part sustains for the two rooflines, next to the published peaks."""
    import ctypes

    lib = ctypes.CDLL(os.path.join(REPO, "flash_attn_v100_amd", "libfa_ceilings.so"))
    st = torch.cuda.current_stream()
    out = {}

    def timed(fn, calls):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for _ in range(calls):
            fn()
        e1.record(st)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / calls

    nbytes = 4 << 30  # 16x the 256 MB MALL
    src = torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device="cuda")
    for blocks in (2048, 8192):
        sink = torch.empty(blocks * 256 * 16, dtype=torch.uint8, device="cuda")
        sec = timed(lambda: lib.fa_ceiling_stream_read(ctypes.c_void_p(src.data_ptr()), ctypes.c_size_t(nbytes),
                                                       ctypes.c_void_p(sink.data_ptr()), blocks,
                                                       ctypes.c_void_p(st.cuda_stream)), 20)
        out[f"stream_read_{blocks}wg"] = dict(gbs=nbytes / sec / 1e9, frac_of_peak=nbytes / sec / 1e9 / HBM_PEAK_GBS,
                                              bytes=nbytes, us=sec * 1e6)
    del src
    # read + write: torch's device copy of 134 MB (config 8's size class), six rotating buffers
    n = 67 * 1000 * 1000
    srcs = [torch.empty(n, dtype=torch.uint8, device="cuda").fill_(i) for i in range(6)]
    dsts = [torch.empty_like(t) for t in srcs]
    turn = [0]

    def copy():
        j = turn[0] % 6
        turn[0] += 1
        dsts[j].copy_(srcs[j])

    sec = timed(copy, 60)
    out["copy_read_write_134MB"] = dict(gbs=2 * n / sec / 1e9, frac_of_peak=2 * n / sec / 1e9 / HBM_PEAK_GBS,
                                        bytes=2 * n, us=sec * 1e6)
    del srcs, dsts
    iters = 4000
    g = torch.Generator(device="cuda").manual_seed(11)
    for blocks in (256 * 2, 256 * 3):  # 2 or 3 waves per SIMD, each with 4 independent accumulators
        n = blocks * 4 * 16 * 64 * 8
        flops = blocks * 4 * iters * 8 * 32768.0
        for name, ops in (("random_normal", torch.randn(n, generator=g, device="cuda").half()),
                          ("constant", torch.full((n,), 0.5, device="cuda").half())):
            sink = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
            sec = timed(lambda: lib.fa_ceiling_mfma_chain(ctypes.c_void_p(ops.data_ptr()), iters,
                                                          ctypes.c_void_p(sink.data_ptr()), blocks,
                                                          ctypes.c_void_p(st.cuda_stream)), 10)
            out[f"mfma_f16_{name}_{blocks // 256}wps"] = dict(
                tflops=flops / sec / 1e12, frac_of_peak=flops / sec / 1e12 / MFMA_FP16_PEAK_TFS, us=sec * 1e6)
    return out


# ----------------------------------------------------------------------------- CPU baseline

def cpu_baseline_cfg2(torch, sample, budget_s=12.0):
    """Oracle decode on the full config-2 problem (it is small), repeated for ~budget_s."""
    from oracle import attention as A

    q, k, v, cl = sample
    sec, reps = time_cpu(lambda: A.decode(q, k, v, True, cl), budget_s, min_reps=3)
    kv_bytes = 2.0 * k.shape[0] * k.shape[1] * (cl + 1) * k.shape[3] * 2 + 2.0 * q.numel() * 2
    return dict(value=kv_bytes / sec / 1e9, unit="GB/s", ms=sec * 1e3, reps=reps,
                sample="full config 2 (B=1, 32:8 heads, 4097 keys, D=128), median of %d runs" % reps)


def cpu_baseline_sampled(torch, results, samples, budget_s=6.0):
    """Oracle on bounded samples of the other configs (a few sequences each)."""
    from oracle import attention as A

    out = {}
    if "1" in samples:
        q, k, v = samples["1"]
        sec, n = time_cpu(lambda: A.prefill(q, k, v, True), budget_s, min_reps=3)
        f = results["1"]["flops"]
        out["1"] = dict(ms=sec * 1e3, tflops=f / sec / 1e12, sample="full config 1")
    if "3" in samples:
        q, k, v, cl = samples["3"]
        idx = list(range(4))
        qs, ks, vs = q[idx].cpu(), k[idx].cpu(), v[idx].cpu()
        sec, n = time_cpu(lambda: A.continuous_batching(qs, ks, vs, cl[idx], True), budget_s)
        rows = torch.clamp(cl[idx].long() + 1, max=k.shape[2]).sum().item()
        by = rows * k.shape[1] * k.shape[3] * 4
        out["3"] = dict(ms=sec * 1e3, gbs=by / sec / 1e9, tokens_per_s=len(idx) / sec,
                        sample="4 of 64 sequences")
    if "4" in samples:
        q, kc, vc, bt, sl, mnb = samples["4"]
        idx = list(range(4))
        pages = torch.unique(bt[idx].reshape(-1)).long()
        # gather only the pages the 4 sequences use, remapping the table
        remap = torch.full((kc.shape[0],), -1, dtype=torch.int32)
        remap[pages] = torch.arange(pages.numel(), dtype=torch.int32)
        kcs, vcs = kc[pages.cuda()].cpu(), vc[pages.cuda()].cpu()
        bts = remap[bt[idx].long()]
        qs = q[idx].cpu()
        sec, n = time_cpu(lambda: A.paged_decode(qs, kcs, vcs, bts, sl[idx], mnb), budget_s)
        by = sl[idx].long().sum().item() * kc.shape[1] * kc.shape[3] * 4
        out["4"] = dict(ms=sec * 1e3, gbs=by / sec / 1e9, tokens_per_s=len(idx) / sec,
                        sample="4 of 128 sequences")
    if "5a" in samples:
        q, k, v, cu, lens = samples["5a"]
        s, n_ = int(cu[0]), lens[0]
        qs, ks, vs = q[s:s + n_, :4].cpu(), k[s:s + n_, :4].cpu(), v[s:s + n_, :4].cpu()
        cu1 = torch.tensor([0, n_], dtype=torch.int32)
        sec, _ = time_cpu(lambda: A.varlen_prefill(qs, ks, vs, cu1, n_, True), budget_s)
        f = 4.0 * 4 * 128 * n_ * (n_ + 1) / 2
        out["5a"] = dict(ms=sec * 1e3, tflops=f / sec / 1e12, sample=f"1 sequence (L={n_}), 4 of 32 heads")
    if "5b" in samples:
        q, k, v, qs_, ks_ = samples["5b"]
        idx = [0, 1]
        args = [t[idx].cpu() for t in (q, k, v, qs_, ks_)]
        cl = k.shape[2] - 1
        sec, _ = time_cpu(lambda: A.decode_int8(*args, cl), budget_s)
        by = 2.0 * len(idx) * k.shape[1] * (cl + 1) * k.shape[3] * 2
        out["5b"] = dict(ms=sec * 1e3, gbs=by / sec / 1e9, tokens_per_s=len(idx) / sec,
                         sample="2 of 16 sequences")
    if "6a" in samples:
        q, k8, v8, ks, vs = samples["6a"]
        idx = [0, 1]
        args = [t[idx].cpu() for t in (q, k8, v8, ks, vs)]
        cl = k8.shape[2] - 1
        sec, _ = time_cpu(lambda: A.decode_int8_kv_cache(*args, cl), budget_s)
        by = 2.0 * len(idx) * k8.shape[1] * (cl + 1) * (k8.shape[3] + 2)
        out["6a"] = dict(ms=sec * 1e3, gbs=by / sec / 1e9, tokens_per_s=len(idx) / sec,
                         sample="2 of 16 sequences")
    if "6b" in samples:
        (q, k, v), cl, w, sk = samples["6b"]
        idx = [0, 1]
        qs, ks, vs = q[idx].cpu(), k[idx].cpu(), v[idx].cpu()
        sec, _ = time_cpu(lambda: A.decode_sliding_window(qs, ks, vs, cl, w, sk), budget_s)
        by = 2.0 * len(idx) * k.shape[1] * (w + sk) * k.shape[3] * 2
        out["6b"] = dict(ms=sec * 1e3, gbs=by / sec / 1e9, tokens_per_s=len(idx) / sec,
                         sample="2 of 16 sequences (the whole cache is read on the CPU)")
    if "8" in samples:
        k, v, sc, e = samples["8"]
        sec, _ = time_cpu(lambda: A.token_eviction(k, v, sc, e), budget_s)
        by = 2.0 * k.shape[0] * k.shape[1] * (k.shape[2] - e) * k.shape[3] * 2 + 2.0 * k.numel() * 2
        out["8"] = dict(ms=sec * 1e3, gbs=by / sec / 1e9, tokens_per_s=k.shape[0] * k.shape[2] / sec,
                        sample="2 of 16 batch rows")
    if "9" in samples:
        tp, dp, tok, rv, kk = samples["9"]
        sec, _ = time_cpu(lambda: A.speculative_verify(tp, dp, tok, rv, kk), budget_s)
        out["9"] = dict(ms=sec * 1e3, rows_per_s=tp.shape[0] / sec, sample="2 of 16 batch rows (numpy float32)")
    for c in ("7", "7b"):
        if c in samples:
            do, q, k, v, o, lse = samples[c]
            sec, _ = time_cpu(lambda: A.backward(do, q, k, v, o, lse, True, compute_dtype=torch.float32), budget_s)
            n, d = q.shape[2], q.shape[3]
            f = 2.5 * 4.0 * d * n * (n + 1) / 2
            out[c] = dict(ms=sec * 1e3, tflops=f / sec / 1e12, tokens_per_s=n / sec,
                          sample="1 of 64 (batch, head) pairs, N=2048, fp32 eager")
    return out


# ----------------------------------------------------------------------------- main

def main():
    args = parse()
    if args.record_traffic:
        record_traffic(*args.record_traffic)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build runs on one GPU only; sharding over several GPUs is a "
                                   "design, not a measured path", "n_gpus": args.gpus}))
        sys.exit(2)

    import torch

    import flash_attn_v100 as fa

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.backends.cuda.matmul.allow_tf32 = False
    want = [c.strip() for c in args.configs.split(",") if c.strip() and c.strip() != "none"]
    if args.only_headline:
        want = ["2"]
    results, samples = {}, {}
    # Timed calls per config: config 2 takes --steps/--warmup as given; the
    # others scale them by their own base counts (a few hundred microseconds
    # to a few milliseconds per call), and every config reports what it ran.
    base = {"1": (500, 50), "2": (200, 20), "3": (30, 5), "4": (30, 5), "5a": (50, 10), "5b": (100, 10),
            "6a": (100, 10), "6b": (100, 10), "7": (20, 3), "7b": (5, 1), "8": (100, 10), "9": (50, 5)}

    def counts(c):
        # config 2 (the headline step) times exactly --steps calls; every other
        # config times at least 20 calls, whatever --steps asks for
        st, wu = base[c]
        if c == "2":
            return args.steps, args.warmup
        return max(20, round(st * args.steps / 200)), max(1, round(wu * args.warmup / 20))

    runners = {
        "1": lambda st, wu: cfg1_prefill(fa, torch, st, wu),
        "2": lambda st, wu: cfg2_decode(fa, torch, st, wu),
        "3": lambda st, wu: cfg3_cb(fa, torch, st, wu),
        "4": lambda st, wu: cfg4_paged(fa, torch, st, wu),
        "5a": lambda st, wu: cfg5a_varlen(fa, torch, st, wu),
        "5b": lambda st, wu: cfg5b_int8(fa, torch, st, wu),
        "6a": lambda st, wu: cfg6a_int8_kv_cache(fa, torch, st, wu),
        "6b": lambda st, wu: cfg6b_sliding_window(fa, torch, st, wu),
        "7": lambda st, wu: cfg7_backward(fa, torch, st, wu, "fp16"),
        "7b": lambda st, wu: cfg7_backward(fa, torch, st, wu, "fp32"),
        "8": lambda st, wu: cfg8_token_eviction(fa, torch, st, wu),
        "9": lambda st, wu: cfg9_speculative_verify(fa, torch, st, wu),
    }
    for c in ["1", "2", "3", "4", "5a", "5b", "6a", "6b", "7", "7b", "8", "9"]:
        if c not in want:
            continue
        log(f"config {c} ...")
        st, wu = counts(c)
        r, s = runners[c](st, wu)
        r["steps"], r["warmup"] = st, wu
        results[c], samples[c] = r, s
        log(f"config {c}: " + json.dumps({k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}))
        if c in ("3", "4"):
            del s  # keep only what the CPU leg needs
        torch.cuda.empty_cache()

    cpu = None
    cores = torch.get_num_threads()
    if not args.no_cpu and "2" in results:
        log(f"CPU baseline on {cores} threads (os.cpu_count()={os.cpu_count()}) ...")
        cpu2 = cpu_baseline_cfg2(torch, samples["2"])
        cpu_other = cpu_baseline_sampled(torch, results, {k: v for k, v in samples.items() if k != "2"})
        cpu = dict(value=cpu2["value"], unit="GB/s", cores=cores, kind="port", sample=cpu2["sample"],
                   ms=cpu2["ms"], other_configs=cpu_other, os_cpu_count=os.cpu_count())
        for c, r in cpu_other.items():
            results[c]["cpu"] = r

    ceilings = None
    if not args.no_ceilings:
        log("ceilings ...")
        ceilings = measure_ceilings(torch)
        log("ceilings: " + json.dumps(ceilings))
    if "2" not in results:  # partial run (e.g. under a profiler): per-config figures only
        print(json.dumps({"configs": results, "ceilings": ceilings}), flush=True)
        return
    head = results["2"]
    traffic, traffic_stale = load_traffic()  # measured by the rocprofv3 --pmc passes summarised beside it
    line = {
        "metric": "decode GQA attn HBM GB/s (% of peak); prefill fp16 TFLOP/s (% MFMA peak)",
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic N(0,1) fp16, seeded; K/V rotated over 40 buffer sets (672 MB) to defeat the 256 MB MALL",
        "config": {"workload": head["workload"], "baseline_config": "configs[1]", "global_batch": 1,
                   "seq_len": 4097, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(head["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_stale": traffic_stale,
                     "kernel": HEADLINE_KERNEL, "avg_launch_us": round(head["ms"] * 1e3, 3),
                     "frac_of_measured_stream_read": (round(head["gbs"] / ceilings["stream_read_2048wg"]["gbs"], 4)
                                                      if ceilings else None),
                     "timing": "HIP events on the launch stream around %d back-to-back calls" % args.steps},
        "cpu_baseline": cpu,
        "ceilings": ceilings,
        "configs": {c: {k: (round(v, 6) if isinstance(v, float) else v) for k, v in r.items()}
                    for c, r in results.items()},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
