"""Writes the small golden fixtures in this directory.

Outputs come from oracle/brute.py, the fp64 loop restatement of the reference
kernels (flash_attn_kernel.cu / continuous_batching_kernel.cu), evaluated on
seeded inputs that mirror the reference's own test cases where it has them
(test.py seed 0, test_decode.py paged layout seed 2025, test_continuous_batching.py
cases).  The reference ships no golden vectors, so these fixtures freeze the
independent restatement; tests/test_oracle.py checks the vectorised oracle
against them and the GPU tests check the kernels against the oracle.

Run:  python tests/golden/make_golden.py               (every fixture)
      python tests/golden/make_golden.py --next-rows   (only the LSE forward, backward,
      sliding-window, INT8-KV-cache, token-eviction and speculative-verify fixtures)
"""
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import brute as Bt  # noqa: E402


def rn(g, *s):
    return torch.randn(*s, generator=g).half()


def save(name, kind, args, out):
    torch.save({"kind": kind, "args": args, "out": torch.tensor(out, dtype=torch.float64)},
               os.path.join(HERE, name + ".pt"))
    print("wrote", name)


def save_multi(name, kind, args, outs, dtype=torch.float64):
    torch.save({"kind": kind, "args": args, "outs": [torch.tensor(o, dtype=dtype) for o in outs]},
               os.path.join(HERE, name + ".pt"))
    print("wrote", name)


def main():
    g = torch.Generator().manual_seed(0)
    q, k, v = rn(g, 1, 2, 20, 16), rn(g, 1, 2, 20, 16), rn(g, 1, 2, 20, 16)
    save("prefill_causal_mha", "prefill", dict(q=q, k=k, v=v, causal=True),
         Bt.prefill(q.double(), k.double(), v.double(), True))

    g = torch.Generator().manual_seed(1234)
    q, k, v = rn(g, 1, 4, 12, 8), rn(g, 1, 2, 12, 8), rn(g, 1, 2, 12, 8)
    save("prefill_gqa_full", "prefill", dict(q=q, k=k, v=v, causal=False),
         Bt.prefill(q.double(), k.double(), v.double(), False))

    g = torch.Generator().manual_seed(1234)
    q, k, v = rn(g, 1, 8, 1, 16), rn(g, 1, 4, 65, 16), rn(g, 1, 4, 65, 16)
    save("decode_gqa_causal", "decode", dict(q=q, k=k, v=v, causal=True, cache_len=40),
         Bt.decode(q.double(), k.double(), v.double(), True, 40))

    g = torch.Generator().manual_seed(0)
    q, k, v = rn(g, 3, 8, 1, 16), rn(g, 3, 2, 17, 16), rn(g, 3, 2, 17, 16)
    cl = torch.tensor([0, 3, 15], dtype=torch.int32)
    save("continuous_batching", "continuous_batching", dict(q=q, k=k, v=v, cache_lens=cl, causal=True),
         Bt.continuous_batching(q.double(), k.double(), v.double(), cl, True))

    g = torch.Generator().manual_seed(2025)
    seq_lens = [16, 23, 33]
    order = [5, 2, 7, 1, 9, 3]
    b, hq, hkv, d = 3, 8, 4, 16
    q = rn(g, b, hq, 1, d)
    kk, vv = rn(g, b, hkv, 33, d), rn(g, b, hkv, 33, d)
    kc = torch.zeros(10, hkv, 16, d, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    bt = torch.full((b, 3), -1, dtype=torch.int32)
    cur = 0
    for i, s in enumerate(seq_lens):
        for blk in range((s + 15) // 16):
            p = order[cur]
            cur += 1
            bt[i, blk] = p
            st, en = blk * 16, min(blk * 16 + 16, s)
            kc[p, :, : en - st] = kk[i, :, st:en]
            vc[p, :, : en - st] = vv[i, :, st:en]
    sl = torch.tensor(seq_lens, dtype=torch.int32)
    save("paged_reference_layout", "paged",
         dict(q=q, k_cache=kc, v_cache=vc, block_table=bt, seq_lens=sl, max_num_blocks=3),
         Bt.paged_decode(q.double(), kc.double(), vc.double(), bt, sl, 3))

    g = torch.Generator().manual_seed(3)
    lens = [6, 0, 41, 3]
    cu = torch.tensor([0, 6, 6, 47, 50], dtype=torch.int32)
    q, k, v = rn(g, 50, 2, 8), rn(g, 50, 2, 8), rn(g, 50, 2, 8)
    save("varlen_causal_rowlimit", "varlen", dict(q=q, k=k, v=v, cu_seqlens=cu, max_seqlen=30, causal=True),
         Bt.varlen_prefill(q.double(), k.double(), v.double(), cu, 30, True))
    assert sum(lens) == 50

    g = torch.Generator().manual_seed(5)
    q, k, v = rn(g, 2, 4, 1, 16), rn(g, 2, 2, 9, 16), rn(g, 2, 2, 9, 16)
    qs = q.float().abs().amax(-1).squeeze(-1) / 127
    ks = (k.float().abs().amax((-1, -2)) / 127).unsqueeze(-1).expand(2, 2, 9).contiguous()
    save("int8_decode", "int8", dict(q=q, k=k, v=v, q_scale=qs, k_scale=ks, cache_len=6),
         Bt.decode_int8(q, k.float(), v.double(), qs, ks, 6))


def next_rows():
    """Fixtures for the entry points beyond the eight hot-path ones."""
    # LSE forward and backward: the reference test_backward.py shape family (D=32 there; 8 here)
    g = torch.Generator().manual_seed(7)
    q, k, v, do = (torch.randn(1, 2, 9, 8, generator=g, dtype=torch.float64) for _ in range(4))
    out, lse = Bt.prefill_lse(q, k, v, True)
    save_multi("prefill_lse_causal", "prefill_lse", dict(q=q, k=k, v=v, causal=True), [out, lse])
    ot, lt = torch.tensor(out, dtype=torch.float64), torch.tensor(lse, dtype=torch.float64)
    save_multi("backward_causal", "backward", dict(dout=do, q=q, k=k, v=v, out=ot, lse=lt, causal=True),
               list(Bt.backward(do, q, k, v, ot, lt, True)))

    # sliding window + sink, INT8 KV cache
    g = torch.Generator().manual_seed(11)
    q, k, v = rn(g, 1, 4, 1, 8), rn(g, 1, 2, 30, 8), rn(g, 1, 2, 30, 8)
    save_multi("sliding_window", "sliding_window", dict(q=q, k=k, v=v, cache_len=25, window=7, sink=3),
               [Bt.decode_sliding_window(q.double(), k.double(), v.double(), 25, 7, 3)])
    g = torch.Generator().manual_seed(12)
    q = rn(g, 1, 4, 1, 8)
    k8 = torch.randint(-128, 128, (1, 2, 12, 8), generator=g, dtype=torch.int8)
    v8 = torch.randint(-128, 128, (1, 2, 12, 8), generator=g, dtype=torch.int8)
    ksc = (torch.rand(1, 2, 12, generator=g) * 0.02 + 0.001).half()
    vsc = (torch.rand(1, 2, 12, generator=g) * 0.02 + 0.001).half()
    save_multi("int8_kv_cache", "int8_kv_cache", dict(q=q, k_i8=k8, v_i8=v8, k_scale=ksc, v_scale=vsc, cache_len=9),
               [Bt.decode_int8_kv_cache(q, k8, v8, ksc, vsc, 9)])

    # token eviction with ties
    g = torch.Generator().manual_seed(13)
    k, v = rn(g, 2, 2, 10, 4), rn(g, 2, 2, 10, 4)
    sc = torch.randint(0, 4, (2, 10), generator=g).float()
    ko, vo, m = Bt.token_eviction(k, v, sc, 4)
    torch.save({"kind": "token_eviction", "args": dict(k=k, v=v, attn_scores=sc, num_evict=4),
                "outs": [torch.tensor(ko, dtype=torch.float16), torch.tensor(vo, dtype=torch.float16),
                         torch.tensor(m, dtype=torch.int32)]}, os.path.join(HERE, "token_eviction.pt"))
    print("wrote token_eviction")

    # speculative verify (test_speculative.py:115-157 shape family, smaller vocabulary)
    g = torch.Generator().manual_seed(42)
    tp = torch.softmax(torch.randn(2, 5, 64, generator=g), -1)
    dp = torch.softmax(torch.randn(2, 4, 64, generator=g), -1)
    tok = torch.randint(0, 64, (2, 4), generator=g)
    rv = torch.rand(2, 4, generator=g)
    acc, outs = Bt.speculative_verify(tp, dp, tok, rv, 4)
    torch.save({"kind": "speculative_verify", "args": dict(target_probs=tp, draft_probs=dp, draft_tokens=tok,
                                                           random_vals=rv, K=4),
                "outs": [torch.tensor(acc, dtype=torch.int32), torch.tensor(outs, dtype=torch.int64)]},
               os.path.join(HERE, "speculative_verify.pt"))
    print("wrote speculative_verify")


if __name__ == "__main__":
    if "--next-rows" not in sys.argv[1:]:
        main()
    next_rows()
