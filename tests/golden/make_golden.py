"""Writes the small golden fixtures in this directory.

Outputs come from oracle/brute.py, the fp64 loop restatement of the reference
kernels (flash_attn_kernel.cu / continuous_batching_kernel.cu), evaluated on
seeded inputs that mirror the reference's own test cases where it has them
(test.py seed 0, test_decode.py paged layout seed 2025, test_continuous_batching.py
cases).  The reference ships no golden vectors, so these fixtures freeze the
independent restatement; tests/test_oracle.py checks the vectorised oracle
against them and the GPU tests check the kernels against the oracle.

Run:  python tests/golden/make_golden.py
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


if __name__ == "__main__":
    main()
