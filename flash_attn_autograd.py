"""Autograd wrapper of the drop-in module (mirrors the reference's
flash_attn_autograd.py:5-33): ``flash_attn(q, k, v, causal=True)`` runs the
MI355X forward with log-sum-exp and, on backward, the MI355X backward kernels.
fp16 inputs use forward_fp16_with_lse, fp32 inputs forward_with_lse."""
import torch

import flash_attn_v100


class FlashAttentionFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, causal=True):
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        if q.dtype == torch.float16:
            out, lse = flash_attn_v100.forward_fp16_with_lse(q, k, v, causal)
        elif q.dtype == torch.float32:
            out, lse = flash_attn_v100.forward_with_lse(q, k, v, causal)
        else:
            raise TypeError(f"flash_attn: q must be torch.float16 or torch.float32, got {q.dtype}")
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.causal = causal
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse = ctx.saved_tensors
        dq, dk, dv = flash_attn_v100.backward(dout.contiguous(), q, k, v, out, lse, ctx.causal)
        return dq, dk, dv, None


def flash_attn(q, k, v, causal=True):
    return FlashAttentionFunction.apply(q, k, v, causal)
