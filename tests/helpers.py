"""Shared helpers for the parity tests: seeded CPU inputs and tolerance checks."""
import torch

# Tolerances stated by the north star: fp16 paths max-abs <= 2e-3 with rtol 1e-2
# against the fp32 oracle; INT8 rel-L2 <= 1.5e-2 against the quantize-dequantize path.
ATOL = 2e-3
RTOL = 1e-2
INT8_REL_L2 = 1.5e-2


def randn(gen, *shape, dtype=torch.float16):
    """N(0,1) values drawn on the CPU from `gen` (identical inputs for CPU and GPU)."""
    return torch.randn(*shape, generator=gen, dtype=torch.float32).to(dtype)


def assert_close(out, ref, atol=ATOL, rtol=RTOL, what=""):
    out = out.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert out.shape == ref.shape, (what, out.shape, ref.shape)
    nan_o, nan_r = torch.isnan(out), torch.isnan(ref)
    assert torch.equal(nan_o, nan_r), f"{what}: NaN pattern differs ({int(nan_o.sum())} vs {int(nan_r.sum())})"
    o, r = out[~nan_o], ref[~nan_r]
    if o.numel() == 0:
        return
    err = (o - r).abs()
    bad = err > atol + rtol * r.abs()
    assert not bool(bad.any()), (
        f"{what}: {int(bad.sum())}/{o.numel()} elements out of tolerance; max abs err {err.max().item():.3e}")


def rel_l2(out, ref):
    out = out.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return ((out - ref).norm() / ref.norm()).item()
