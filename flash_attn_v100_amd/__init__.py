"""MI355X (gfx950) implementation of the flash_attn_v100 attention hot path.

Importing this package loads the in-tree native extension
(``_flash_attn_v100*.so``, which links ``libflash_attn_mi355x.so``) and
re-exports the reference module's functions.  There is no Python or CPU
fallback: a missing or stale build raises ImportError.  Build with
``python flash_attn_v100_amd/build.py``.
"""
from __future__ import annotations

import importlib
import os

import torch  # noqa: F401  (loads libamdhip64 / libc10_hip before the extension)

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))

try:
    _ext = importlib.import_module("flash_attn_v100_amd._flash_attn_v100")
except ImportError as e:  # pragma: no cover - exercised only without a build
    raise ImportError(
        "flash_attn_v100_amd: native extension not built in " + _PKG_DIR +
        " (run `python flash_attn_v100_amd/build.py`): " + str(e)) from e

# The reference module's exported names (flash_attn.cpp:224-255).
API_NAMES = (
    "forward", "forward_fp16", "forward_with_lse", "forward_fp16_with_lse", "backward",
    "forward_fp16_warp", "forward_decode_fp16", "forward_decode_gqa_fp16",
    "forward_decode_gqa_fp16_out", "forward_fp16_wmma", "forward_prefill_gqa_fp16",
    "forward_prefill_gqa_fp16_out", "forward_prefill_gqa_fp16_warp",
    "forward_paged_decode_gqa_fp16", "forward_decode_int8_gqa", "forward_varlen_prefill_fp16",
    "forward_decode_gqa_fp16_stream", "forward_varlen_prefill_fp16_stream",
    "forward_continuous_batching_fp16", "async_h2d_transfer", "alloc_pinned_tensor",
    "pipeline_decode_step", "pipeline_decode_step_out", "speculative_verify",
    "forward_decode_int8_kv_cache_gqa", "token_eviction", "forward_decode_sliding_window_gqa",
    "cross_gpu_allreduce_fp16", "scatter_heads", "gather_heads",
)

# The eight north-star entry points, all native.
HOT_PATH = (
    "forward_fp16", "forward_fp16_wmma", "forward_decode_fp16", "forward_decode_gqa_fp16",
    "forward_continuous_batching_fp16", "forward_varlen_prefill_fp16",
    "forward_paged_decode_gqa_fp16", "forward_decode_int8_gqa",
)

for _name in API_NAMES:
    globals()[_name] = getattr(_ext, _name)

__all__ = list(API_NAMES)


def library_path() -> str:
    """Path of the C-ABI shared library the extension is linked against."""
    return os.path.join(_PKG_DIR, "libflash_attn_mi355x.so")


def version() -> str:
    return _ext._fa_version()
