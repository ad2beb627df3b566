"""In-tree build of the MI355X attention library and its PyTorch extension.

Produces, next to this file:
  libflash_attn_mi355x.so   HIP kernels + C ABI (include/flash_attn_mi355x.h), gfx950
  _flash_attn_v100*.so      PyTorch-ROCm extension exposing the reference API
  libfa_ceilings.so         roofline probes used by bench.py --ceilings (not the library)

Run ``python flash_attn_v100_amd/build.py`` (or ``__graft_entry__.build()``); it is a
standalone script so it works before the package is importable.
Compilation is explicit hipcc / g++ so nothing is hipified or JIT-cached
outside the tree.
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "libflash_attn_mi355x.so"
CEILINGS_LIB = "libfa_ceilings.so"
EXT_NAME = "_flash_attn_v100"
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

KERNEL_SOURCES = ["decode.hip", "prefill.hip", "train.hip", "train_fp32.hip", "token_ops.hip", "tp_ops.hip"]
HOST_SOURCES = ["capi.cpp"]

HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # Keep the compiler from forming packed-fp32 VALU ops (v_pk_*_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-variable", "-Wno-unused-but-set-variable",
]
# MFMA accumulators in ordinary VGPRs: without it the compiler parks them in
# AGPRs and copies them back and forth around every branch of the kernels.
# The fp32 training kernels (train_fp32.hip) need more operand registers than
# 256 VGPRs hold, so they keep their accumulators (only ever accumulated and
# stored) in AGPRs.
VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
SOURCE_FLAGS = {"decode.hip": VGPR_FORM, "prefill.hip": VGPR_FORM, "train.hip": VGPR_FORM}


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError("build step failed:\n" + " ".join(cmd) + "\n" + r.stdout)
    # hipcc's host pass does not know the packed-fp32 feature; drop that noise.
    noise = "is not a recognized feature for this target"
    out = "\n".join(l for l in r.stdout.splitlines() if noise not in l)
    if out.strip():
        print(out)


def lib_path() -> str:
    return os.path.join(PKG_DIR, LIB_NAME)


def ext_path() -> str:
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    return os.path.join(PKG_DIR, EXT_NAME + suffix)


def build_library(verbose: bool = True) -> str:
    """Compile the HIP kernels and the C ABI into libflash_attn_mi355x.so.

    ``FA_EXTRA_HIPFLAGS`` (environment, space-separated) is appended to every
    kernel compile: it is how measurement builds switch on the tuning and
    ablation macros the kernel sources document (e.g. ``-DFA_ABL_NOCOPY``).
    The shipped build leaves it unset."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    objs = []
    jobs = []
    extra = os.environ.get("FA_EXTRA_HIPFLAGS", "").split()
    for src in KERNEL_SOURCES + HOST_SOURCES:
        obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
        cmd = [HIPCC, *HIP_FLAGS, *SOURCE_FLAGS.get(src, []), *extra, "-I", os.path.join(REPO_DIR, "include")]
        if src.endswith(".cpp"):
            cmd += ["-x", "hip"]
        cmd += ["-c", os.path.join(CSRC, src), "-o", obj]
        jobs.append(cmd)
        objs.append(obj)
    with ThreadPoolExecutor(max_workers=min(len(jobs), 8)) as ex:
        list(ex.map(_run, jobs))
    out = lib_path()
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", out])
    if verbose:
        print(f"[build] {out}")
    return out


def build_ceilings(verbose: bool = True) -> str:
    """Compile the roofline probes (csrc/ceilings.hip) into libfa_ceilings.so,
    a separate library that only bench.py --ceilings loads."""
    out = os.path.join(PKG_DIR, CEILINGS_LIB)
    _run([HIPCC, *HIP_FLAGS, "-shared", os.path.join(CSRC, "ceilings.hip"), "-o", out])
    if verbose:
        print(f"[build] {out}")
    return out


def build_extension(verbose: bool = True) -> str:
    """Compile the pybind11/ATen binding against torch and link the C-ABI library."""
    import torch
    from torch.utils import cpp_extension

    torch_dir = os.path.dirname(torch.__file__)
    includes = cpp_extension.include_paths() + [
        sysconfig.get_paths()["include"],
        os.path.join(ROCM, "include"),
        os.path.join(REPO_DIR, "include"),
    ]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    out = ext_path()
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=" + EXT_NAME,
           "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-Wno-deprecated-declarations"]
    for inc in includes:
        cmd += ["-I", inc]
    cmd += [os.path.join(CSRC, "binding.cpp"), "-o", out,
            "-L", PKG_DIR, "-lflash_attn_mi355x",
            "-L", os.path.join(torch_dir, "lib"),
            "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python", "-lamdhip64",
            "-Wl,-rpath,$ORIGIN", "-Wl,-rpath," + os.path.join(torch_dir, "lib")]
    _run(cmd)
    if verbose:
        print(f"[build] {out}")
    return out


def build_all(verbose: bool = True) -> None:
    build_library(verbose)
    build_extension(verbose)
    build_ceilings(verbose)


if __name__ == "__main__":
    build_all()
    sys.exit(0)
