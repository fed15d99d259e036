"""Builds libnsg_spec.so (the C-ABI library of the verify step) in-tree.

    python -m nanosglang_amd.build

compiles every ``csrc/*.hip`` for gfx950 with hipcc and links them into
``nanosglang_amd/libnsg_spec.so`` (the C ABI), then ``csrc/torch_ops.cpp``
into ``nanosglang_amd/libnsg_torch.so`` (the torch operators over it).
Packed-fp32 instructions are disabled on purpose
(``-target-feature -packed-fp32-ops``).
"""

from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libnsg_spec.so")
ARCH = os.environ.get("NSG_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-file additions.  spec_accept.hip: logits are never NaN (a NaN logit
# makes the reference's softmax NaN too), so max/min need no NaN
# canonicalisation -- it doubled the cost of the per-logit max in the
# acceptance pass.  verify_attention.hip likewise: its scores come from
# finite Q and K (masked ones are a finite sentinel), and the canonicalising
# maxes were 100 of the kernel's 3,240 instructions.  linear.hip, lm_head.hip: their asm copies into LDS set
# m0 and say so in their clobber lists, which the compiler warns about for
# every kernel instance (the files' kernels use m0 for nothing else).
# The files with MFMA kernels keep the accumulators in ordinary VGPRs
# (-amdgpu-mfma-vgpr-form): left to its heuristics the compiler put them in
# AGPRs and copied them back and forth around every softmax / epilogue step
# (about 490 v_accvgpr moves in the verify-shape attention kernel, 4,200 in
# linear.hip); measured 8.74 -> 8.40 us per cache-cold verify-shape
# attention launch, 80 -> 77 us for the 160-row lm_head, 12,000 -> 12,160
# tok/s end to end, outputs bit-identical.
MFMA_VGPR = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
FILE_FLAGS = {"spec_accept.hip": ["-fno-honor-nans"],
              "linear.hip": ["-Wno-inline-asm", *MFMA_VGPR],
              "lm_head.hip": ["-Wno-inline-asm", *MFMA_VGPR],
              "verify_attention.hip": ["-fno-honor-nans", *MFMA_VGPR]}


def _hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found; the verify-step library needs ROCm's hipcc")


def _compile(src: str, obj: str) -> None:
    cmd = [_hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o",
           obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


TORCH_OPS_SRC = os.path.join(CSRC, "torch_ops.cpp")
TORCH_OPS_LIB = os.path.join(PKG, "libnsg_torch.so")


def build_torch_ops(verbose: bool = True) -> str:
    """The torch operators (csrc/torch_ops.cpp: TORCH_LIBRARY over the C ABI)
    as libnsg_torch.so, host C++ against the installed PyTorch-ROCm, linked to
    libnsg_spec.so beside it."""
    import torch
    from torch.utils import cpp_extension
    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cxx = os.environ.get("CXX", shutil.which("g++") or "c++")
    tmp = TORCH_OPS_LIB + ".tmp"
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wno-unused-function",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           *[f"-I{d}" for d in cpp_extension.include_paths()], f"-I{rocm}/include",
           TORCH_OPS_SRC, "-o", tmp, f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch",
           "-ltorch_cpu", "-ltorch_hip", f"-L{rocm}/lib", "-lamdhip64", f"-L{PKG}",
           "-lnsg_spec", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"torch operator library failed to build:\n{r.stderr}")
    os.replace(tmp, TORCH_OPS_LIB)
    if verbose:
        print(f"built {TORCH_OPS_LIB}")
    return TORCH_OPS_LIB


def build(verbose: bool = True) -> str:
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    objdir = os.path.join(PKG, "_build")
    os.makedirs(objdir, exist_ok=True)
    objs = [os.path.join(objdir, os.path.basename(s)[:-4] + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        list(ex.map(_compile, srcs, objs))
    tmp = LIB + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    build_torch_ops(verbose)
    return LIB


if __name__ == "__main__":
    build()
