"""Builds libca_hip.so in-tree with hipcc for gfx950.

Usage: python continuum-attention_amd/build.py [--verbose]
The shared library is written next to this file and loaded by _native.py.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libca_hip.so")
SOURCES = ["ca_fwd.hip", "ca_bwd.hip", "ca_bwd_dkdv.hip", "ca_weights.hip", "ca_norm.hip",
           "ca_optim.hip", "ca_swiglu.hip", "ca_abi.hip", "ca_noalloc.hip"]
ARCH = os.environ.get("CA_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=fast",
    # packed fp32 VALU forms are disabled: some of them have returned wrong
    # results on this GPU pool with no error
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # keep MFMA accumulators in VGPRs: the dK/dV kernel otherwise shuffles
    # loop-carried tiles between AGPRs every iteration (~100 moves per tile)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall",
    "-Wno-unused-function",
]


# The attention kernels compute no output from a NaN or infinity they form
# themselves (the backward's fast-path segment math may form one in lane 0,
# which has no left neighbour, and discards it), so they are built assuming
# finite values, which lets fmax/fmin skip canonicalisation.  NaN or infinite
# inputs still propagate through their arithmetic (tests pin that).  The
# other sources (norms, optimizer, SwiGLU, weight rows) keep IEEE semantics:
# a diverging run's non-finite values must behave there as in torch.
_FINITE_MATH = ["-fno-honor-nans", "-fno-honor-infinities"]
# The attention kernels contract multiply-adds only within one source
# expression (their fused multiply-adds are written as fmaf): every template
# instantiation (fp32, bf16, fp16 operands; each head dim) then rounds the same
# arithmetic the same way, so the bf16 forward, which skips the zero limb
# products of bf16-valued operands, returns the fp32 forward's results on the
# same values bit for bit.  Measured: the same instruction counts in the tile
# loops as contraction across statements.
_ATTN = _FINITE_MATH + ["-ffp-contract=on"]

# Per-source flags: the dK/dV kernel schedules better with LLVM's max-ILP
# machine-scheduler strategy (about 2% faster); the other kernels are slower
# with it, so it applies to that translation unit only.
SOURCE_FLAGS = {"ca_fwd.hip": _ATTN,
                "ca_bwd.hip": _ATTN,
                "ca_bwd_dkdv.hip": _ATTN + ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def _jobs() -> int:
    # at most 8 compiles at once (one per source; hipcc is single-threaded)
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(8, n, len(SOURCES)))


def build(verbose: bool = False, extra_flags=None) -> str:
    build_dir = os.path.join(HERE, "_build")
    os.makedirs(build_dir, exist_ok=True)
    flags = HIPCC_FLAGS + list(extra_flags or [])

    def compile_one(src):
        obj = os.path.join(build_dir, src.replace(".hip", ".o"))
        cmd = [hipcc(), *flags, *SOURCE_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
        res = subprocess.run(cmd, capture_output=True, text=True)
        out = "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                        if "packed-fp32-ops" not in l)
        return src, cmd, obj, res.returncode, out

    objs = []
    with concurrent.futures.ThreadPoolExecutor(_jobs()) as pool:
        for src, cmd, obj, rc, out in pool.map(compile_one, SOURCES):
            if verbose:
                print(" ".join(cmd), flush=True)
            if rc != 0:
                raise RuntimeError(f"hipcc failed on {src}:\n{out}")
            if verbose and out.strip():
                print(out, flush=True)
            objs.append(obj)
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv))
