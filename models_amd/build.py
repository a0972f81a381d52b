"""Builds libjmodels_attn.so (gfx950) in-tree with hipcc.

Run ``python -m models_amd.build`` or call :func:`build`. The library is the product: the HIP
kernels (csrc/jma_kernels.hip, csrc/jma_quant.hip) and the C-ABI runtime (csrc/jma_runtime.cpp) declared in
include/jmodels_attn.h.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_NAME = "libjmodels_attn.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
SOURCES = [os.path.join(HERE, "csrc", "jma_kernels.hip"), os.path.join(HERE, "csrc", "jma_quant.hip"),
           os.path.join(HERE, "csrc", "jma_runtime.cpp")]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-fvisibility=hidden",
    # no packed-FP32 instructions in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # keep single-lane atomics as written: the wave-level aggregation rewrite waits for an
    # atomic's result right after issuing it, which puts a memory round trip in front of the
    # decode kernel's tile loads
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    # the decode kernel's seven leading scalar arguments arrive in SGPRs at wave start (kernels
    # whose first argument is a struct preload nothing)
    "-mllvm", "-amdgpu-kernarg-preload-count=7",
    # matrix-op results and accumulators in ordinary vector registers: the accumulation registers
    # then hold only what a kernel pins there (the d-512 prefill's q operands) or what exceeds 256
    # vector registers, instead of every matrix result plus copies (several decode and prefill
    # instances stop spilling)
    "-mllvm", "--amdgpu-mfma-vgpr-form=true",
    "-Wall",
    "-Wno-unused-result",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.isabs(cand) and os.path.exists(cand) or not os.path.isabs(cand)):
            return cand
    return "hipcc"


def build(verbose: bool = False) -> str:
    """Compiles every source for gfx950 and links the shared library; returns its path."""
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", os.path.join(ROOT, "include"), *SOURCES, "-o", LIB_PATH + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    errors = [ln for ln in (proc.stdout + proc.stderr).splitlines()
              if "packed-fp32-ops" not in ln and ln.strip()]
    if proc.returncode != 0:
        sys.stderr.write("\n".join(errors) + "\n")
        raise RuntimeError(f"hipcc failed with exit code {proc.returncode}")
    if verbose and errors:
        print("\n".join(errors))
    # A kernel template whose host-side instantiation fails leaves its launch stub undefined; the
    # shared library still links, so check for the library's own unresolved symbols here.
    nm = subprocess.run(["nm", "-D", "--undefined-only", LIB_PATH + ".tmp"], capture_output=True, text=True)
    own = [ln.split()[-1] for ln in nm.stdout.splitlines() if "jma" in ln or "jmodels" in ln]
    if own:
        os.remove(LIB_PATH + ".tmp")
        raise RuntimeError(f"built library leaves its own symbols undefined: {own}")
    os.replace(LIB_PATH + ".tmp", LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
