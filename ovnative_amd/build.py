"""Build libovnative_amd.so (HIP, gfx950) in-tree with hipcc.

The library is the product: the C ABI in include/ovnative_amd.h over the
kernels in ovnative_amd/csrc/.  It is compiled for gfx950 only, with
-ffp-contract=off (the kernels spell out every fused operation themselves) and
packed-FP32 instructions disabled.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libovnative_amd.so")
SOURCES = ["quant.hip", "gemm.hip", "gemm_skinny.hip", "gemm_f32.hip", "attn.hip", "capi.hip",
           "lm.hip", "diag.hip"]
HOST_SOURCES = ["ovw1.cpp"]  # plain host C++ (no device code)
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall", "-Wextra"]

HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in arch VGPRs: the per-block epilogue reads every accumulator
    # with VALU ops, which cannot take AGPR operands (each would cost an extra
    # v_accvgpr_read).
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-fvisibility=hidden",
    "-Wall",
    "-Wno-unused-function",
]


def build(verbose: bool = False) -> str:
    """Compile every HIP source and link the shared library; returns its path."""
    objs = []
    build_dir = os.path.join(HERE, "_build")
    os.makedirs(build_dir, exist_ok=True)
    procs = []
    for src in SOURCES:
        obj = os.path.join(build_dir, src.replace(".hip", ".o"))
        cmd = [HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT), src))
        objs.append(obj)
    for src in HOST_SOURCES:
        obj = os.path.join(build_dir, src.replace(".cpp", ".o"))
        cmd = [CXX, *HOST_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT), src))
        objs.append(obj)
    failed = []
    for p, src in procs:
        out = p.communicate()[0].decode(errors="replace")
        lines = [l for l in out.splitlines() if "packed-fp32-ops" not in l]
        if lines and (verbose or p.returncode):
            print("\n".join(lines), file=sys.stderr)
        if p.returncode:
            failed.append(src)
    if failed:
        raise RuntimeError(f"compile failed for {failed}")
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
