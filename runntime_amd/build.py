"""Builds libmoe.so (the HIP kernels and the C ABI) for gfx950, in-tree.

hipcc cross-compiles on a machine without a GPU, so this runs anywhere the
ROCm toolchain is installed. Output: runntime_amd/libmoe.so.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmoe.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    # Packed-f32 VALU forms are kept out of the device code on purpose.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]
# Per-file floating-point contraction. The router follows a canonical f32
# order with explicit fmaf(): nothing else may be fused there.
PER_FILE = {
    "router.hip": ["-ffp-contract=off"],
    "norm.hip": ["-ffp-contract=off"],
}
SOURCES = ["moe_abi.hip", "router.hip", "dispatch.hip", "expert.hip", "gemm.hip", "gemm_wide.hip", "gemm_i8.hip", "pack.hip", "norm.hip", "float.hip", "attn.hip", "linear.hip"]


# Host-only C++ (no device code), compiled by the host compiler.
HOST_SOURCES = ["viterbi.cpp"]
CXX = os.environ.get("CXX", "g++")


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    if src in HOST_SOURCES:
        cmd = [CXX, "-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-c",
               os.path.join(CSRC, src), "-o", obj]
    else:
        cmd = [HIPCC, *COMMON, *PER_FILE.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


NODE_INCLUDE = "/usr/include/node"
NAPI_SRC = os.path.join(HERE, "napi", "runntime_moe_addon.cc")
NAPI_OUT = os.path.join(HERE, "napi", "runntime_moe.node")


def build_napi(verbose: bool = False):
    """The Node addon (runntime_amd/napi/runntime_moe.node) over libmoe.so,
    when Node's headers are installed; returns its path or None."""
    if not os.path.exists(os.path.join(NODE_INCLUDE, "node_api.h")):
        if verbose:
            print(f"no {NODE_INCLUDE}/node_api.h: the Node addon is not built")
        return None
    tmp = NAPI_OUT + ".tmp"
    cmd = [CXX, "-O2", "-std=c++17", "-shared", "-fPIC", "-fvisibility=hidden",
           "-DNODE_GYP_MODULE_NAME=runntime_moe", f"-I{NODE_INCLUDE}", NAPI_SRC, f"-L{HERE}",
           "-lmoe", "-Wl,-rpath,$ORIGIN/..", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"addon build failed:\n{r.stderr}")
    os.replace(tmp, NAPI_OUT)
    if verbose:
        print(NAPI_OUT)
    return NAPI_OUT


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES + HOST_SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(LIB)
    build_napi(verbose)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
