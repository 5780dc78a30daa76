"""Builds libwindlass_moe.so (gfx950) in-tree with hipcc.

Usage: python -m windlass_amd.build   (or windlass_amd.build.build())
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libwindlass_moe.so")
SOURCES = ["moe_decode.hip", "moe_batched.hip", "synth.hip", "native.hip", "noalloc.hip", "moe_host.cpp",
           "expert_files.cpp", "safetensors.cpp", "loader.cpp", "attention.hip", "attn_host.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Packed-FP32 VALU forms are disabled on purpose: some of them have given
# wrong results on this hardware without any error.
DEVICE_FLAGS = ["--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
# Kernel arguments preloaded into SGPRs (gfx950 kernarg preloading): the
# first dwords of every kernel's scalar arguments are in registers when its
# waves start (a struct argument is not preloaded), so the first loads of the
# decode kernel need no memory round trip to learn their addresses.
# 14 = internal.h kPreloadDwords.
PRELOAD_FLAGS = ["-mllvm", "-amdgpu-kernarg-preload-count=14"]
COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function", "-Wno-unknown-pragmas"]


def build(verbose: bool = False) -> str:
    """Compiles every source (in parallel, one hipcc per source), then links."""
    from concurrent.futures import ThreadPoolExecutor

    def compile_one(src):
        path = os.path.join(CSRC, src)
        obj = os.path.join(CSRC, "_build", src + ".o")
        os.makedirs(os.path.dirname(obj), exist_ok=True)
        cmd = [HIPCC] + COMMON + DEVICE_FLAGS + PRELOAD_FLAGS + ["-c", path, "-o", obj]
        if src.endswith(".cpp"):  # host code: no kernels, but compiled for gfx950 only like the rest
            cmd = [HIPCC] + COMMON + DEVICE_FLAGS + ["-c", path, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            sys.stderr.write(r.stdout + r.stderr)
            raise RuntimeError(f"hipcc failed on {src}")
        return obj

    jobs = max(1, min(len(SOURCES), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(compile_one, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC] + DEVICE_FLAGS + ["-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("link of libwindlass_moe.so failed")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
