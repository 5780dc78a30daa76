"""Builds the shim caller (tests/shim/reference_caller.cpp) for gfx950 into
tests/shim/_build/reference_caller, linked against the in-tree
libwindlass_moe.so (found at run time relative to the binary)."""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT = os.path.join(HERE, "_build", "reference_caller")


def build(out=OUT):
    sys.path.insert(0, ROOT)
    from windlass_amd import build as B
    os.makedirs(os.path.dirname(out), exist_ok=True)
    lib_dir = os.path.dirname(B.LIB)
    rpath = os.path.relpath(lib_dir, os.path.dirname(out))
    cmd = [B.HIPCC, "-O2", "-std=c++17", "-Wall", "-Werror"] + B.DEVICE_FLAGS + [
        "-I", os.path.join(ROOT, "include"), os.path.join(HERE, "reference_caller.cpp"), "-o", out,
        "-L", lib_dir, "-lwindlass_moe", "-Wl,-rpath,$ORIGIN/" + rpath]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed on tests/shim/reference_caller.cpp")
    return out


if __name__ == "__main__":
    print(build())
