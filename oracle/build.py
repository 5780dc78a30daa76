"""Builds the C half of the oracle (oracle/liboracle_moe.so) with gcc.

TEST INFRASTRUCTURE ONLY (the checker, never the product)."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle_moe.so")


def build():
    src = os.path.join(HERE, "moe_oracle.c")
    tmp = LIB + ".tmp"
    subprocess.run(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-Wall", "-o", tmp, src, "-lm"], check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
