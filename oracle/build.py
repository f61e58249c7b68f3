"""Build recipe for the CPU oracle (test infrastructure only).

``python -m oracle.build`` or ``oracle.build.build()`` compiles ifn_oracle.c
with gcc into ``oracle/libifn_oracle.so`` (git-ignored; it travels to the GPU
box with the tree).  ``-ffp-contract=off`` keeps every multiply and add a
separately rounded fp32 operation, so the oracle's accumulation order is the
one written in the source.

There is no ``oracle/_ref`` build: the reference's implementation of this path
is Python/tinygrad (its kernels/ and cache/ modules are 0-byte placeholders),
so there are no C/C++ sources under /root/reference to compile.
"""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "ifn_oracle.c")
LIB_PATH = os.path.join(HERE, "libifn_oracle.so")


def build() -> str:
    tmp = LIB_PATH + ".tmp"
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
           "-Wall", "-Wextra", "-o", tmp, SRC, "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build())
