"""Build recipe for the CPU oracle (test infrastructure; see oracle/__init__.py).

Compiles ``convrot_oracle.c`` with gcc into ``oracle/liboracle.so``.  The
reference's own native code (``_int4/int4_gemm.hip``) is not built here: it
targets RDNA4 WMMA (gfx12) only and does not compile for any CPU or for gfx950,
so there is no ``oracle/_ref`` build for this path.
"""
from __future__ import annotations

import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))


def build() -> str:
    src = os.path.join(_HERE, "convrot_oracle.c")
    out = os.path.join(_HERE, "liboracle.so")
    tmp = out + ".tmp"
    cmd = ["gcc", "-O2", "-std=gnu11", "-fno-fast-math", "-ffp-contract=off", "-Wall", "-fopenmp",
           "-shared", "-fPIC", src, "-o", tmp, "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build())
