"""Ahead-of-time build of the gfx950 kernel library (replaces the reference's
JIT ``_int4/build.py``, which compiled for whatever arch the GPU reported).

``build()`` runs hipcc for gfx950 only and writes ``libconvrot_gfx950.so`` next
to this file.  The library is loaded by ``native.py``; nothing builds at import
or at first use.
"""
from __future__ import annotations

import os
import shutil
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
_PKG = os.path.dirname(_HERE)
_CSRC = os.path.join(_PKG, "csrc")
SOURCES = ("rotquant.hip", "gemm.hip", "gemm_bf6.hip", "lora.hip", "capi.hip")
HEADERS = ("common.h", "gemm_common.h", "b6t_layout.h")
ARCH = "gfx950"


def lib_path() -> str:
    return os.path.join(_HERE, "libconvrot_gfx950.so")


def sources() -> list[str]:
    return [os.path.join(_CSRC, s) for s in SOURCES]


def is_stale() -> bool:
    out = lib_path()
    if not os.path.exists(out):
        return True
    deps = sources() + [os.path.join(_CSRC, h) for h in HEADERS] + [
        os.path.join(os.path.dirname(_PKG), "include", "convrot_mi355x.h")]
    t = os.path.getmtime(out)
    return any(os.path.getmtime(d) > t for d in deps if os.path.exists(d))


def hipcc_cmd(out: str) -> list[str]:
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    return [
        hipcc, "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-shared",
        "-fvisibility=hidden", "-ffp-contract=off",
        "-fhip-fp32-correctly-rounded-divide-sqrt",
        # packed-fp32 VALU forms stay off (compiler-generated v_pk_*_f32 disabled)
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        *sources(), "-o", out,
    ]


def build(verbose: bool = False) -> str:
    out = lib_path()
    tmp = out + ".tmp"
    cmd = hipcc_cmd(tmp)
    if verbose:
        print("building:", " ".join(cmd))
    cp = subprocess.run(cmd, capture_output=True, text=True)
    if cp.returncode != 0 or not os.path.exists(tmp):
        raise RuntimeError(f"hipcc build failed:\n{cp.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print("built:", build(verbose=True))
