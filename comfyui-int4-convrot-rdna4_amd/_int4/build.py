"""Ahead-of-time build of the gfx950 kernel library (replaces the reference's
JIT ``_int4/build.py``, which compiled for whatever arch the GPU reported).

``build()`` runs hipcc for gfx950 only: every source is compiled to an object
in parallel (``_build/`` next to this file), then the objects are linked into
``libconvrot_gfx950.so`` next to this file.  The library is loaded by
``native.py``; nothing builds at import or at first use.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

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


def _deps() -> list[str]:
    return sources() + [os.path.join(_CSRC, h) for h in HEADERS] + [
        os.path.join(os.path.dirname(_PKG), "include", "convrot_mi355x.h")]


def is_stale() -> bool:
    out = lib_path()
    if not os.path.exists(out):
        return True
    t = os.path.getmtime(out)
    return any(os.path.getmtime(d) > t for d in _deps() if os.path.exists(d))


def _hipcc() -> str:
    return shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


# Flags of every translation unit.  -ffp-contract=off keeps the epilogue's
# separately rounded products and sums; packed-fp32 VALU forms stay off
# (compiler-generated v_pk_*_f32 disabled).
CFLAGS = ["-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-fvisibility=hidden", "-ffp-contract=off",
          "-fhip-fp32-correctly-rounded-divide-sqrt", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc_cmd(out: str) -> list[str]:
    """One-step command (all sources, one hipcc process); build() uses the
    equivalent compile-then-link steps below."""
    return [_hipcc(), *CFLAGS, "-shared", *sources(), "-o", out]


def _obj_dir() -> str:
    d = os.path.join(_HERE, "_build")
    os.makedirs(d, exist_ok=True)
    return d


def _compile(src: str) -> str:
    obj = os.path.join(_obj_dir(), os.path.basename(src) + ".o")
    tmp = obj + ".tmp"
    cp = subprocess.run([_hipcc(), *CFLAGS, "-c", src, "-o", tmp], capture_output=True, text=True)
    if cp.returncode != 0 or not os.path.exists(tmp):
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{cp.stderr}")
    os.replace(tmp, obj)
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> str:
    out = lib_path()
    tmp = out + ".tmp"
    srcs = sources()
    if verbose:
        print("building:", " ".join([_hipcc(), *CFLAGS, "-c", "<src>"]), "for", ", ".join(SOURCES))
    n = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=n) as ex:
        objs = list(ex.map(_compile, srcs))
    cp = subprocess.run([_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp],
                        capture_output=True, text=True)
    if cp.returncode != 0 or not os.path.exists(tmp):
        raise RuntimeError(f"hipcc link failed:\n{cp.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print("built:", build(verbose=True))
