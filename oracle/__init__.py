"""CPU oracle for the W4A4 ConvRot linear path -- TEST INFRASTRUCTURE ONLY.

This package is the checker.  The shipped package never imports it; only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
do, and they use it to compute the expected answer, never as the thing that is
measured or shipped.

The arithmetic lives in ``convrot_oracle.c`` (plain C, built with gcc by
``oracle/build.py``); this module is a numpy/ctypes wrapper.  bf16 and f16
arrays are passed as their uint16 bit patterns, f32 as float32.

Reference semantics followed (paths relative to the reference repository):

* ``hadamard``           -- ``_int4/eager.py:20-46``
* ``rotate``             -- ``_int4/eager.py:65-79`` / ``:49-62`` (correctly rounded)
* ``quant_rows``         -- ``_int4/eager.py:104-120``; pack ``_int4/_codec.py:19-25``
* ``rotquant``           -- ``_int4/eager.py:191-195``
* ``unpack`` / ``pack``  -- ``_int4/_codec.py:19-36``
* ``int_gemm``           -- ``_int4/eager.py:160-162`` (exact integer accumulation)
* ``epilogue_f32``       -- ``_int4/eager.py:163-168`` with out_dtype float32
* ``epilogue_eager_bf16``-- ``_int4/eager.py:163-168`` with out_dtype bfloat16
* ``linear_eager``       -- ``_int4/eager.py:172-197``
* ``quantize_weight``    -- ``_int4/eager.py:123-135`` (fp16 weights, as ``int4_ops.py:344-350``)
* ``dequantize_weight``  -- ``_int4/eager.py:138-151``
* ``quant_rows8``        -- ``_int4/int8_eager.py:22-28`` (W8A8 tier)
* ``rotquant8``          -- ``_int4/int8_eager.py:81-83`` (activation) / ``:31-47`` (weight)
* ``int8_gemm``          -- exact int32 accumulators of the W8A8 product
  (``_int4/int4_gemm.hip:420-470``; the eager fp32 matmul of
  ``_int4/int8_eager.py:86`` equals it while partial sums stay below 2^24)
* ``linear_w8a8``        -- ``_int4/int8_eager.py:65-92`` with the exact product

Parity pinning: every function is checked in ``tests/test_oracle.py`` against
closed forms / brute force and against the golden vectors of ``tests/golden``.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

F32, BF16, F16 = 0, 1, 2

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH) or (
        os.path.getmtime(_LIB_PATH) < os.path.getmtime(os.path.join(_HERE, "convrot_oracle.c"))
    ):
        from .build import build

        build()
    lib = ctypes.CDLL(_LIB_PATH)
    vp, i = ctypes.c_void_p, ctypes.c_int
    lib.orc_rotate.argtypes = [vp, i, i, i, i, vp]
    lib.orc_rotate.restype = i
    lib.orc_quant_rows.argtypes = [vp, i, i, i, vp, vp, vp, vp]
    lib.orc_quant_rows.restype = None
    lib.orc_rotquant.argtypes = [vp, i, i, i, i, vp, vp, vp, vp]
    lib.orc_rotquant.restype = i
    lib.orc_int_gemm.argtypes = [vp, vp, i, i, i, vp]
    lib.orc_int_gemm.restype = None
    lib.orc_quant_rows8.argtypes = [vp, i, i, i, vp, vp]
    lib.orc_quant_rows8.restype = None
    lib.orc_rotquant8.argtypes = [vp, i, i, i, i, vp, vp, vp]
    lib.orc_rotquant8.restype = i
    lib.orc_int8_gemm.argtypes = [vp, vp, i, i, i, vp]
    lib.orc_int8_gemm.restype = None
    lib.orc_epilogue_f32.argtypes = [vp, vp, vp, vp, i, i, i, vp, vp]
    lib.orc_epilogue_f32.restype = None
    lib.orc_epilogue_eager_bf16.argtypes = [vp, vp, vp, vp, i, i, vp]
    lib.orc_epilogue_eager_bf16.restype = None
    lib.orc_hadamard.argtypes = [i, vp]
    lib.orc_hadamard.restype = None
    lib.orc_hadamard_sign.argtypes = [i, i, i]
    lib.orc_hadamard_sign.restype = i
    lib.orc_rotate_one_exact.argtypes = [vp, i, i, i, i, i]
    lib.orc_rotate_one_exact.restype = ctypes.c_double
    lib.orc_round_double_bits.argtypes = [ctypes.c_double, i]
    lib.orc_round_double_bits.restype = ctypes.c_uint16
    lib.orc_round_to.argtypes = [ctypes.c_float, i]
    lib.orc_round_to.restype = ctypes.c_float
    lib.orc_num_threads.argtypes = []
    lib.orc_num_threads.restype = i
    lib.orc_f32_to_bf16.argtypes = [ctypes.c_float]
    lib.orc_f32_to_bf16.restype = ctypes.c_uint16
    _lib = lib
    return lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _check(x, dt):
    want = np.float32 if dt == F32 else np.uint16
    if x.dtype != want:
        raise TypeError(f"dtype code {dt} expects numpy {want}, got {x.dtype}")
    return np.ascontiguousarray(x)


# ----------------------------------------------------------------------------
# scalar / array format helpers
# ----------------------------------------------------------------------------

def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    return h.view(np.float16).astype(np.float32)


def to_f32(x: np.ndarray, dt: int) -> np.ndarray:
    if dt == F32:
        return x.astype(np.float32)
    if dt == BF16:
        return bf16_to_f32(x)
    return f16_to_f32(x)


def round_double_bits(v: float, dt: int) -> int:
    return int(_load().orc_round_double_bits(float(v), dt))


# ----------------------------------------------------------------------------
# Hadamard, codec
# ----------------------------------------------------------------------------

def hadamard(G: int) -> np.ndarray:
    """H_G = kron^(log4 G)(H4) / sqrt(G) as float32 [G, G]  (_int4/eager.py:20-46)."""
    if G < 4 or (G & (G - 1)) or (G.bit_length() - 1) % 2:
        raise ValueError(f"Regular Hadamard size must be a power of 4, got {G}")
    out = np.empty((G, G), dtype=np.float32)
    _load().orc_hadamard(G, _p(out))
    return out


def pack(codes: np.ndarray) -> np.ndarray:
    """(..., K) int codes -> (..., K//2) int8; even k in the low nibble (_codec.py:19-25)."""
    c = np.asarray(codes).astype(np.int32)
    if c.shape[-1] % 2:
        raise ValueError(f"last dim must be even, got {c.shape[-1]}")
    lo = c[..., 0::2] & 0xF
    hi = c[..., 1::2] & 0xF
    return (lo | (hi << 4)).astype(np.uint8).view(np.int8)


def unpack(packed: np.ndarray) -> np.ndarray:
    """Inverse of pack with signed-nibble interpretation [-8, 7] (_codec.py:28-36)."""
    b = np.asarray(packed).view(np.uint8).astype(np.int32)
    lo = b & 0xF
    hi = (b >> 4) & 0xF
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    return np.stack([lo, hi], axis=-1).reshape(*b.shape[:-1], -1).astype(np.int8)


# ----------------------------------------------------------------------------
# rotation + quantization
# ----------------------------------------------------------------------------

def rotate(x: np.ndarray, dt: int, G: int) -> np.ndarray:
    """Correctly rounded block-Hadamard rotation of rows of x ([M, K])."""
    x = _check(x, dt)
    M, K = x.shape
    if K % G:
        raise ValueError(f"features {K} not divisible by group_size {G}")
    out = np.empty_like(x)
    _load().orc_rotate(_p(x), dt, M, K, G, _p(out))
    return out


def quant_rows(xr: np.ndarray, dt: int, noise: np.ndarray | None = None):
    """Rowwise symmetric int4 quantization -> (packed int8 [M,K/2], scales f32 [M], codes int8 [M,K])."""
    xr = _check(xr, dt)
    M, K = xr.shape
    if noise is not None:
        noise = _check(noise, dt)
    packed = np.empty((M, K // 2), dtype=np.int8)
    scales = np.empty((M,), dtype=np.float32)
    codes = np.empty((M, K), dtype=np.int8)
    _load().orc_quant_rows(_p(xr), dt, M, K, _p(noise), _p(packed), _p(scales), _p(codes))
    return packed, scales, codes


def rotquant(x: np.ndarray, dt: int, G: int, noise: np.ndarray | None = None):
    """Rotate + quantize -> (packed, scales, xr)."""
    x = _check(x, dt)
    M, K = x.shape
    if K % G:
        raise ValueError(f"features {K} not divisible by group_size {G}")
    if noise is not None:
        noise = _check(noise, dt)
    packed = np.empty((M, K // 2), dtype=np.int8)
    scales = np.empty((M,), dtype=np.float32)
    xr = np.empty_like(x)
    _load().orc_rotquant(_p(x), dt, M, K, G, _p(noise), _p(packed), _p(scales), _p(xr))
    return packed, scales, xr


def rotate_one_exact(x: np.ndarray, dt: int, G: int, m: int, col: int) -> float:
    """One correctly rounded rotated element via the exact integer accumulator only."""
    x = _check(x, dt)
    M, K = x.shape
    return float(_load().orc_rotate_one_exact(_p(x), dt, K, G, m, col))


# ----------------------------------------------------------------------------
# GEMM + epilogues
# ----------------------------------------------------------------------------

def int_gemm(Xp: np.ndarray, Wp: np.ndarray) -> np.ndarray:
    """Exact int32 accumulators acc[m, n] = sum_k qx[m,k] qw[n,k]."""
    Xp = np.ascontiguousarray(Xp.view(np.int8))
    Wp = np.ascontiguousarray(Wp.view(np.int8))
    M, Kp = Xp.shape
    N, Kp2 = Wp.shape
    if Kp != Kp2:
        raise ValueError(f"K mismatch: x {Xp.shape} w {Wp.shape}")
    acc = np.empty((M, N), dtype=np.int32)
    _load().orc_int_gemm(_p(Xp), _p(Wp), M, N, 2 * Kp, _p(acc))
    return acc


def epilogue_f32(acc, xs, ws, bias=None, out_bf16=False):
    """fl32(fl32(fl32(acc*xs)*ws)+b) (-> one RNE to bf16 when out_bf16)."""
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    ws = np.ascontiguousarray(ws, dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    M, N = acc.shape
    if out_bf16:
        out = np.empty((M, N), dtype=np.uint16)
        _load().orc_epilogue_f32(_p(acc), _p(xs), _p(ws), _p(b), M, N, 1, None, _p(out))
    else:
        out = np.empty((M, N), dtype=np.float32)
        _load().orc_epilogue_f32(_p(acc), _p(xs), _p(ws), _p(b), M, N, 0, _p(out), None)
    return out


def epilogue_eager_bf16(acc, xs, ws, bias=None):
    """The eager bf16 rounding chain o1..o4 -> bf16 bits."""
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    ws = np.ascontiguousarray(ws, dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    M, N = acc.shape
    out = np.empty((M, N), dtype=np.uint16)
    _load().orc_epilogue_eager_bf16(_p(acc), _p(xs), _p(ws), _p(b), M, N, _p(out))
    return out


def linear_eager(x, dt, qweight, wscales, bias=None, G=256):
    """The whole eager ConvRot W4A4 linear (_int4/eager.py:172-197).

    x: [M, K] (bits for bf16/f16), returns the output in x's dtype
    (bf16 bits / f16 bits / float32).  bias holds float values (e.g. fp16
    values widened to float32).
    """
    if dt == F16:
        raise NotImplementedError("f16 activations: eager output rounding chain is f16; not modelled")
    packed, xs, _ = rotquant(x, dt, G)
    acc = int_gemm(packed, qweight)
    if dt == BF16:
        return epilogue_eager_bf16(acc, xs, wscales, bias)
    return epilogue_f32(acc, xs, wscales, bias, out_bf16=False)


def quantize_weight(w: np.ndarray, dt: int, G: int, noise: np.ndarray | None = None):
    """quantize_convrot_w4a4_weight semantics -> (packed int8 [N,K/2], scales f32 [N])."""
    if w.shape[-1] % 64:
        raise ValueError(f"in_features {w.shape[-1]} not divisible by quant_group_size 64")
    packed, scales, _ = rotquant(w, dt, G, noise)
    return packed, scales


def dequantize_weight(packed: np.ndarray, scales: np.ndarray, G: int) -> np.ndarray:
    """(_int4/eager.py:138-151): unpack * scale, rotate back, in float64 here."""
    w = unpack(packed).astype(np.float64) * scales.astype(np.float64)[:, None]
    H = hadamard(G).astype(np.float64)
    N, K = w.shape
    return (w.reshape(N, K // G, G) @ H.T).reshape(N, K)


# ----------------------------------------------------------------------------
# W8A8 tier
# ----------------------------------------------------------------------------

def quant_rows8(xr: np.ndarray, dt: int):
    """Rowwise symmetric int8 quantization -> (codes int8 [M,K], scales f32 [M])."""
    xr = _check(xr, dt)
    M, K = xr.shape
    q = np.empty((M, K), dtype=np.int8)
    scales = np.empty((M,), dtype=np.float32)
    _load().orc_quant_rows8(_p(xr), dt, M, K, _p(q), _p(scales))
    return q, scales


def rotquant8(x: np.ndarray, dt: int, G: int):
    """Rotate + int8 quantize -> (codes int8 [M,K], scales f32 [M], xr)."""
    x = _check(x, dt)
    M, K = x.shape
    if K % G:
        raise ValueError(f"features {K} not divisible by group_size {G}")
    q = np.empty((M, K), dtype=np.int8)
    scales = np.empty((M,), dtype=np.float32)
    xr = np.empty_like(x)
    _load().orc_rotquant8(_p(x), dt, M, K, G, _p(q), _p(scales), _p(xr))
    return q, scales, xr


def int8_gemm(X: np.ndarray, W: np.ndarray) -> np.ndarray:
    """Exact int32 accumulators acc[m, n] = sum_k x[m,k] w[n,k] of int8 operands."""
    X = np.ascontiguousarray(X.view(np.int8))
    W = np.ascontiguousarray(W.view(np.int8))
    M, K = X.shape
    N, K2 = W.shape
    if K != K2:
        raise ValueError(f"K mismatch: x {X.shape} w {W.shape}")
    acc = np.empty((M, N), dtype=np.int32)
    _load().orc_int8_gemm(_p(X), _p(W), M, N, K, _p(acc))
    return acc


def quantize_weight8(w: np.ndarray, dt: int, G: int):
    """quantize_convrot_w8a8_weight semantics -> (int8 [N,K], scales f32 [N])."""
    q, scales, _ = rotquant8(w, dt, G)
    return q, scales


def linear_w8a8(x, dt, qweight, wscales, bias=None, G=256, out_bf16=True):
    """convrot_w8a8_linear (_int4/int8_eager.py:65-92) with the exact integer
    product: rotate + int8 quantize x, exact int32 GEMM, fl32 epilogue, one RNE
    to bf16 when out_bf16 (x bf16), else the f32 values."""
    q, xs, _ = rotquant8(x, dt, G)
    acc = int8_gemm(q, qweight)
    return epilogue_f32(acc, xs, wscales, bias, out_bf16=out_bf16)


def num_threads() -> int:
    """Threads of the oracle's parallel row loops (OpenMP, OMP_NUM_THREADS)."""
    return int(_load().orc_num_threads())
