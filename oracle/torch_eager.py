"""Torch restatement of the reference's eager W4A4 ConvRot linear -- TEST
INFRASTRUCTURE ONLY (the CPU baseline that bench.py times, and a checker).

It runs the same torch operations, in the same dtypes, as the reference's eager
path (``_int4/eager.py``), so on the same CPU it reproduces that path's output
bit for bit (``tests/test_oracle.py`` pins it to the reference's config-1
golden SHA-256).  Where torch's own bf16 matmul is not correctly rounded (rare
near-ties of the rotation) it follows torch, unlike ``convrot_oracle.c``.

Stages, each citing the reference lines it restates:

* ``block_hadamard``  -- H_G = kron^(log4 G)(H4) / sqrt(G)   (_int4/eager.py:20-46)
* ``rotate``          -- x_g @ H in x's dtype                  (_int4/eager.py:49-79)
* ``quantize_rows``   -- rowwise absmax / 7, round half to even, clamp +-7
                         (_int4/eager.py:104-120)
* ``pack`` / ``unpack`` -- two nibbles per byte, even k low    (_int4/_codec.py:19-36)
* ``int4_linear``     -- codes as out_dtype, matmul, * xs, * ws, + bias, each
                         rounded in out_dtype                  (_int4/eager.py:154-169)
* ``linear``          -- the whole eager linear                (_int4/eager.py:172-197)
"""
from __future__ import annotations

import math
import time

import torch

# the regular 4 x 4 Hadamard factor of the reference (_int4/eager.py:32-36)
_H4 = ((1, 1, 1, -1), (1, 1, -1, 1), (1, -1, 1, 1), (-1, 1, 1, 1))
QMAX = 7


def block_hadamard(G: int, dtype: torch.dtype) -> torch.Tensor:
    """The normalised block factor; every entry is +-1/sqrt(G), exact in bf16/f16."""
    levels = round(math.log(G, 4))
    if 4 ** levels != G:
        raise ValueError(f"block size must be a power of 4, got {G}")
    base = torch.tensor(_H4, dtype=torch.float64)
    h = base
    for _ in range(levels - 1):
        h = torch.kron(h, base)
    return (h / math.sqrt(G)).to(dtype)


def rotate(x: torch.Tensor, G: int) -> torch.Tensor:
    """Each G-block of every row times H_G, one torch matmul in x's dtype."""
    rows, k = x.shape
    h = block_hadamard(G, x.dtype)
    return torch.matmul(x.reshape(rows, k // G, G), h).reshape(rows, k)


def pack(codes: torch.Tensor) -> torch.Tensor:
    """int8 codes [..., K] -> int8 [..., K/2]: element 2j in bits 0-3, 2j+1 in bits 4-7."""
    c = codes.to(torch.int16)
    return ((c[..., 1::2] << 4) | (c[..., 0::2] & 15)).to(torch.int8)


def unpack(packed: torch.Tensor) -> torch.Tensor:
    """Inverse of pack with signed nibbles in [-8, 7] (arithmetic shifts)."""
    p = packed.to(torch.int16)
    lo, hi = (p << 12) >> 12, (p << 8) >> 12
    return torch.stack((lo, hi), dim=-1).reshape(*packed.shape[:-1], -1).to(torch.int8)


def quantize_rows(xr: torch.Tensor):
    """Symmetric rowwise int4: scale = max(absmax, 1e-10) / 7 and codes
    round(xr / scale) clamped to +-7, all in xr's dtype.  Returns (packed int8
    [rows, K/2], f32 scales [rows])."""
    scale = xr.abs().amax(dim=-1, keepdim=True).clamp(min=1e-10) / QMAX
    codes = torch.round(xr / scale).clamp(-QMAX, QMAX).to(torch.int8)
    return pack(codes), scale.reshape(-1).to(torch.float32)


def quantize_weight(w: torch.Tensor, G: int):
    """The load-time weight quantization (round mode), in w's dtype (fp16 for
    the reference's loader)."""
    return quantize_rows(rotate(w, G))


def int4_linear(qx, qw, xs, ws, bias, out_dtype):
    """Integer codes as out_dtype through one matmul, then * xs, * ws, + bias,
    each rounded in out_dtype."""
    y = unpack(qx).to(out_dtype) @ unpack(qw).to(out_dtype).t()
    y = y * xs.reshape(-1, 1).to(out_dtype)
    y = y * ws.reshape(1, -1).to(out_dtype)
    if bias is not None:
        y = y + bias.reshape(1, -1).to(out_dtype)
    return y


def linear(x, qw, ws, bias=None, G=256, stage_seconds=None):
    """The whole eager linear on x [M, K] (codes of the weight from
    quantize_weight).  With a dict ``stage_seconds`` it adds the time of the
    rotation, the quantize+pack and the int GEMM + epilogue."""
    t0 = time.perf_counter()
    xr = rotate(x, G)
    t1 = time.perf_counter()
    qx, xs = quantize_rows(xr)
    t2 = time.perf_counter()
    y = int4_linear(qx, qw, xs, ws, bias, x.dtype)
    t3 = time.perf_counter()
    if stage_seconds is not None:
        for k, dt in (("rotate", t1 - t0), ("quantize_pack", t2 - t1), ("gemm_epilogue", t3 - t2)):
            stage_seconds[k] = stage_seconds.get(k, 0.0) + dt
    return y
