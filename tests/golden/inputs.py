"""Seeded synthetic inputs shared by the golden generator, the tests and bench.py.

Everything is drawn with ``numpy.random.RandomState`` (stable across numpy
versions) and converted to bf16 / fp16 with torch's round-to-nearest-even
casts, so a fixture's inputs can be regenerated anywhere from the seed alone.
"""
from __future__ import annotations

import numpy as np
import torch


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def outlier_activations(M: int, K: int, seed: int = 0, scale: float = 20.0, frac: float = 0.01,
                        student_t: bool = False, dtype=torch.bfloat16) -> torch.Tensor:
    """x ~ N(0,1) with round(frac*K) outlier channels.

    ``student_t=False``: the outlier channels are multiplied by ``scale``
    (the DiT-linear configuration).  ``student_t=True``: they are replaced by
    Student-t(nu=3) draws (the heavy-tailed rotate+quant configuration).
    """
    rs = np.random.RandomState(seed)
    x = rs.standard_normal((M, K)).astype(np.float32)
    nout = int(round(frac * K))
    ch = rs.choice(K, size=nout, replace=False)
    if student_t:
        x[:, ch] = rs.standard_t(3, size=(M, nout)).astype(np.float32)
    else:
        x[:, ch] *= scale
    return torch.from_numpy(x).to(dtype)


def normal_weight(N: int, K: int, seed: int = 1, std: float = 0.02, dtype=torch.float16) -> torch.Tensor:
    rs = np.random.RandomState(seed)
    return torch.from_numpy((rs.standard_normal((N, K)) * std).astype(np.float32)).to(dtype)


def normal_bias(N: int, seed: int = 2, std: float = 0.01, dtype=torch.float16) -> torch.Tensor:
    rs = np.random.RandomState(seed)
    return torch.from_numpy((rs.standard_normal((N,)) * std).astype(np.float32)).to(dtype)


def config1_x() -> torch.Tensor:
    """x bf16 [256, 3072], N(0,1), 1% of channels x20, seed 0."""
    return outlier_activations(256, 3072, seed=0)


def config1_weight() -> torch.Tensor:
    """W [3072, 3072] ~ N(0, 0.02) cast to fp16 (weights are quantized from fp16)."""
    return normal_weight(3072, 3072, seed=1)


def config1_bias() -> torch.Tensor:
    return normal_bias(3072, seed=2)


def hadamard_np(G: int) -> np.ndarray:
    h4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float64)
    h = h4
    while h.shape[0] < G:
        h = np.kron(h, h4)
    return h / np.sqrt(G)


def preimage_rows(v: np.ndarray, G: int) -> np.ndarray:
    """x = v @ H (float64); rotating x returns v exactly when x is representable."""
    H = hadamard_np(G)
    M, K = v.shape
    return (v.reshape(M, K // G, G) @ H).reshape(M, K)


def tie_rows(K: int = 256) -> torch.Tensor:
    """bf16 rows whose exact rotation hits quantizer ties (x/s = k + 1/2)."""
    G = 256
    rows = []
    # row 0: absmax 7 -> s = 1, values at every half-integer tie
    v = np.zeros(K)
    v[0] = 7.0
    ties = [0.5, 1.5, 2.5, 3.5, 4.5, 5.5, 6.5]
    for i, t in enumerate(ties):
        v[1 + 2 * i] = t
        v[2 + 2 * i] = -t
    rows.append(v)
    # row 1: absmax 3.5 -> s = 0.5, ties at (k+1/2)*0.5
    v = np.zeros(K)
    v[5] = 3.5
    for i, t in enumerate(ties):
        v[20 + i] = t * 0.5
        v[40 + i] = -t * 0.5
    rows.append(v)
    v = np.stack(rows)
    x = preimage_rows(v, G)
    xt = torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16)
    if not np.array_equal(xt.float().numpy().astype(np.float64), x):
        raise AssertionError("tie preimage not representable in bf16")
    return xt


def edge_cases() -> dict:
    """name -> (x tensor [M,K], convrot groupsize)."""
    cases = {}
    rs = np.random.RandomState(7)
    # zero row, single nonzero, tiny row (hits the 1e-10 clamp), normal row
    z = np.zeros((4, 256), dtype=np.float32)
    z[1, 17] = 3.0
    z[2, :] = rs.standard_normal(256).astype(np.float32) * 1e-12
    z[3, :] = rs.standard_normal(256).astype(np.float32)
    cases["zeros"] = (torch.from_numpy(z).to(torch.bfloat16), 256)
    cases["ties"] = (tie_rows(), 256)
    cases["g16"] = (torch.from_numpy(rs.standard_normal((8, 80)).astype(np.float32)).to(torch.bfloat16), 16)
    cases["g64"] = (torch.from_numpy(rs.standard_normal((8, 192)).astype(np.float32)).to(torch.bfloat16), 64)
    cases["f32"] = (torch.from_numpy(rs.standard_normal((8, 512)).astype(np.float32)), 256)
    cases["f16"] = (torch.from_numpy(rs.standard_normal((8, 512)).astype(np.float32)).to(torch.float16), 256)
    w = rs.standard_normal((4, 256)).astype(np.float32)
    w[:, ::7] *= 1e-30                                  # >100 binades inside one group
    w[:, 3] = 1e3
    cases["wide_span"] = (torch.from_numpy(w).to(torch.bfloat16), 256)
    cases["student_t"] = (outlier_activations(16, 1024, seed=3, student_t=True), 256)
    return cases


def tie_rows8(K: int = 256) -> torch.Tensor:
    """bf16 rows for the int8 quantizer itself (already-rotated values):
    half-integer quotients (ties to even) and scales that are not powers of
    two.  (No input reaches the clamp: s = RNE(a/127) is within 2^-9 of a/127,
    so every quotient rounds to at most 127.)"""
    rows = []
    v = np.zeros(K)                        # absmax 127 -> s = 1
    v[0] = 127.0
    ties = [0.5, 1.5, 2.5, 3.5, 64.5, 125.5, 126.5]
    for i, t in enumerate(ties):
        v[1 + 2 * i] = t
        v[2 + 2 * i] = -t
    rows.append(v)
    v = np.zeros(K)                        # absmax 127.5 -> s = bf16(127.5/127) = 1.0078125: 127.5/s = 126.5 ties to 126
    v[3] = 127.5
    v[4] = -127.5
    v[5] = 63.5
    rows.append(v)
    v = np.zeros(K)                        # absmax 254 -> s = 2: ties at odd integers
    v[7] = -254.0
    for i, t in enumerate([1.0, 3.0, 5.0, 7.0, 251.0, 253.0]):
        v[10 + i] = t
        v[20 + i] = -t
    rows.append(v)
    rs = np.random.RandomState(17)         # generic scale (absmax 100)
    v = rs.uniform(-100.0, 100.0, K)
    v[0] = 100.0
    rows.append(v)
    return torch.from_numpy(np.stack(rows).astype(np.float32)).to(torch.bfloat16)


def clamp_rows8() -> torch.Tensor:
    """bf16 x [2, 16] (G = 16) whose exact rotation is +-127.5 e_0, the largest
    bf16 absmax below 128: s = bf16(127.5/127) = 1.0078125 and the quotient
    127.5/s = 126.5 is a tie that rounds to 126."""
    v = np.zeros((2, 16))
    v[0, 0] = 127.5
    v[1, 0] = -127.5
    x = preimage_rows(v, 16)
    xt = torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16)
    if not np.array_equal(xt.float().numpy().astype(np.float64), x):
        raise AssertionError("preimage not representable in bf16")
    return xt


def small_w8a8_case():
    """x bf16 [64, 512], W fp16 [96, 512] ~ N(0, 0.02), bias fp16 [96]: K small
    enough that every fp32 partial sum of the int8 product is exact (< 2^24)."""
    x = outlier_activations(64, 512, seed=21)
    w = normal_weight(96, 512, seed=22)
    b = normal_bias(96, seed=23)
    return x, w, b


def stochastic_weight_case() -> torch.Tensor:
    return normal_weight(64, 512, seed=11)


def small_linear_case():
    """Random packed codes over all byte values (nibble -8 included), scales U(0.005,0.05)."""
    rs = np.random.RandomState(5)
    M, N, K = 64, 48, 256
    xp = torch.from_numpy(rs.randint(-128, 128, size=(M, K // 2)).astype(np.int8))
    wp = torch.from_numpy(rs.randint(-128, 128, size=(N, K // 2)).astype(np.int8))
    xs = torch.from_numpy(rs.uniform(0.005, 0.05, size=M).astype(np.float32))
    ws = torch.from_numpy(rs.uniform(0.005, 0.05, size=N).astype(np.float32))
    bias = torch.from_numpy((rs.standard_normal(N) * 0.01).astype(np.float32)).to(torch.float16)
    return xp, wp, xs, ws, bias


def wide_span_rows(M, K, G, seed, kind):
    """bf16 rows whose convrot groups span far more than the 36 binades inside
    which every fp64 partial sum of the rotation is exact.
      "mixed": N(0,1) values with a random fifth scaled by 2^-e, e uniform in
        [20, 140] (down to bf16 subnormals and underflow to zero);
      "pairs": values of 2^-30 .. 2^-90 and, per group, one value of 1 .. 16
        at two positions, so that half of the group's outputs cancel it after
        fp64 partial sums have added the small values to it;
      "ties": even integers of magnitude <= 256, whose rotated sums often fall
        exactly on a bf16 rounding midpoint, and a tenth of the values
        replaced by ones of 2^-40 .. 2^-100 that decide those ties."""
    rs = np.random.RandomState(seed)
    if kind == "ties":
        x = 2.0 * rs.randint(-128, 129, size=(M, K))
        tiny = rs.rand(M, K) < 0.1
        x = np.where(tiny, rs.standard_normal((M, K)) * np.exp2(-rs.randint(40, 101, size=(M, K)).astype(np.float64)), x)
        return torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16)
    if kind == "mixed":
        x = rs.standard_normal((M, K))
        tiny = rs.rand(M, K) < 0.2
        x = np.where(tiny, x * np.exp2(-rs.randint(20, 141, size=(M, K)).astype(np.float64)), x)
    else:
        x = rs.standard_normal((M, K)) * np.exp2(-rs.randint(30, 91, size=(M, K)).astype(np.float64))
    for g in range(K // G):
        a, b = g * G + rs.choice(G, 2, replace=False)
        x[:, b] = x[:, a] = rs.choice([-1.0, 1.0], size=M) * 2.0 ** rs.randint(0, 5)
    return torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16)


def wide_span_rows_typed(M, K, G, seed, kind, dtype):
    """The wide-span kinds of wide_span_rows for f32 (24-bit significands: fp64
    partial sums of a group are exact only within a 20-binade span) and f16
    (every value a multiple of 2^-24 below 2^16, so a group's sums are
    multiples of 2^-24 below 2^48 and fp64 holds them all exactly: these rows
    reach the type's whole range, subnormals included).
      "mixed": N(0,1) (f16: x4) with a fifth of the values scaled down by
        2^-20 .. 2^-140 (f16: 2^-8 .. 2^-26, subnormals and underflow);
      "pairs": small values and, per group, one large value at two positions;
      "ties": integers of up to 24 (f16: 11) bits, whose rotated sums often
        fall exactly on a rounding midpoint, and a tenth of the values tiny."""
    rs = np.random.RandomState(seed)
    f16 = dtype == torch.float16
    if kind == "ties":
        hi = 2 ** 10 if f16 else 2 ** 23
        x = rs.randint(-hi, hi + 1, size=(M, K)).astype(np.float64)
        lo = (12, 25) if f16 else (30, 120)
        tiny = rs.rand(M, K) < 0.1
        x = np.where(tiny, rs.standard_normal((M, K)) * np.exp2(-rs.randint(*lo, size=(M, K)).astype(np.float64)), x)
        return torch.from_numpy(x).to(dtype)
    if kind == "mixed":
        x = rs.standard_normal((M, K)) * (4.0 if f16 else 1.0)
        lo = (8, 27) if f16 else (20, 141)
        tiny = rs.rand(M, K) < 0.2
        x = np.where(tiny, x * np.exp2(-rs.randint(*lo, size=(M, K)).astype(np.float64)), x)
    else:
        lo = (10, 25) if f16 else (30, 91)
        x = rs.standard_normal((M, K)) * np.exp2(-rs.randint(*lo, size=(M, K)).astype(np.float64))
    big = (2.0 ** 11, 2.0 ** 12) if f16 else (1.0, 16.0)
    for g in range(K // G):
        a, b = g * G + rs.choice(G, 2, replace=False)
        x[:, b] = x[:, a] = rs.choice([-1.0, 1.0], size=M) * rs.choice(big)
    return torch.from_numpy(x).to(dtype)


# (kind, M, K, G) of the wide-span golden vectors
WIDE_SPAN_CASES = [("mixed", 16, 3072, 256), ("pairs", 16, 3072, 256), ("ties", 16, 3072, 256),
                   ("ties", 16, 3072, 64), ("ties", 16, 1024, 16), ("mixed", 16, 1024, 16)]
