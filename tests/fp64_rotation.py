"""CPU restatement of the rotate+quantize kernel's own fp64 rotation (test
infrastructure, numpy).

The oracle rotates exactly and rounds once.  The kernel (csrc/rotquant.hip,
rotate_chunk / h4_stage / jam_to_f32) runs the butterflies in fp64, which is
exact while a group's nonzero inputs span at most 36 binades (bf16, G = 256)
and rounds partial sums beyond that.  This module repeats the kernel's
arithmetic operation for operation, so that its results on wide-span groups
can be checked bit for bit:

  * a group's index is split into base-4 digits d0 (lowest) .. d3; radix-4
    stages run over d0, d1, d2, d3 in that order (G = 256; G = 64: d0..d2;
    G = 16: d0, d1);
  * a stage maps (a, b, c, d) at digit values 0..3 to
    S = ((a + b) + (c + d)) * scale, then S - 2*scale*d, S - 2*scale*c,
    S - 2*scale*b, S - 2*scale*a, each one fp64 rounding (the product with a
    power of two is exact, the kernel fuses it into one fma); scale is 1
    except in the last stage, 1/sqrt(G);
  * the fp64 result is rounded once to the input type: bf16 through a jam (its
    low word replaced by the float bits of the low word read as an unsigned
    integer, nonzero iff the low word is), an exact conversion to f32 and a
    round to nearest even; f16 through a jam of the low word into bit 32, the
    exact conversion to f32 and a round to nearest even; f32 directly.

On groups of narrower span it equals the exact rotation (tests/test_wide_span.py
checks that for all three input types)."""
import numpy as np
import torch

_SCALE = {16: 0.25, 64: 0.125, 256: 1.0 / 16.0}
_DIGITS = {16: 2, 64: 3, 256: 4}


def _stage(v: np.ndarray, axis: int, scale: float) -> np.ndarray:
    a, b, c, d = (np.take(v, i, axis=axis) for i in range(4))
    S = (a + b) + (c + d)
    if scale != 1.0:
        S = S * scale
    t = -2.0 * scale
    return np.stack([S + t * d, S + t * c, S + t * b, S + t * a], axis=axis)


F32, BF16, F16 = 0, 1, 2


def rotate_fp64_kernel_order(x: np.ndarray, G: int, dt: int = BF16) -> np.ndarray:
    """x [M, K] (float32 values for F32, uint16 bits for BF16 / F16) -> the
    kernel's fp64 rotation rounded to the input type, in the same form."""
    M, K = x.shape
    n = _DIGITS[G]
    if dt == F32:
        x = x.astype(np.float32).astype(np.float64)
    elif dt == F16:
        x = x.astype(np.uint16).view(np.float16).astype(np.float64)
    else:
        x = torch.from_numpy(x.astype(np.uint16).view(np.int16)).view(torch.bfloat16).double().numpy()
    # index = d0 + 4 d1 + 16 d2 + 64 d3: axis -1 is d0, axis -2 d1, ...
    v = x.reshape((M, K // G) + (4,) * n)
    for s in range(n):
        v = _stage(v, axis=v.ndim - 1 - s, scale=_SCALE[G] if s == n - 1 else 1.0)
    y = np.ascontiguousarray(v.reshape(M, K))
    if dt == F32:
        return y.astype(np.float32)
    u = y.view(np.uint64)
    if dt == F16:
        hi = (u >> np.uint64(32)) | ((u & np.uint64(0xffffffff)) != 0).astype(np.uint64)
        return (hi << np.uint64(32)).view(np.float64).astype(np.float32).astype(np.float16).view(np.uint16)
    lo = (u & np.uint64(0xffffffff)).astype(np.uint32).astype(np.float32).view(np.uint32).astype(np.uint64)
    f = ((u & np.uint64(0xffffffff00000000)) | lo).view(np.float64).astype(np.float32)
    return torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
