"""W4A4 weight helpers under the module name the reference's sensitivity node
imports them from (``_int4.eager``: int4_sensitivity.py:43-46, which scores a
layer by quantizing its fp16 weight and dequantizing it back).

Despite the name, nothing here is the reference's torch eager path: the
quantizer is the package's gfx950 kernel (the exactly rounded block-Hadamard
rotation in the weight's dtype, then the eager quantizer's arithmetic,
reference _int4/eager.py:123-135), and the linear is the package's W4A4 linear
with the eager bf16 rounding chain as its epilogue (reference
_int4/eager.py:154-197).  Only the load-time dequantization helper is torch
code (fp32, reference _int4/eager.py:138-151).
"""
from __future__ import annotations

import torch

from . import (
    _INT4_GROUP_SIZE,
    convrot_w4a4_linear as _gpu_linear,
    dequantize_convrot_w4a4_weight,
    quantize_convrot_w4a4_weight,
    validate_w4a4_shape,
)

__all__ = [
    "quantize_convrot_w4a4_weight",
    "dequantize_convrot_w4a4_weight",
    "validate_w4a4_shape",
    "convrot_w4a4_linear",
]


def convrot_w4a4_linear(
    x: torch.Tensor,
    qweight: torch.Tensor,
    wscales: torch.Tensor,
    bias: torch.Tensor | None = None,
    convrot_groupsize: int = 256,
    quant_group_size: int = _INT4_GROUP_SIZE,
    linear_dtype: str = "int4",
) -> torch.Tensor:
    """``x @ W.T + bias`` with the reference eager path's output rounding
    (reference _int4/eager.py:172-197): for bf16 x each of acc, *xs, *ws and
    +bias is rounded to bf16 in turn, which the gfx950 linear reproduces bit
    for bit.  f32 x gets the fp32 chain (the same arithmetic); f16 x the fp32
    epilogue rounded once to f16.  ``linear_dtype`` is validated as the
    reference does and changes nothing else (the eager path ignores it too)."""
    if linear_dtype not in {"int4", "int8"}:
        raise ValueError(f"ConvRot W4A4 linear_dtype must be 'int4' or 'int8', got {linear_dtype!r}")
    return _gpu_linear(x, qweight, wscales, bias, convrot_groupsize, quant_group_size, linear_dtype="int8")
