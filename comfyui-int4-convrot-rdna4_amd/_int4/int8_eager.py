"""W8A8 (int8) tier of the ConvRot backend, under the module name the
reference's loader, Save and sensitivity nodes import it from
(``_int4.int8_eager``: int4_ops.py:340, int4_sensitivity.py:67-70,98).  Despite
the name, quantization runs on the gfx950 kernels; only the load-time
dequantization helper is torch code.

Numerics: those of the reference eager path (reference _int4/int8_eager.py):
the exactly rounded block-Hadamard rotation in the input dtype, then
s = dt(fl32(absmax / 127)), q = clamp(rint_even(dt(fl32(x / s))), -127, 127),
stored as plain int8 [rows, K] with f32 scales.
"""
from __future__ import annotations

import torch

from . import _check_groupsize, _check_width, _hadamard, _on_gpu, convrot_w8a8_linear, native

__all__ = ["quantize_convrot_w8a8_weight", "dequantize_convrot_w8a8_weight", "convrot_w8a8_linear"]


def quantize_convrot_w8a8_weight(
    weight: torch.Tensor,
    convrot_groupsize: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Rotate a weight with ConvRot and quantize it to signed int8 per row
    (reference _int4/int8_eager.py:31-47).  Runs the fused kernel in the
    weight's dtype (the loader passes fp16, int4_ops.py:339-342).  Returns
    (qweight int8 [N, K], scale f32 [N]) on the weight's device."""
    if weight.dim() != 2:
        raise ValueError(f"ConvRot W8A8 expects a 2D tensor, got {tuple(weight.shape)}")
    if weight.shape[-1] % convrot_groupsize != 0:
        raise ValueError(f"in_features {weight.shape[-1]} not divisible by "
                         f"convrot_groupsize {convrot_groupsize}")
    _check_groupsize(convrot_groupsize)
    _check_width(weight.shape[-1])
    dev = weight.device
    w = _on_gpu(weight).contiguous()
    if w.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        w = w.to(torch.float32)
    q, s = native.convrot_quant_int8(w, convrot_groupsize)
    return q.to(dev), s.to(dev)


def dequantize_convrot_w8a8_weight(
    qdata: torch.Tensor,
    scales: torch.Tensor,
    convrot_groupsize: int,
    output_dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """Dequantize int8 ConvRot weights and rotate back to the original basis
    (reference _int4/int8_eager.py:50-57).  A load-time / diagnostic helper,
    computed with torch ops in fp32."""
    w = qdata.to(torch.float32) * scales.to(qdata.device, torch.float32).reshape(-1, 1)
    N, K = w.shape
    G = convrot_groupsize
    h = _hadamard(G, qdata.device)
    return torch.matmul(w.reshape(N, K // G, G), h.T).reshape(N, K).to(output_dtype)
