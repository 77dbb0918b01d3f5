"""Signed-int4 nibble codec and quantizer constants.

The packed layout is the reference's (``_int4/_codec.py:12-36``) and must stay
byte-identical so existing checkpoints load: int8 [..., K/2], element 2j in the
low nibble of byte j, element 2j+1 in the high nibble; codes are produced in
[-7, 7] (scale = absmax / 7) and read back as signed nibbles in [-8, 7].
"""
from __future__ import annotations

import torch

# quant_group_size accepted by the API (a divisibility requirement on K; the
# scales are per row), reference _int4/_codec.py:15
_INT4_GROUP_SIZE = 64
# symmetric code range [-7, 7], reference _int4/_codec.py:16
_INT4_MAX = 7


def _pack_int4_row_major(values: torch.Tensor) -> torch.Tensor:
    """(..., K) codes -> (..., K // 2) int8 with the even column in the low nibble."""
    if values.shape[-1] % 2 != 0:
        raise ValueError(f"last dim must be even, got {values.shape[-1]}")
    v = values.to(torch.int32) & 0x0F
    return (v[..., 0::2] | (v[..., 1::2] << 4)).to(torch.int8)


def _unpack_int4_row_major(packed: torch.Tensor) -> torch.Tensor:
    """(..., K // 2) int8 -> (..., K) int8 codes in [-8, 7] (signed nibbles)."""
    b = packed.to(torch.int32)
    # shift each nibble to the top of an int32 and shift back arithmetically
    lo = (b << 28) >> 28
    hi = (b << 24) >> 28
    return torch.stack([lo, hi], dim=-1).reshape(*packed.shape[:-1], -1).to(torch.int8)
