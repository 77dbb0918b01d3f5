"""int4 ConvRot W4A4 backend for AMD MI355X (gfx950 / CDNA4).

Drop-in for the reference backend package ``_int4`` (reference
``_int4/__init__.py:9-13,35-42``): same public names, signatures, dtypes and
exceptions, with every stage of the linear running in hand-written gfx950 HIP
kernels (``csrc/``) reached through the C-ABI in ``native.py``.

Public API:
    quantize_convrot_w4a4_weight(weight, convrot_groupsize, ...) -> (qweight_i8, scale_f32)
    dequantize_convrot_w4a4_weight(qdata, scales, convrot_groupsize, ...) -> tensor
    convrot_w4a4_linear(x, qweight, wscales, bias, convrot_groupsize, ...) -> tensor
    is_available() -> bool          # gfx950 ROCm device + loadable kernel library
    pick_groupsize(in_features) -> int | None

Numerics are those of the reference eager path (``_int4/eager.py``): packed
codes and scales equal the eager ones, the integer accumulators are exact, and
the epilogue is the fp32 chain fl32(fl32(fl32(acc*xs)*ws)+b) rounded once to
the output dtype.
"""
from __future__ import annotations

import math

import torch

from . import native
from ._codec import _INT4_GROUP_SIZE, _INT4_MAX, _pack_int4_row_major, _unpack_int4_row_major
from .native import is_available as _native_available

__all__ = [
    "quantize_convrot_w4a4_weight",
    "dequantize_convrot_w4a4_weight",
    "convrot_w4a4_linear",
    "convrot_w8a8_linear",
    "is_available",
    "pick_groupsize",
    "fuse_lora_pairs",
    "MAX_LORA_RANK",
    "prepare_convrot_w4a4_weight_bf6",
    "bf6_path_ok",
    "i8t_path_ok",
    "prepare_convrot_w8a8_weight_i8t",
    "max_quant_k",
]

# largest concatenated rank of the fused LoRA side path (padded to a multiple of 32)
MAX_LORA_RANK = 128

# dtypes the GEMM emits natively; others compute in fp32 then cast
# (reference _int4/__init__.py:45)
_NATIVE_OUT = frozenset({torch.float32, torch.bfloat16})


def pick_groupsize(in_features: int) -> int | None:
    """Largest supported ConvRot groupsize dividing in_features (256/64/16)
    (reference _int4/__init__.py:69-74)."""
    for g in (256, 64, 16):
        if in_features % g == 0:
            return g
    return None


def is_available() -> bool:
    """True only on a gfx950 ROCm device with a loadable kernel library."""
    return _native_available()


def _check_groupsize(G: int) -> None:
    if G < 4 or (G & (G - 1)) != 0 or math.log(G, 4) % 1 != 0:
        raise ValueError(f"Regular Hadamard size must be a power of 4, got {G}")
    if G not in (16, 64, 256):
        raise ValueError(f"convrot_groupsize must be 16, 64 or 256, got {G}")


def validate_w4a4_shape(tensor: torch.Tensor, convrot_groupsize: int, quant_group_size: int) -> None:
    """reference _int4/eager.py:82-89"""
    if tensor.dim() != 2:
        raise ValueError(f"ConvRot W4A4 expects a 2D tensor, got shape {tuple(tensor.shape)}")
    k = tensor.shape[-1]
    if k % convrot_groupsize != 0:
        raise ValueError(f"in_features {k} not divisible by convrot_groupsize {convrot_groupsize}")
    if k % quant_group_size != 0:
        raise ValueError(f"in_features {k} not divisible by quant_group_size {quant_group_size}")


def max_quant_k() -> int:
    """Widest row (in_features) the fused rotate+quantize kernels take: 32768."""
    return native.max_quant_k()


def _check_width(k: int) -> None:
    """Rows wider than the fused kernels take raise here, with the reason, so a
    loader that catches the error keeps the layer in bf16 (the reference's
    dispatcher instead rotates such rows with torch, _int4/__init__.py:59-66)."""
    cap = max_quant_k()
    if k > cap:
        raise ValueError(f"in_features {k} exceeds {cap}, the widest row the gfx950 rotate+quantize kernels take")


def _on_gpu(t: torch.Tensor) -> torch.Tensor:
    if t.is_cuda:
        return t
    if not torch.cuda.is_available():
        raise RuntimeError("the ConvRot int4 kernels need a gfx950 GPU; none is visible")
    return t.to("cuda")


def quantize_convrot_w4a4_weight(
    weight: torch.Tensor,
    convrot_groupsize: int = 256,
    quant_group_size: int = _INT4_GROUP_SIZE,
    stochastic_rounding: int | None = 0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Rotate a weight with ConvRot and pack it as signed W4 (reference
    _int4/eager.py:123-135).  Runs the fused gfx950 kernel in the weight's
    dtype (the loader passes fp16, int4_ops.py:344-350).  Returns tensors on
    the weight's device.

    stochastic_rounding > 0 draws the rounding noise exactly as the reference
    does (torch.rand with a generator seeded on the weight's device,
    _int4/eager.py:92-101) and rounds with floor(t + u).
    """
    if quant_group_size != _INT4_GROUP_SIZE:
        raise ValueError(f"int4 MMA kernel requires quant_group_size {_INT4_GROUP_SIZE}")
    validate_w4a4_shape(weight, convrot_groupsize, quant_group_size)
    _check_groupsize(convrot_groupsize)
    _check_width(weight.shape[-1])
    dev = weight.device
    w = _on_gpu(weight).contiguous()
    if w.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        w = w.to(torch.float32)
    if stochastic_rounding is not None and stochastic_rounding > 0:
        gen = torch.Generator(device=weight.device)
        gen.manual_seed(stochastic_rounding)
        noise = torch.rand(weight.shape, dtype=w.dtype, layout=weight.layout, device=weight.device,
                           generator=gen)
        q, s = native.convrot_quant_int4_stochastic(w, convrot_groupsize, _on_gpu(noise))
    else:
        q, s = native.convrot_quant_int4(w, convrot_groupsize)
    return q.to(dev), s.to(dev)


def _hadamard(G: int, device, dtype=torch.float32) -> torch.Tensor:
    """H_G = kron^(log4 G)(H4)/sqrt(G) (reference _int4/eager.py:20-46)."""
    h4 = torch.tensor([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]],
                      dtype=dtype, device=device)
    h = h4
    while h.shape[0] < G:
        h = torch.kron(h, h4)
    return h / (G ** 0.5)


def dequantize_convrot_w4a4_weight(
    qdata: torch.Tensor,
    scales: torch.Tensor,
    convrot_groupsize: int = 256,
    quant_group_size: int = _INT4_GROUP_SIZE,
    output_dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """Dequantize packed ConvRot W4A4 weights and rotate back to the original
    basis (reference _int4/eager.py:138-151).  A load-time / diagnostic helper,
    not on the forward path; computed with torch ops in fp32."""
    if quant_group_size != _INT4_GROUP_SIZE:
        raise ValueError(f"int4 MMA kernel requires quant_group_size {_INT4_GROUP_SIZE}")
    w = _unpack_int4_row_major(qdata).to(torch.float32)
    w = w * scales.to(device=qdata.device, dtype=torch.float32).reshape(-1, 1)
    N, K = w.shape
    G = convrot_groupsize
    h = _hadamard(G, qdata.device)
    return torch.matmul(w.reshape(N, K // G, G), h.T).reshape(N, K).to(output_dtype)


def bf6_path_ok(in_features: int) -> bool:
    """True when a linear of this input width runs on the bf6 matrix-core GEMM
    (K % 128 == 0 and the fused quantizer covers K); others use the int8 GEMM."""
    return in_features % 128 == 0 and in_features <= native.max_quant_bf6_k()


def i8t_path_ok(in_features: int) -> bool:
    """True when a W8A8 linear of this input width runs on the tile-major (I8T)
    int8 GEMM (K % 64 == 0 and the fused quantizer covers K); others use the
    row-major int8 GEMM."""
    return in_features % 64 == 0 and in_features <= native.max_quant_bf6_k()


def prepare_convrot_w8a8_weight_i8t(qweight: torch.Tensor) -> torch.Tensor | None:
    """Load-time re-layout of an int8 weight [N, K] into the I8T operand layout
    of the W8A8 GEMM (int8 [ceil(N/256)*256, K], the same codes).  Returns None
    when the weight's K cannot use that path."""
    if not i8t_path_ok(qweight.shape[-1]):
        return None
    return native.int8_to_i8t(_on_gpu(qweight).contiguous())


def prepare_convrot_w4a4_weight_bf6(qweight: torch.Tensor) -> torch.Tensor | None:
    """Load-time re-encoding of a packed int4 weight [N, K/2] into the B6T bf6
    operand layout of the fast GEMM (uint8 [ceil(N/256)*256, 3K/4], the same
    integer codes).  Returns None when the weight's K cannot use that path."""
    K = qweight.shape[-1] * 2
    if not bf6_path_ok(K):
        return None
    return native.int4_to_bf6(_on_gpu(qweight).contiguous())


def convrot_w4a4_linear(
    x: torch.Tensor,
    qweight: torch.Tensor,
    wscales: torch.Tensor,
    bias: torch.Tensor | None = None,
    convrot_groupsize: int = 256,
    quant_group_size: int = _INT4_GROUP_SIZE,
    linear_dtype: str = "int4",
    *,
    lora: tuple[torch.Tensor, torch.Tensor] | None = None,
    qweight_bf6: torch.Tensor | None = None,
) -> torch.Tensor:
    """Compute ``x @ W.T + bias`` with the gfx950 W4A4 ConvRot path
    (reference _int4/__init__.py:94-138).

    ``lora=(D, U)`` (from :func:`fuse_lora_pairs`) adds the dynamic-LoRA term
    ``(x @ D.T) @ U.T`` inside the GEMM epilogue (one extra kernel for the
    down projection), the fused form of the per-adapter side path of the
    reference's Linear (int4_ops.py:181-192).

    ``qweight_bf6`` (from :func:`prepare_convrot_w4a4_weight_bf6`, made once
    at load time) selects the bf6 matrix-core GEMM: the activation is
    quantized straight into the bf6 operand layout and the integer products
    run on v_mfma_scale_f32_32x32x64_f8f6f4, whose fp32 accumulation of these
    small integers is exact, so the output is bit-identical to the int8-MFMA
    GEMM's.  Without it, inputs whose K allows it still take the bf6 GEMM with
    the weight re-encoded on the fly.

    Two kernels per call, both on torch's current stream: the fused
    rotate+quantize of x, then the W4A4 GEMM with the dequant epilogue.  Every
    row count takes the same kernels (the reference's torch-rotation branch
    for M < 512 is not needed: the fused kernel is exact and fast at any M).

    linear_dtype "int8" marks layers the reference sends to its eager path
    (_int4/__init__.py:104-111 -> _int4/eager.py:172-197), whose output is the
    eager rounding chain in x's dtype.  Here the same kernels run with that
    chain as the epilogue: for bf16 x each of acc, *xs, *ws, +bias (and the
    LoRA term) is rounded to bf16 in turn (_int4/eager.py:162-168); for f32 x
    the eager chain and the default fp32 epilogue are the same arithmetic.  For
    f16 x the output is the fp32 epilogue rounded once to f16 (the eager f16
    chain, which overflows once |acc| > 65504, is not reproduced).
    """
    if linear_dtype not in {"int4", "int8"}:
        raise ValueError(f"ConvRot W4A4 linear_dtype must be 'int4' or 'int8', got {linear_dtype!r}")
    if quant_group_size != _INT4_GROUP_SIZE:
        raise ValueError(f"int4 MMA kernel requires quant_group_size {_INT4_GROUP_SIZE}")
    if x.shape[-1] != qweight.shape[-1] * 2:
        raise ValueError(f"Input K={x.shape[-1]} does not match qweight K={qweight.shape[-1] * 2}")
    if x.shape[-1] % convrot_groupsize != 0:
        raise ValueError(f"Input K={x.shape[-1]} not divisible by convrot_groupsize {convrot_groupsize}")
    _check_groupsize(convrot_groupsize)
    _check_width(x.shape[-1])

    orig_shape = x.shape
    x2d = x.reshape(-1, orig_shape[-1]).contiguous()
    if x2d.dtype not in native._IN_DTYPE_CODE:
        x2d = x2d.to(torch.float32)
    out_dtype = x.dtype if x.dtype in _NATIVE_OUT else torch.float32
    if out_dtype == torch.bfloat16:
        epi = native.EPI_BF16_EAGER if linear_dtype == "int8" else native.EPI_BF16
    else:
        epi = native.EPI_F32
    K, N = x2d.shape[1], qweight.shape[0]
    if lora is not None:
        down, up = lora
        if down.dim() != 2 or up.dim() != 2 or down.shape[1] != K or up.shape[0] != N \
                or up.shape[1] != down.shape[0]:
            raise ValueError(f"LoRA shapes D {tuple(down.shape)} U {tuple(up.shape)} do not fit K={K} N={N}")
        if down.dtype != torch.bfloat16 or up.dtype != torch.bfloat16:
            raise ValueError(f"LoRA D / U must be bf16, got {down.dtype} / {up.dtype}")
        if not (down.is_contiguous() and up.is_contiguous()):
            raise ValueError("LoRA D / U must be contiguous")
    if wscales.numel() != N:
        raise ValueError(f"wscales has {wscales.numel()} elements, the weight has N={N} rows")
    if bias is not None and bias.numel() != N:
        raise ValueError(f"bias has {bias.numel()} elements, the weight has N={N} rows")
    if bf6_path_ok(K) and x2d.is_cuda and (lora is None or x2d.dtype in (torch.bfloat16, torch.float16)):
        # the whole linear in one library call (same kernels, same bits as the steps below)
        w6 = qweight_bf6 if qweight_bf6 is not None else prepare_convrot_w4a4_weight_bf6(qweight)
        if w6.shape != (native.bf6_rows(N), K // 4 * 3):
            raise ValueError(f"qweight_bf6 of shape {tuple(w6.shape)} does not encode a [{N}, {K}] weight")
        wsc = wscales if wscales.dtype == torch.float32 and wscales.is_contiguous() else \
            wscales.reshape(-1).to(torch.float32).contiguous()
        # the bias is read as stored (f32 / bf16 / f16): no conversion launch per call
        b32 = None if bias is None else (bias.reshape(-1) if bias.dtype in native._IN_DTYPE_CODE else
                                         bias.reshape(-1).to(torch.float32))
        if b32 is not None and not b32.is_contiguous():
            b32 = b32.contiguous()
        down = up = None
        if lora is not None:
            down, up = lora
        native._check_cuda(x2d, w6, wsc, b32, down, up)
        out = native.convrot_w4a4_linear_bf6(native._aligned(x2d), w6, wsc, b32, down, up, 1.0, epi,
                                             convrot_groupsize, N)
        if out.dtype != x.dtype:
            out = out.to(x.dtype)
        return out.reshape(*orig_shape[:-1], N)
    t = up = None
    if lora is not None:
        down, up = lora
        xd = x2d if x2d.dtype in (torch.bfloat16, torch.float16) else x2d.to(torch.bfloat16)
        t = native.lora_down(xd, down)
    if bf6_path_ok(K):
        w6 = qweight_bf6 if qweight_bf6 is not None else prepare_convrot_w4a4_weight_bf6(qweight)
        if w6.shape != (native.bf6_rows(N), K // 4 * 3):
            raise ValueError(f"qweight_bf6 of shape {tuple(w6.shape)} does not encode a [{N}, {K}] weight")
        a6, x_scale = native.convrot_quant_bf6(x2d, convrot_groupsize)
        if t is None:
            out = native.int4_convrot_gemm_bf6(a6, w6, x_scale, wscales, bias, epi)
        else:
            out = native.int4_convrot_gemm_bf6_lora(a6, w6, x_scale, wscales, bias, t, up, 1.0, epi)
    else:
        qact, x_scale = native.convrot_quant_int4(x2d, convrot_groupsize)
        if t is None:
            out = native.int4_convrot_gemm_ex(qact, qweight, x_scale, wscales, bias, epi)
        else:
            out = native.int4_convrot_gemm_lora(qact, qweight, x_scale, wscales, bias, t, up, 1.0, epi)
    if out.dtype != x.dtype:
        out = out.to(x.dtype)
    return out.reshape(*orig_shape[:-1], qweight.shape[0])


def fuse_lora_pairs(pairs, device=None):
    """Concatenate plain LoRA adapters into the one (D, U) pair of the fused
    side path.

    ``pairs``: (down [r, K], up [N, r], scale) per adapter, where scale is the
    factor the adapter's bypass applies to up(down(x)), i.e. multiplier *
    alpha / r (reference int4_ops.py:181-192, "h() returns up(down(x)) already
    scaled by (alpha/rank)*strength").  The scale is folded into U (in fp32,
    then rounded once to bf16).  The total rank is padded with zero rows to a
    multiple of 32.  Returns (D bf16 [R, K], U bf16 [N, R]) on ``device`` (the
    first adapter's device by default), or None when R would exceed
    ``MAX_LORA_RANK``.
    """
    pairs = list(pairs)
    if not pairs:
        return None
    K = pairs[0][0].shape[1]
    N = pairs[0][1].shape[0]
    ranks = []
    for down, up, _ in pairs:
        if down.dim() != 2 or up.dim() != 2 or down.shape[1] != K or up.shape[0] != N \
                or up.shape[1] != down.shape[0]:
            raise ValueError(f"LoRA pair shapes down {tuple(down.shape)} up {tuple(up.shape)} "
                             f"do not fit K={K} N={N}")
        ranks.append(down.shape[0])
    R = -(-sum(ranks) // 32) * 32
    if R > MAX_LORA_RANK or R == 0:
        return None
    dev = device if device is not None else pairs[0][0].device
    D = torch.zeros((R, K), dtype=torch.bfloat16, device=dev)
    U = torch.zeros((N, R), dtype=torch.bfloat16, device=dev)
    r0 = 0
    for (down, up, scale), r in zip(pairs, ranks):
        D[r0:r0 + r] = down.to(dev, torch.float32).to(torch.bfloat16)
        U[:, r0:r0 + r] = (up.to(dev, torch.float32) * float(scale)).to(torch.bfloat16)
        r0 += r
    return D, U


def convrot_w8a8_linear(
    x: torch.Tensor,
    qweight: torch.Tensor,
    wscales: torch.Tensor,
    bias: torch.Tensor | None = None,
    convrot_groupsize: int = 256,
    *,
    qweight_i8t: torch.Tensor | None = None,
) -> torch.Tensor:
    """Compute ``x @ W.T + bias`` with the gfx950 W8A8 ConvRot path (the int8
    tier, reference _int4/__init__.py:141-175): fused rotate + int8 quantize of
    x (the eager arithmetic of _int4/int8_eager.py:22-28), then the int8 GEMM
    with exact int32 accumulation and the fp32 epilogue, both on torch's current
    stream.  qweight int8 [N, K], wscales [N] f32.  When K allows it the
    activation is quantized straight into the tile-major I8T layout and the GEMM
    reads ``qweight_i8t`` (from :func:`prepare_convrot_w8a8_weight_i8t`, made
    once at load time; re-laid here when not given): the same codes and
    accumulators, bit-identical outputs."""
    if x.shape[-1] != qweight.shape[-1]:
        raise ValueError(f"Input K={x.shape[-1]} does not match qweight K={qweight.shape[-1]}")
    if x.shape[-1] % convrot_groupsize != 0:
        raise ValueError(f"Input K={x.shape[-1]} not divisible by convrot_groupsize {convrot_groupsize}")
    _check_groupsize(convrot_groupsize)
    _check_width(x.shape[-1])
    orig_shape = x.shape
    x2d = x.reshape(-1, orig_shape[-1]).contiguous()
    if x2d.dtype not in native._IN_DTYPE_CODE:
        x2d = x2d.to(torch.float32)
    out_dtype = x.dtype if x.dtype in _NATIVE_OUT else torch.float32
    M, N = x2d.shape[0], qweight.shape[0]
    if i8t_path_ok(x2d.shape[1]) and x2d.is_cuda:
        w8t = qweight_i8t if qweight_i8t is not None else prepare_convrot_w8a8_weight_i8t(qweight)
        a8t, x_scale = native.convrot_quant_int8_i8t(x2d, convrot_groupsize)
        epi = native.EPI_F32 if out_dtype == torch.float32 else native.EPI_BF16
        out = native.int8_convrot_gemm_i8t(a8t, w8t, x_scale, wscales, bias, epi, M, N)
    else:
        qact, x_scale = native.convrot_quant_int8(x2d, convrot_groupsize)
        out = native.int8_convrot_gemm(qact, qweight, x_scale, wscales, bias, out_dtype)
    if out.dtype != x.dtype:
        out = out.to(x.dtype)
    return out.reshape(*orig_shape[:-1], qweight.shape[0])
