"""ctypes binding of libconvrot_gfx950.so (replaces the reference's
``_int4/hip_loader.py`` + JIT ``_int4/build.py``).

Same wrapper names, argument meaning and error behaviour as the reference
loader (``_int4/hip_loader.py:74-92`` ``convrot_quant_int4``,
``:158-207`` ``int4_convrot_gemm``, ``:150-155`` ``is_available``): outputs are
allocated here with torch, the work is enqueued on torch's current stream, a
nonzero return code raises ``RuntimeError``.  The library is prebuilt for
gfx950 (``build.py``); a missing library raises instead of building or falling
back to anything else.
"""
from __future__ import annotations

import collections
import ctypes
import os
import threading

import torch

from . import build as _build

_lib = None
_lock = threading.Lock()

# dtype codes of the C-ABI (reference _int4/hip_loader.py:38-39)
_DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1}
_IN_DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}

EPI_F32, EPI_BF16, EPI_BF16_EAGER, EPI_ACC = 0, 1, 2, 3

# cr_abi_version() of the library these signatures describe
ABI_VERSION = 13

_vp, _i = ctypes.c_void_p, ctypes.c_int
_SIGNATURES = {
    "ck_convrot_quant_int4": ([_vp, _i, _vp, _vp, _i, _i, _i, _vp], _i),
    "ck_int4_convrot_gemm": ([_vp] * 6 + [_i] * 4 + [_vp], _i),
    "ck_int4_convrot_gemm_splitk": ([_vp] * 5 + [_i] * 4 + [_vp], _i),
    "cr_int4_convrot_gemm_ex": ([_vp] * 6 + [_i] * 4 + [_vp], _i),
    "cr_convrot_quant_int4_stochastic": ([_vp, _i, _vp, _vp, _vp, _i, _i, _i, _vp], _i),
    "cr_lora_down": ([_vp, _i, _vp, _vp, _i, _i, _i, _vp, ctypes.c_size_t, _vp], _i),
    "cr_lora_down_workspace": ([_i, _i, _i], ctypes.c_size_t),
    "cr_int4_convrot_gemm_lora": ([_vp] * 7 + [_i, ctypes.c_float, _vp] + [_i] * 4 + [_vp], _i),
    "cr_int4_to_bf6": ([_vp, _vp, _i, _i, _vp], _i),
    "cr_bf6_to_int4": ([_vp, _vp, _i, _i, _vp], _i),
    "cr_convrot_quant_bf6": ([_vp, _i, _vp, _vp, _i, _i, _i, _vp], _i),
    "cr_max_quant_bf6_k": ([], _i),
    "cr_int4_convrot_gemm_bf6": ([_vp] * 6 + [_i] * 4 + [_vp], _i),
    "cr_int4_convrot_gemm_bf6_lora": ([_vp] * 7 + [_i, ctypes.c_float, _vp] + [_i] * 4 + [_vp], _i),
    "ck_convrot_quant_int8": ([_vp, _i, _vp, _vp, _i, _i, _i, _vp], _i),
    "ck_int8_convrot_gemm": ([_vp] * 6 + [_i] * 4 + [_vp], _i),
    "cr_int8_convrot_gemm_ex": ([_vp] * 6 + [_i] * 4 + [_vp], _i),
    "cr_convrot_quant_int8_i8t": ([_vp, _i, _vp, _vp, _i, _i, _i, _vp], _i),
    "cr_int8_to_i8t": ([_vp, _vp, _i, _i, _vp], _i),
    "cr_i8t_to_int8": ([_vp, _vp, _i, _i, _vp], _i),
    "cr_int8_convrot_gemm_i8t": ([_vp] * 6 + [_i] * 4 + [_vp], _i),
    "cr_gemm_bf6_choose_nsplit": ([_i, _i, _i], _i),
    "cr_gemm_bf6_splitk_workspace": ([_i, _i, _i], ctypes.c_size_t),
    "cr_gemm_bf6_tile": ([_i, _i, _i, _i, ctypes.POINTER(_i), ctypes.POINTER(_i)], _i),
    "cr_int4_convrot_gemm_bf6_splitk": ([_vp] * 7 + [_i, ctypes.c_float, _vp] + [_i] * 5 + [_vp, ctypes.c_size_t, _vp],
                                        _i),
    "cr_convrot_w4a4_linear_bf6": ([_vp, _i, _vp, _vp, _vp, _i, _vp, _vp, _i, ctypes.c_float, _vp] + [_i] * 5
                                   + [_vp, ctypes.c_size_t, _vp], _i),
    "cr_convrot_w4a4_linear_bf6_workspace": ([_i, _i, _i, _i], ctypes.c_size_t),
    "cr_convrot_w4a4_linear_bf6_noalloc": ([_vp, _i, _vp, _vp, _vp, _i, _vp, _vp, _i, ctypes.c_float, _vp] + [_i] * 5
                                           + [_vp], _i),
    "cr_max_quant_k": ([], _i),
    "cr_abi_version": ([], _i),
}


def lib_path() -> str:
    return _build.lib_path()


def load_library():
    """Load (once) and return the ctypes handle.  Loaded after torch so the
    library binds to the HIP runtime torch already mapped."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = lib_path()
        if not os.path.exists(path):
            raise RuntimeError(
                f"{os.path.basename(path)} is not built; run the package's _int4/build.py "
                "(hipcc --offload-arch=gfx950) first")
        lib = ctypes.CDLL(path)
        ver = lib.cr_abi_version
        ver.argtypes, ver.restype = [], _i
        if ver() != ABI_VERSION:
            raise RuntimeError(f"{os.path.basename(path)} has ABI version {ver()}, these bindings need "
                               f"{ABI_VERSION}; rebuild it with the package's _int4/build.py")
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def _is_gfx950() -> bool:
    if getattr(torch.version, "hip", None) is None or not torch.cuda.is_available():
        return False
    try:
        arch = (torch.cuda.get_device_properties(0).gcnArchName or "").split(":")[0]
    except Exception:
        return False
    return arch == "gfx950"


def is_available() -> bool:
    """True only on a gfx950 ROCm device with the library loadable."""
    if not _is_gfx950():
        return False
    try:
        load_library()
        return True
    except Exception:
        return False


def _ptr(t):
    # a plain int: the c_void_p argtypes convert it (None is NULL)
    return t.data_ptr() if t is not None else None


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device) -> int:
    """The current HIP stream of ``device`` as an integer handle (the raw
    query skips building a torch Stream object per call)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return _raw_stream(index)
    return torch.cuda.current_stream(index).cuda_stream


# One reusable workspace per (device, stream): calls on a stream run in stream
# order, so a call may reuse the workspace of the previous call on the same
# stream; calls on other streams get their own.  It only grows.  A dropped
# buffer (replaced, or evicted when more than _MAX_WORKSPACES streams are in
# use) goes back to torch's allocator, which allocated it on that stream and
# hands it out again only in that stream's order.  Calls captured into a HIP
# graph get a buffer of their own.
# The library keeps the split counters of its bf6 GEMM in the first
# SPLIT_COUNTER_BYTES of every workspace: they must be zero when a buffer is
# first used (every call leaves them zero), so a new buffer gets them cleared
# by a fill kernel on the stream that will use it.
_MAX_WORKSPACES = 16
SPLIT_COUNTER_BYTES = 2048
_workspaces: "collections.OrderedDict" = collections.OrderedDict()
_workspaces_lock = threading.Lock()


def _new_workspace(device, nbytes: int) -> torch.Tensor:
    ws = torch.empty((max(nbytes, SPLIT_COUNTER_BYTES),), dtype=torch.uint8, device=device)
    ws[:SPLIT_COUNTER_BYTES].zero_()
    return ws


def _workspace(device, stream: int, nbytes: int) -> torch.Tensor:
    if torch.cuda.is_current_stream_capturing():
        # a graph keeps the address it captured: give it a buffer of its own
        # (from the graph's pool; its counters cleared inside the graph), never
        # the stream's shared one
        return _new_workspace(device, nbytes)
    key = (device.index, stream)
    with _workspaces_lock:
        ws = _workspaces.get(key)
        if ws is None or ws.numel() < nbytes:
            ws = _new_workspace(device, nbytes)
            _workspaces[key] = ws
        _workspaces.move_to_end(key)
        while len(_workspaces) > _MAX_WORKSPACES:
            _workspaces.popitem(last=False)
    return ws


def _check_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"expected a CUDA (HIP) tensor, got device {t.device}")


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """Contiguous and 16-byte aligned (the kernels use 128-bit loads/stores)."""
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


_limits: dict = {}


def _limit(name: str) -> int:
    # constants of the loaded library, queried once
    v = _limits.get(name)
    if v is None:
        v = _limits[name] = int(getattr(load_library(), name)())
    return v


def max_quant_k() -> int:
    return _limit("cr_max_quant_k")


def convrot_quant_int4(x: torch.Tensor, convrot_groupsize: int):
    """Fused ConvRot rotation + rowwise int4 quantize (reference hip_loader.py:74-92).

    Returns (qpacked int8 [M, K/2], scale f32 [M]).  Supports groupsize 16/64/256.
    """
    lib = load_library()
    if convrot_groupsize not in (16, 64, 256):
        raise ValueError("fused convrot_quant_int4 supports groupsize 16/64/256")
    if x.dtype not in _IN_DTYPE_CODE:
        raise ValueError(f"convrot_quant_int4 input dtype must be f32/bf16/f16, got {x.dtype}")
    _check_cuda(x)
    x = _aligned(x)
    M, K = x.shape
    qout = torch.empty((M, K // 2), dtype=torch.int8, device=x.device)
    scale = torch.empty((M,), dtype=torch.float32, device=x.device)
    rc = lib.ck_convrot_quant_int4(_ptr(x), _IN_DTYPE_CODE[x.dtype], _ptr(qout), _ptr(scale),
                                   M, K, convrot_groupsize, _stream(x.device))
    if rc != 0:
        raise RuntimeError(f"ck_convrot_quant_int4 failed, hipError={rc}")
    return qout, scale


def convrot_quant_int4_stochastic(x: torch.Tensor, convrot_groupsize: int, noise: torch.Tensor):
    """Rotation + int4 quantize with stochastic rounding q = floor(t + u)."""
    lib = load_library()
    if convrot_groupsize not in (16, 64, 256):
        raise ValueError("fused convrot_quant_int4 supports groupsize 16/64/256")
    if x.dtype not in _IN_DTYPE_CODE or noise.dtype != x.dtype or noise.shape != x.shape:
        raise ValueError("noise must match x in shape and dtype")
    _check_cuda(x, noise)
    x = _aligned(x)
    noise = noise.contiguous()
    M, K = x.shape
    qout = torch.empty((M, K // 2), dtype=torch.int8, device=x.device)
    scale = torch.empty((M,), dtype=torch.float32, device=x.device)
    rc = lib.cr_convrot_quant_int4_stochastic(_ptr(x), _IN_DTYPE_CODE[x.dtype], _ptr(noise), _ptr(qout),
                                              _ptr(scale), M, K, convrot_groupsize, _stream(x.device))
    if rc != 0:
        raise RuntimeError(f"cr_convrot_quant_int4_stochastic failed, hipError={rc}")
    return qout, scale


def _gemm_args(x_packed, w_packed, x_scale, w_scale, bias):
    _check_cuda(x_packed, w_packed, x_scale, w_scale, bias)
    x_packed = _aligned(x_packed)
    w_packed = _aligned(w_packed)
    if x_packed.dtype != torch.int8 or w_packed.dtype != torch.int8:
        raise ValueError("packed operands must be int8")
    M, Kp = x_packed.shape
    N, Kp2 = w_packed.shape
    if Kp != Kp2:
        raise ValueError(f"K mismatch: x {tuple(x_packed.shape)} w {tuple(w_packed.shape)}")
    x_scale = x_scale.to(torch.float32).contiguous() if x_scale is not None else None
    w_scale = w_scale.to(torch.float32).contiguous() if w_scale is not None else None
    if bias is not None:
        bias = bias.to(torch.float32).contiguous()
    return x_packed, w_packed, x_scale, w_scale, bias, M, N, 2 * Kp


def int4_convrot_gemm_ex(x_packed, w_packed, x_scale, w_scale, bias, epilogue: int):
    """out = epilogue(sum_k qx qw, x_scale, w_scale, bias); see include/convrot_mi355x.h."""
    lib = load_library()
    x_packed, w_packed, x_scale, w_scale, bias, M, N, K = _gemm_args(
        x_packed, w_packed, x_scale, w_scale, bias)
    odt = {EPI_F32: torch.float32, EPI_BF16: torch.bfloat16, EPI_BF16_EAGER: torch.bfloat16,
           EPI_ACC: torch.int32}[epilogue]
    out = torch.empty((M, N), dtype=odt, device=x_packed.device)
    rc = lib.cr_int4_convrot_gemm_ex(_ptr(x_packed), _ptr(w_packed), _ptr(x_scale), _ptr(w_scale),
                                     _ptr(bias), _ptr(out), M, N, K, epilogue, _stream(x_packed.device))
    if rc != 0:
        raise RuntimeError(f"cr_int4_convrot_gemm_ex failed, hipError={rc}")
    return out


def int4_gemm_acc(x_packed, w_packed):
    """Exact int32 accumulators acc[m, n] = sum_k qx[m,k] * qw[n,k]."""
    return int4_convrot_gemm_ex(x_packed, w_packed, None, None, None, EPI_ACC)


def int4_convrot_gemm(x_packed, w_packed, x_scale, w_scale, bias, out_dtype):
    """out[M,N] = (Xint @ Wint^T) * x_scale[:,None] * w_scale[None,:] (+ bias)
    (reference hip_loader.py:158-207, without its split-K branch: the gfx950
    kernel fills the device at every shape that path served)."""
    if out_dtype not in _DTYPE_CODE:
        raise ValueError(f"hip int4 gemm output dtype must be float32/bfloat16, got {out_dtype}")
    lib = load_library()
    x_packed, w_packed, x_scale, w_scale, bias, M, N, K = _gemm_args(
        x_packed, w_packed, x_scale, w_scale, bias)
    out = torch.empty((M, N), dtype=out_dtype, device=x_packed.device)
    rc = lib.ck_int4_convrot_gemm(_ptr(x_packed), _ptr(w_packed), _ptr(x_scale), _ptr(w_scale),
                                  _ptr(bias), _ptr(out), M, N, K, _DTYPE_CODE[out_dtype],
                                  _stream(x_packed.device))
    if rc != 0:
        raise RuntimeError(f"ck_int4_convrot_gemm failed, hipError={rc}")
    return out


def int4_convrot_gemm_splitk(x_packed, w_packed, x_scale, w_scale, nsplit: int):
    """Split-K form (reference hip_loader.py:176-192): returns the f32 [M, N]
    product (Xint @ Wint^T) * x_scale[:,None] * w_scale[None,:] without bias,
    accumulated by ck_int4_convrot_gemm_splitk into a zeroed buffer.  Bit-
    identical to int4_convrot_gemm(..., bias=None, float32) for every nsplit."""
    if nsplit < 1:
        raise ValueError(f"nsplit must be >= 1, got {nsplit}")
    lib = load_library()
    x_packed, w_packed, x_scale, w_scale, _, M, N, K = _gemm_args(x_packed, w_packed, x_scale, w_scale, None)
    if x_scale is None or w_scale is None or x_scale.numel() != M or w_scale.numel() != N:
        raise ValueError("x_scale [M] and w_scale [N] are required")
    accum = torch.zeros((M, N), dtype=torch.float32, device=x_packed.device)
    rc = lib.ck_int4_convrot_gemm_splitk(_ptr(x_packed), _ptr(w_packed), _ptr(x_scale), _ptr(w_scale), _ptr(accum),
                                         M, N, K, nsplit, _stream(x_packed.device))
    if rc != 0:
        raise RuntimeError(f"ck_int4_convrot_gemm_splitk failed, hipError={rc}")
    return accum


def lora_down(x: torch.Tensor, down: torch.Tensor) -> torch.Tensor:
    """t = bf16(x @ down^T) for the dynamic-LoRA side path.  x [M, K] bf16/f16,
    down [R, K] bf16 with R in {32, 64, 96, 128} -> t [M, R] bf16."""
    lib = load_library()
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"lora_down input must be bf16/f16, got {x.dtype}")
    if down.dtype != torch.bfloat16:
        raise ValueError("lora down weights must be bf16")
    _check_cuda(x, down)
    x = _aligned(x)
    down = _aligned(down)
    M, K = x.shape
    R, K2 = down.shape
    if K != K2:
        raise ValueError(f"K mismatch: x {tuple(x.shape)} down {tuple(down.shape)}")
    t = torch.empty((M, R), dtype=torch.bfloat16, device=x.device)
    if M == 0:
        return t
    nbytes = lib.cr_lora_down_workspace(M, K, R)        # 0 for an unsplit shape
    st = _stream(x.device)
    ws = _workspace(x.device, st, nbytes)
    rc = lib.cr_lora_down(_ptr(x), _IN_DTYPE_CODE[x.dtype], _ptr(down), _ptr(t), M, K, R, _ptr(ws), nbytes, st)
    if rc != 0:
        raise RuntimeError(f"cr_lora_down failed, hipError={rc}")
    return t


def int4_convrot_gemm_lora(x_packed, w_packed, x_scale, w_scale, bias, t, up, scale: float, epilogue: int):
    """GEMM + dequant epilogue + scale * (t @ up^T); t [M, R], up [N, R] bf16."""
    lib = load_library()
    x_packed, w_packed, x_scale, w_scale, bias, M, N, K = _gemm_args(
        x_packed, w_packed, x_scale, w_scale, bias)
    _check_cuda(t, up)
    t = _aligned(t)
    up = _aligned(up)
    R = t.shape[1]
    if t.dtype != torch.bfloat16 or up.dtype != torch.bfloat16 or up.shape != (N, R) or t.shape[0] != M:
        raise ValueError("lora operands: t [M, R] and up [N, R] bf16")
    odt = {EPI_F32: torch.float32, EPI_BF16: torch.bfloat16, EPI_BF16_EAGER: torch.bfloat16}[epilogue]
    out = torch.empty((M, N), dtype=odt, device=x_packed.device)
    rc = lib.cr_int4_convrot_gemm_lora(_ptr(x_packed), _ptr(w_packed), _ptr(x_scale), _ptr(w_scale), _ptr(bias),
                                       _ptr(t), _ptr(up), R, ctypes.c_float(scale), _ptr(out), M, N, K, epilogue,
                                       _stream(x_packed.device))
    if rc != 0:
        raise RuntimeError(f"cr_int4_convrot_gemm_lora failed, hipError={rc}")
    return out


def bf6_rows(rows: int) -> int:
    """Rows of a B6T operand buffer: the row count padded to a multiple of 256."""
    return (rows + 255) // 256 * 256


def int4_to_bf6(packed: torch.Tensor) -> torch.Tensor:
    """Packed int4 [rows, K/2] -> B6T bf6 operand, uint8 [bf6_rows(rows), 3K/4] (K % 128 == 0).
    The row padding holds zero codes; the logical row count travels with the scales."""
    lib = load_library()
    _check_cuda(packed)
    if packed.dtype not in (torch.int8, torch.uint8) or packed.dim() != 2:
        raise ValueError("packed int4 operand must be a 2-D int8 tensor")
    packed = _aligned(packed)
    rows, K = packed.shape[0], packed.shape[1] * 2
    if K % 128 != 0:
        raise ValueError(f"bf6 operands need K % 128 == 0, got K={K}")
    out = torch.empty((bf6_rows(rows), K // 4 * 3), dtype=torch.uint8, device=packed.device)
    rc = lib.cr_int4_to_bf6(_ptr(packed), _ptr(out), rows, K, _stream(packed.device))
    if rc != 0:
        raise RuntimeError(f"cr_int4_to_bf6 failed, hipError={rc}")
    return out


def bf6_to_int4(a6: torch.Tensor, rows: int, K: int) -> torch.Tensor:
    """B6T operand -> packed int4 [rows, K/2] (the inverse of int4_to_bf6 on the
    first ``rows`` rows, bit for bit)."""
    lib = load_library()
    _check_cuda(a6)
    if a6.dtype != torch.uint8 or a6.shape != (bf6_rows(rows), K // 4 * 3) or K % 128 != 0:
        raise ValueError(f"a B6T operand of a [{rows}, {K}] matrix is uint8 [{bf6_rows(rows)}, {K // 4 * 3}], "
                         f"got {a6.dtype} {tuple(a6.shape)}")
    a6 = _aligned(a6)
    out = torch.empty((rows, K // 2), dtype=torch.int8, device=a6.device)
    rc = lib.cr_bf6_to_int4(_ptr(a6), _ptr(out), rows, K, _stream(a6.device))
    if rc != 0:
        raise RuntimeError(f"cr_bf6_to_int4 failed, hipError={rc}")
    return out


def max_quant_bf6_k() -> int:
    return _limit("cr_max_quant_bf6_k")


def convrot_quant_bf6(x: torch.Tensor, convrot_groupsize: int):
    """Fused rotate + int4 quantize of x [M, K] (f32/bf16/f16) straight into the
    B6T bf6 operand layout.  Returns (a6 uint8 [bf6_rows(M), 3K/4], scale f32 [M]);
    the codes and scales equal convrot_quant_int4's.  K % 128 == 0, K <= max_quant_bf6_k()."""
    lib = load_library()
    _check_cuda(x)
    if x.dim() != 2 or x.dtype not in _IN_DTYPE_CODE:
        raise ValueError("x must be a 2-D f32/bf16/f16 tensor")
    x = _aligned(x)
    M, K = x.shape
    if K % 128 != 0 or K > lib.cr_max_quant_bf6_k() or K % convrot_groupsize != 0:
        raise ValueError(f"bf6 activation quantization needs K % 128 == 0 and K <= {lib.cr_max_quant_bf6_k()}")
    a6 = torch.empty((bf6_rows(M), K // 4 * 3), dtype=torch.uint8, device=x.device)
    s = torch.empty((M,), dtype=torch.float32, device=x.device)
    rc = lib.cr_convrot_quant_bf6(_ptr(x), _IN_DTYPE_CODE[x.dtype], _ptr(a6), _ptr(s), M, K, convrot_groupsize,
                                  _stream(x.device))
    if rc != 0:
        raise RuntimeError(f"cr_convrot_quant_bf6 failed, hipError={rc}")
    return a6, s


def _bf6_gemm_args(a6, w6, x_scale, w_scale, bias, M, N):
    _check_cuda(a6, w6, x_scale, w_scale, bias)
    if a6.dtype != torch.uint8 or w6.dtype != torch.uint8 or a6.dim() != 2 or w6.dim() != 2:
        raise ValueError("bf6 operands must be 2-D uint8 tensors")
    if a6.shape[1] != w6.shape[1] or a6.shape[1] % 96 != 0:
        raise ValueError(f"bf6 operand widths {a6.shape[1]} / {w6.shape[1]} do not match a K % 128 == 0")
    K = a6.shape[1] // 3 * 4
    M = x_scale.numel() if M is None else M
    N = w_scale.numel() if N is None else N
    if a6.shape[0] != bf6_rows(M) or w6.shape[0] != bf6_rows(N):
        raise ValueError(f"bf6 operands of {a6.shape[0]} / {w6.shape[0]} rows do not hold M={M} / N={N}")
    xs = _aligned(x_scale.reshape(-1).to(torch.float32)) if x_scale is not None else None
    wsc = _aligned(w_scale.reshape(-1).to(torch.float32)) if w_scale is not None else None
    if (xs is not None and xs.numel() != M) or (wsc is not None and wsc.numel() != N):
        raise ValueError("scale lengths do not match the operands")
    b = None
    if bias is not None:
        b = _aligned(bias.reshape(-1).to(torch.float32))
        if b.numel() != N:
            raise ValueError("bias length does not match N")
    return _aligned(a6), _aligned(w6), xs, wsc, b, M, N, K


def choose_nsplit_bf6(M: int, N: int, K: int) -> int:
    """The library's k-split count for an M x N x K bf6 GEMM (1: no split)."""
    return int(load_library().cr_gemm_bf6_choose_nsplit(M, N, K))


def gemm_tile_bf6(M: int, N: int, K: int, nsplit: int = 1) -> tuple[int, int]:
    """The workgroup tile (rows of A, rows of B) of a bf6 GEMM launch."""
    bm, bn = ctypes.c_int(0), ctypes.c_int(0)
    if load_library().cr_gemm_bf6_tile(M, N, K, nsplit, ctypes.byref(bm), ctypes.byref(bn)) != 0:
        raise ValueError(f"no bf6 GEMM launch takes M={M} N={N} K={K} nsplit={nsplit}")
    return bm.value, bn.value


def _bf6_launch(a6, w6, xs, wsc, b, t, up, R, scale, out, M, N, K, epilogue, nsplit):
    """One bf6 GEMM: unsplit through the plain entry points, split-K through
    cr_int4_convrot_gemm_bf6_splitk with the stream's workspace."""
    lib = load_library()
    if nsplit is None:
        nsplit = lib.cr_gemm_bf6_choose_nsplit(M, N, K) if M > 0 and N > 0 else 1
    st = _stream(a6.device)
    if nsplit <= 1:
        if t is None:
            rc = lib.cr_int4_convrot_gemm_bf6(_ptr(a6), _ptr(w6), _ptr(xs), _ptr(wsc), _ptr(b), _ptr(out),
                                              M, N, K, epilogue, st)
            name = "cr_int4_convrot_gemm_bf6"
        else:
            rc = lib.cr_int4_convrot_gemm_bf6_lora(_ptr(a6), _ptr(w6), _ptr(xs), _ptr(wsc), _ptr(b), _ptr(t),
                                                   _ptr(up), R, ctypes.c_float(scale), _ptr(out), M, N, K,
                                                   epilogue, st)
            name = "cr_int4_convrot_gemm_bf6_lora"
    else:
        nbytes = lib.cr_gemm_bf6_splitk_workspace(M, N, nsplit)
        ws = _workspace(a6.device, st, nbytes)
        rc = lib.cr_int4_convrot_gemm_bf6_splitk(_ptr(a6), _ptr(w6), _ptr(xs), _ptr(wsc), _ptr(b), _ptr(t),
                                                 _ptr(up), R, ctypes.c_float(scale), _ptr(out), M, N, K, epilogue,
                                                 nsplit, _ptr(ws), nbytes, st)
        name = "cr_int4_convrot_gemm_bf6_splitk"
    if rc != 0:
        raise RuntimeError(f"{name} failed, hipError={rc}")
    return out


def int4_convrot_gemm_bf6(a6, w6, x_scale, w_scale, bias, epilogue: int, M=None, N=None, nsplit=None):
    """W4A4 GEMM on B6T operands (exact accumulators), epilogue 0..3 as
    int4_convrot_gemm_ex.  M / N default to the scale lengths.  nsplit: k
    splits (None: the library's choice; the outputs are identical either way)."""
    a6, w6, xs, wsc, b, M, N, K = _bf6_gemm_args(a6, w6, x_scale, w_scale, bias, M, N)
    odt = {EPI_F32: torch.float32, EPI_BF16: torch.bfloat16, EPI_BF16_EAGER: torch.bfloat16,
           EPI_ACC: torch.int32}[epilogue]
    out = torch.empty((M, N), dtype=odt, device=a6.device)
    return _bf6_launch(a6, w6, xs, wsc, b, None, None, 0, 0.0, out, M, N, K, epilogue, nsplit)


def int4_gemm_acc_bf6(a6, w6, M: int, N: int, nsplit=None):
    """int32 accumulators of the bf6 GEMM (exact)."""
    return int4_convrot_gemm_bf6(a6, w6, None, None, None, EPI_ACC, M=M, N=N, nsplit=nsplit)


def int4_convrot_gemm_bf6_lora(a6, w6, x_scale, w_scale, bias, t, up, scale: float, epilogue: int, nsplit=None):
    """int4_convrot_gemm_bf6 + scale * (t @ up^T) in the epilogue (0..2)."""
    a6, w6, xs, wsc, b, M, N, K = _bf6_gemm_args(a6, w6, x_scale, w_scale, bias, None, None)
    _check_cuda(t, up)
    t = _aligned(t)
    up = _aligned(up)
    R = t.shape[1]
    if t.dtype != torch.bfloat16 or up.dtype != torch.bfloat16 or up.shape != (N, R) or t.shape[0] != M:
        raise ValueError("lora operands: t [M, R] and up [N, R] bf16")
    odt = {EPI_F32: torch.float32, EPI_BF16: torch.bfloat16, EPI_BF16_EAGER: torch.bfloat16}[epilogue]
    out = torch.empty((M, N), dtype=odt, device=a6.device)
    return _bf6_launch(a6, w6, xs, wsc, b, t, up, R, scale, out, M, N, K, epilogue, nsplit)


# ----------------------------------------------------------------------------
# W8A8 tier (reference _int4/int8_eager.py, hip_loader.py:95-147)
# ----------------------------------------------------------------------------

def convrot_quant_int8(x: torch.Tensor, convrot_groupsize: int):
    """Fused ConvRot rotation + rowwise int8 quantize (reference hip_loader.py:95-113).

    Returns (q int8 [M, K], scale f32 [M]).  Supports groupsize 16/64/256."""
    lib = load_library()
    if convrot_groupsize not in (16, 64, 256):
        raise ValueError("fused convrot_quant_int8 supports groupsize 16/64/256")
    if x.dtype not in _IN_DTYPE_CODE:
        raise ValueError(f"convrot_quant_int8 input dtype must be f32/bf16/f16, got {x.dtype}")
    _check_cuda(x)
    x = _aligned(x)
    M, K = x.shape
    qout = torch.empty((M, K), dtype=torch.int8, device=x.device)
    scale = torch.empty((M,), dtype=torch.float32, device=x.device)
    rc = lib.ck_convrot_quant_int8(_ptr(x), _IN_DTYPE_CODE[x.dtype], _ptr(qout), _ptr(scale),
                                   M, K, convrot_groupsize, _stream(x.device))
    if rc != 0:
        raise RuntimeError(f"ck_convrot_quant_int8 failed, hipError={rc}")
    return qout, scale


def int8_convrot_gemm_ex(x_int8, w_int8, x_scale, w_scale, bias, epilogue: int):
    """W8A8 GEMM with epilogue 0 (f32), 1 (bf16) or 3 (int32 accumulators)."""
    lib = load_library()
    _check_cuda(x_int8, w_int8, x_scale, w_scale, bias)
    if x_int8.dtype != torch.int8 or w_int8.dtype != torch.int8:
        raise ValueError("W8A8 operands must be int8")
    x_int8, w_int8 = _aligned(x_int8), _aligned(w_int8)
    M, K = x_int8.shape
    N, K2 = w_int8.shape
    if K != K2:
        raise ValueError(f"K mismatch: x {tuple(x_int8.shape)} w {tuple(w_int8.shape)}")
    xs = x_scale.to(torch.float32).contiguous() if x_scale is not None else None
    wsc = w_scale.to(torch.float32).contiguous() if w_scale is not None else None
    b = bias.to(torch.float32).contiguous() if bias is not None else None
    odt = {EPI_F32: torch.float32, EPI_BF16: torch.bfloat16, EPI_ACC: torch.int32}[epilogue]
    out = torch.empty((M, N), dtype=odt, device=x_int8.device)
    rc = lib.cr_int8_convrot_gemm_ex(_ptr(x_int8), _ptr(w_int8), _ptr(xs), _ptr(wsc), _ptr(b), _ptr(out),
                                     M, N, K, epilogue, _stream(x_int8.device))
    if rc != 0:
        raise RuntimeError(f"cr_int8_convrot_gemm_ex failed, hipError={rc}")
    return out


def int8_gemm_acc(x_int8, w_int8):
    """Exact int32 accumulators of the W8A8 product."""
    return int8_convrot_gemm_ex(x_int8, w_int8, None, None, None, EPI_ACC)


def int8_convrot_gemm(x_int8, w_int8, x_scale, w_scale, bias, out_dtype):
    """out[M,N] = (X[M,K] @ W[N,K]^T) * x_scale[:,None] * w_scale[None,:] (+bias)
    (reference hip_loader.py:116-147); out_dtype float32 or bfloat16."""
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"int8 gemm output dtype must be float32/bfloat16, got {out_dtype}")
    return int8_convrot_gemm_ex(x_int8, w_int8, x_scale, w_scale, bias,
                                EPI_F32 if out_dtype == torch.float32 else EPI_BF16)


def i8t_rows(rows: int) -> int:
    """Rows of an I8T operand: the logical rows padded to a multiple of 256."""
    return (rows + 255) // 256 * 256


def int8_to_i8t(q: torch.Tensor) -> torch.Tensor:
    """Row-major int8 codes [rows, K] -> the I8T operand of the W8A8 GEMM,
    int8 [i8t_rows(rows), K] in chunk order (K % 64 == 0; padding rows zero)."""
    lib = load_library()
    _check_cuda(q)
    if q.dtype != torch.int8 or q.dim() != 2:
        raise ValueError("int8 codes must be a 2-D int8 tensor")
    q = _aligned(q)
    rows, K = q.shape
    if K % 64 != 0:
        raise ValueError(f"I8T operands need K % 64 == 0, got K={K}")
    out = torch.empty((i8t_rows(rows), K), dtype=torch.int8, device=q.device)
    rc = lib.cr_int8_to_i8t(_ptr(q), _ptr(out), rows, K, _stream(q.device))
    if rc != 0:
        raise RuntimeError(f"cr_int8_to_i8t failed, hipError={rc}")
    return out


def i8t_to_int8(q8t: torch.Tensor, rows: int) -> torch.Tensor:
    """I8T operand -> row-major int8 [rows, K] (the inverse of int8_to_i8t on
    the first ``rows`` rows)."""
    lib = load_library()
    _check_cuda(q8t)
    K = q8t.shape[-1]
    if q8t.dtype != torch.int8 or q8t.shape != (i8t_rows(rows), K) or K % 64 != 0:
        raise ValueError(f"an I8T operand of {rows} rows is int8 [{i8t_rows(rows)}, K], got {q8t.dtype} "
                         f"{tuple(q8t.shape)}")
    q8t = _aligned(q8t)
    out = torch.empty((rows, K), dtype=torch.int8, device=q8t.device)
    rc = lib.cr_i8t_to_int8(_ptr(q8t), _ptr(out), rows, K, _stream(q8t.device))
    if rc != 0:
        raise RuntimeError(f"cr_i8t_to_int8 failed, hipError={rc}")
    return out


def convrot_quant_int8_i8t(x: torch.Tensor, convrot_groupsize: int):
    """Fused rotate + int8 quantize of x [M, K] straight into the I8T layout.
    Returns (q int8 [i8t_rows(M), K], scale f32 [M]); the codes and scales equal
    convrot_quant_int8's.  K % 64 == 0, K <= max_quant_bf6_k()."""
    lib = load_library()
    _check_cuda(x)
    if x.dim() != 2 or x.dtype not in _IN_DTYPE_CODE:
        raise ValueError("x must be a 2-D f32/bf16/f16 tensor")
    if convrot_groupsize not in (16, 64, 256):
        raise ValueError("fused convrot_quant_int8 supports groupsize 16/64/256")
    x = _aligned(x)
    M, K = x.shape
    if K % 64 != 0 or K > lib.cr_max_quant_bf6_k() or K % convrot_groupsize != 0:
        raise ValueError(f"I8T activation quantization needs K % 64 == 0 and K <= {lib.cr_max_quant_bf6_k()}")
    q = torch.empty((i8t_rows(M), K), dtype=torch.int8, device=x.device)
    s = torch.empty((M,), dtype=torch.float32, device=x.device)
    rc = lib.cr_convrot_quant_int8_i8t(_ptr(x), _IN_DTYPE_CODE[x.dtype], _ptr(q), _ptr(s), M, K, convrot_groupsize,
                                       _stream(x.device))
    if rc != 0:
        raise RuntimeError(f"cr_convrot_quant_int8_i8t failed, hipError={rc}")
    return q, s


def int8_convrot_gemm_i8t(a8t, w8t, x_scale, w_scale, bias, epilogue: int, M: int, N: int):
    """W8A8 GEMM on I8T operands (a8t [i8t_rows(M), K], w8t [i8t_rows(N), K])
    with epilogue 0 (f32), 1 (bf16) or 3 (int32 accumulators); bit-identical to
    int8_convrot_gemm_ex on the row-major codes."""
    lib = load_library()
    _check_cuda(a8t, w8t, x_scale, w_scale, bias)
    if a8t.dtype != torch.int8 or w8t.dtype != torch.int8:
        raise ValueError("I8T operands must be int8")
    K = a8t.shape[1]
    if w8t.shape[1] != K or a8t.shape[0] != i8t_rows(M) or w8t.shape[0] != i8t_rows(N):
        raise ValueError(f"I8T operand shapes {tuple(a8t.shape)} / {tuple(w8t.shape)} do not match M={M}, N={N}")
    xs = x_scale.to(torch.float32).contiguous() if x_scale is not None else None
    wsc = w_scale.to(torch.float32).contiguous() if w_scale is not None else None
    b = bias.to(torch.float32).contiguous() if bias is not None else None
    odt = {EPI_F32: torch.float32, EPI_BF16: torch.bfloat16, EPI_ACC: torch.int32}[epilogue]
    out = torch.empty((M, N), dtype=odt, device=a8t.device)
    rc = lib.cr_int8_convrot_gemm_i8t(_ptr(a8t), _ptr(w8t), _ptr(xs), _ptr(wsc), _ptr(b), _ptr(out),
                                      M, N, K, epilogue, _stream(a8t.device))
    if rc != 0:
        raise RuntimeError(f"cr_int8_convrot_gemm_i8t failed, hipError={rc}")
    return out


def convrot_w4a4_linear_bf6(x2d, w6, w_scale, bias, down, up, scale: float, epilogue: int, convrot_groupsize: int,
                            N: int):
    """The whole bf6 linear in one library call (cr_convrot_w4a4_linear_bf6):
    rotate + quantize x2d [M, K], the LoRA down projection when ``down`` is given,
    the GEMM with the epilogue (and the LoRA term).  w_scale f32 [N]; bias [N]
    f32 / bf16 / f16 as stored, or None; down [R, K] / up [N, R] bf16."""
    lib = load_library()
    M, K = x2d.shape
    odt = {EPI_F32: torch.float32, EPI_BF16: torch.bfloat16, EPI_BF16_EAGER: torch.bfloat16}[epilogue]
    out = torch.empty((M, N), dtype=odt, device=x2d.device)
    R = 0 if down is None else down.shape[0]
    nbytes = lib.cr_convrot_w4a4_linear_bf6_workspace(M, N, K, R)
    st = _stream(x2d.device)
    ws = _workspace(x2d.device, st, nbytes)
    bdt = 0 if bias is None else _IN_DTYPE_CODE[bias.dtype]
    rc = lib.cr_convrot_w4a4_linear_bf6(_ptr(x2d), _IN_DTYPE_CODE[x2d.dtype], _ptr(w6), _ptr(w_scale), _ptr(bias),
                                        bdt, _ptr(down), _ptr(up), R, scale, _ptr(out), epilogue,
                                        M, N, K, convrot_groupsize, _ptr(ws), nbytes, st)
    if rc != 0:
        raise RuntimeError(f"cr_convrot_w4a4_linear_bf6 failed, hipError={rc}")
    return out
