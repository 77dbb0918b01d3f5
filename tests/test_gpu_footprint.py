"""A quantized layer holds one copy of its weight on the device: the GEMM's
operand (B6T for int4: 0.75 B per parameter; I8T for int8: 1 B per
parameter), plus f32 scales and the fp16 bias (6 B per output row).  The
checkpoint layout the Save node reads (``_q``) is decoded from that operand
on demand, and what a save writes still equals the reference eager
quantization (config-1 weight goldens)."""
import hashlib
import importlib

import numpy as np
import pytest
import torch

from inputs import config1_bias, config1_weight

pytestmark = pytest.mark.gpu


def _ops():
    from fake_comfy import install_fake_comfy
    install_fake_comfy()
    m = importlib.import_module("comfyui-int4-convrot-rdna4_amd.int4_ops")
    if m.Int4ConvRotOps is None:
        m = importlib.reload(m)
    return m.Int4ConvRotOps


def _held_bytes(mod):
    """Bytes of the device tensors a quantized layer keeps."""
    ts = [mod._qpack, mod._q6, mod._q8t, mod._qs, mod.bias]
    return sum(t.numel() * t.element_size() for t in ts if t is not None and t.device.type == "cuda")


@pytest.mark.parametrize("mode,weight_bpp", [("int4", 0.75), ("int8", 1.0)])
def test_one_device_copy_per_layer(gpu, mode, weight_bpp):
    print(f"device footprint {mode} 3072x3072", flush=True)
    Ops = _ops()
    N = K = 3072
    w, b = config1_weight(), config1_bias()
    parent = torch.nn.Module()
    parent.lin = Ops.Linear(K, N, bias=True)
    Ops.int8_exact = {"lin"} if mode == "int8" else set()
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    try:
        parent.load_state_dict({"lin.weight": w.clone(), "lin.bias": b.clone()}, strict=False)
    finally:
        Ops.int8_exact = set()
    torch.cuda.synchronize()
    grown = torch.cuda.memory_allocated() - before
    lin = parent.lin
    assert lin._qmode == mode and lin._qpack is None          # no checkpoint-layout copy on the device
    op = lin._q6 if mode == "int4" else lin._q8t
    assert op is not None and op.numel() * op.element_size() == weight_bpp * N * K
    held = _held_bytes(lin)
    assert held == weight_bpp * N * K + 4 * N + 2 * N
    assert grown == held, (grown, held)                      # the temporaries of the load are freed
    per_param = held / (N * K)
    print(f"  {mode}: {per_param:.4f} B/param on the device (weight {weight_bpp} + scales and bias)", flush=True)
    assert per_param <= weight_bpp + 0.0021


def test_save_after_single_copy_load_matches_reference(goldens, gpu):
    """The Save path reads _q (decoded from the operand) and writes the
    reference eager quantization's bytes; reading _q allocates only a
    transient."""
    Ops = _ops()
    fmt = importlib.import_module("comfyui-int4-convrot-rdna4_amd.convrot_format")
    parent = torch.nn.Module()
    parent.l4 = Ops.Linear(3072, 3072, bias=False)
    parent.l8 = Ops.Linear(3072, 3072, bias=False)
    w = config1_weight()
    Ops.int8_exact = {"l8"}
    try:
        parent.load_state_dict({"l4.weight": w.clone(), "l8.weight": w.clone()}, strict=False)
    finally:
        Ops.int8_exact = set()
    torch.cuda.synchronize()
    held = torch.cuda.memory_allocated()
    sd, prec, _ = fmt.quantized_state_dict(parent, native=True)
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == held
    sha = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
    assert prec == {"l4": "int4", "l8": "int8"}
    assert sha(sd["l4.weight"].numpy()) == str(goldens["c1_qw_sha"])
    assert np.array_equal(sd["l4.weight_scale"].numpy(), goldens["c1_wscale"])
    assert sha(sd["l8.weight"].numpy()) == str(goldens["i8_c1_qw_sha"])
    assert np.array_equal(sd["l8.weight_scale"].reshape(-1).numpy(), goldens["i8_c1_wscale"])
