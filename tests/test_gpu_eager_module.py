"""``_int4.eager`` on the GPU, called the way the reference's sensitivity node
calls it (int4_sensitivity.py:43-61): the fp16 weight quantized by the gfx950
kernel equals the reference eager quantization (config-1 goldens), the fp32
dequantization equals the oracle's float64 one within fp32 rounding, and the
module's linear reproduces the reference eager output bit for bit."""
import hashlib
import importlib

import numpy as np
import pytest
import torch

from inputs import config1_bias, config1_weight, config1_x

pytestmark = pytest.mark.gpu


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def eager(gpu):
    return importlib.import_module("comfyui-int4-convrot-rdna4_amd._int4.eager")


def test_sensitivity_round_trip(eager, oracle, goldens):
    print("eager module: weight round trip 3072x3072", flush=True)
    w = config1_weight()
    w32 = w.float().cuda()
    qw, ws = eager.quantize_convrot_w4a4_weight(w32.to(torch.float16), convrot_groupsize=256)
    assert qw.is_cuda and qw.dtype == torch.int8 and ws.dtype == torch.float32
    assert sha(qw.cpu().numpy()) == str(goldens["c1_qw_sha"])
    assert np.array_equal(ws.cpu().numpy(), goldens["c1_wscale"])
    deq = eager.dequantize_convrot_w4a4_weight(qw, ws, convrot_groupsize=256, output_dtype=torch.float32)
    assert deq.dtype == torch.float32 and deq.shape == (3072, 3072)
    want = oracle.dequantize_weight(qw.cpu().numpy(), ws.cpu().numpy(), 256)
    d = deq.cpu().numpy().astype(np.float64)
    # fp32 matmul of 256-term rows: within a few fp32 ulps of the row's scale
    tol = 1e-5 * np.abs(want).max()
    assert np.abs(d - want).max() <= tol
    # the score the node computes: int4 weight error of a N(0, 0.02) weight
    rel = float(np.linalg.norm(w.double().numpy() - d) / np.linalg.norm(w.double().numpy()))
    assert 0.05 < rel < 0.3, rel


def test_eager_linear_equals_reference_eager_output(eager, backend, goldens):
    print("eager module: linear 256x3072->3072", flush=True)
    qw, ws = backend.quantize_convrot_w4a4_weight(config1_weight().cuda())
    y = eager.convrot_w4a4_linear(config1_x().cuda(), qw, ws, config1_bias().cuda(), 256)
    assert y.dtype == torch.bfloat16
    assert sha(y.cpu().view(torch.int16).numpy().view(np.uint16)) == str(goldens["c1_y_sha"])
