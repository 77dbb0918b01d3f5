"""The on-disk format on the GPU path: a stack quantized on load (int4 and
int8 layers) is written with convrot_format, the tensors equal the reference
eager quantization of the fp16 weights (the config-1 weight against the
reference goldens), and the file reloads through Int4ConvRotOps's prequantized
path into layers and forward outputs identical to the on-the-fly ones, in
native (comfy_quant tags) and legacy (header map) modes."""
import hashlib
import importlib
import json

import numpy as np
import pytest
import torch

import dit_stack as ds
from inputs import config1_weight

pytestmark = pytest.mark.gpu

INT8_LAYERS = {"double_blocks.0.img_mlp.2", "double_blocks.1.txt_attn.proj"}


def np_of(t):
    t = t.detach().cpu()
    return t.numpy() if t.dtype == torch.float32 else t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _ops():
    from fake_comfy import install_fake_comfy
    install_fake_comfy()
    m = importlib.import_module("comfyui-int4-convrot-rdna4_amd.int4_ops")
    if m.Int4ConvRotOps is None:
        m = importlib.reload(m)
    return m.Int4ConvRotOps


@pytest.fixture(scope="module")
def fmt(gpu):
    return importlib.import_module("comfyui-int4-convrot-rdna4_amd.convrot_format")


@pytest.fixture(scope="module")
def quantized(gpu):
    Ops = _ops()
    Ops.int8_exact = set(INT8_LAYERS)
    try:
        model, ref_sd, _, _ = ds.build_int4_stack(Ops, None, depth=2)
    finally:
        Ops.int8_exact = set()
    return model, ref_sd


def test_saved_tensors_are_the_eager_quantization(quantized, fmt, oracle):
    model, ref_sd = quantized
    sd, prec, _ = fmt.quantized_state_dict(model, native=True)
    assert {k for k, v in prec.items() if v == "int8"} == INT8_LAYERS
    assert len(prec) == 16
    for name in ["double_blocks.0.img_attn.qkv", "double_blocks.0.img_mlp.2", "double_blocks.1.txt_attn.proj"]:
        w16 = np_of(ref_sd[name + ".weight"].to(torch.float16))
        if prec[name] == "int8":
            qw, ws = oracle.quantize_weight8(w16, oracle.F16, 256)
            assert sd[name + ".weight_scale"].shape == (qw.shape[0], 1)
            tag = {"format": "int8_tensorwise", "convrot": True, "convrot_groupsize": 256}
        else:
            qw, ws = oracle.quantize_weight(w16, oracle.F16, 256)
            tag = {"format": "convrot_w4a4", "convrot_groupsize": 256}
        assert np.array_equal(sd[name + ".weight"].numpy(), qw)
        assert np.array_equal(sd[name + ".weight_scale"].reshape(-1).numpy(), ws)
        assert json.loads(bytes(sd[name + ".comfy_quant"].tolist())) == tag
        assert sd[name + ".bias"].dtype == torch.float16
    # bf16 layers are stored as they were loaded
    assert torch.equal(sd["txt_in.weight"], ref_sd["txt_in.weight"].cpu())
    assert sd["txt_in.weight"].dtype == torch.bfloat16


@pytest.mark.parametrize("native_mode", [True, False])
def test_reload_prequantized_identical(quantized, fmt, tmp_path, native_mode):
    model, _ = quantized
    path = str(tmp_path / f"stack_{native_mode}.safetensors")
    counts = fmt.save_quantized(model, path, native=native_mode)
    assert counts["int4"] == 14 and counts["int8"] == 2
    sd, meta = fmt.load_quantized(path)
    assert ("convrot_w4a4" in meta) == (not native_mode)
    Ops = _ops()
    saved = (Ops.enable, list(Ops.excluded_names))
    try:
        Ops.enable, Ops.excluded_names = True, list(ds.FLUX2_EXCLUDED)
        m2 = ds.DoubleStreamDiT(Ops, depth=2, device="cpu")
        m2.load_state_dict(sd, strict=False)
    finally:
        Ops.enable, Ops.excluded_names = saved
    m2 = m2.to("cuda")
    a, b = dict(model.named_modules()), dict(m2.named_modules())
    for name, mod in a.items():
        if not hasattr(mod, "in_features"):
            continue
        other = b[name]
        assert other._qmode == mod._qmode and other._qgs == mod._qgs, name
        if mod._q is not None:
            assert torch.equal(other._q, mod._q) and torch.equal(other._qs, mod._qs), name
            assert (other._q6 is None) == (mod._q6 is None)
            if mod._q6 is not None:
                assert torch.equal(other._q6, mod._q6)
            assert torch.equal(other.bias, mod.bias)
        else:
            assert torch.equal(other.weight, mod.weight)
    img, ctx, t = ds.synthetic_inputs(64, 32, device="cuda")
    with torch.no_grad():
        assert torch.equal(model(img, ctx, t), m2(img, ctx, t))


def test_config1_weight_bytes_match_reference(fmt, goldens, gpu):
    """The saved int4 and int8 tensors of the config-1 weight hash to the
    reference eager quantization's (its Save node writes those tensors)."""
    Ops = _ops()
    parent = torch.nn.Module()
    parent.l4 = Ops.Linear(3072, 3072, bias=False)
    parent.l8 = Ops.Linear(3072, 3072, bias=False)
    w = config1_weight()
    Ops.int8_exact = {"l8"}
    try:
        parent.load_state_dict({"l4.weight": w.clone(), "l8.weight": w.clone()}, strict=False)
    finally:
        Ops.int8_exact = set()
    sd, prec, _ = fmt.quantized_state_dict(parent, native=False)
    assert prec == {"l4": "int4", "l8": "int8"}
    sha = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
    assert sha(sd["l4.weight"].numpy()) == str(goldens["c1_qw_sha"])
    assert np.array_equal(sd["l4.weight_scale"].numpy(), goldens["c1_wscale"])
    assert sha(sd["l8.weight"].numpy()) == str(goldens["i8_c1_qw_sha"])
    assert np.array_equal(sd["l8.weight_scale"].numpy(), goldens["i8_c1_wscale"])
