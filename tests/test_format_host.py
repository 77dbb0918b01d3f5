"""CPU checks of the on-disk format writer/reader (convrot_format): which
tensors a save holds in native and legacy mode, the comfy_quant tag strings,
the header metadata, and a safetensors round trip."""
import importlib
import json

import pytest
import torch

from conftest import import_pkg


@pytest.fixture(scope="module")
def fmt():
    import_pkg()
    return importlib.import_module("comfyui-int4-convrot-rdna4_amd.convrot_format")


def _module():
    """A two-layer module shaped like quantized Linear replacements (plain
    attributes _q/_qs/_qgs/_qmode, no weight parameter) plus a bf16 layer."""
    g = torch.Generator().manual_seed(0)
    m = torch.nn.Module()
    m.a = torch.nn.Module()
    m.a.bias = torch.nn.Parameter(torch.randn(8, generator=g).half(), requires_grad=False)
    m.a._q = torch.randint(-128, 128, (8, 16), generator=g, dtype=torch.int8)      # int4, K = 32
    m.a._qs = torch.rand(8, generator=g)
    m.a._qgs, m.a._qmode = 16, "int4"
    m.b = torch.nn.Module()
    m.b._q = torch.randint(-127, 128, (4, 64), generator=g, dtype=torch.int8)      # int8, K = 64
    m.b._qs = torch.rand(4, generator=g)
    m.b._qgs, m.b._qmode = 64, "int8"
    m.b._dyn_lora = [object()]
    m.c = torch.nn.Linear(4, 4, dtype=torch.bfloat16)
    return m


def test_native_layout(fmt):
    m = _module()
    sd, prec, n_dyn = fmt.quantized_state_dict(m, native=True)
    assert prec == {"a": "int4", "b": "int8"} and n_dyn == 1
    assert set(sd) == {"a.bias", "a.weight", "a.weight_scale", "a.comfy_quant", "b.weight", "b.weight_scale",
                       "b.comfy_quant", "c.weight", "c.bias"}
    assert torch.equal(sd["a.weight"], m.a._q) and sd["a.weight_scale"].shape == (8,)
    assert sd["b.weight_scale"].shape == (4, 1) and sd["b.weight_scale"].dtype == torch.float32
    assert sd["a.bias"].dtype == torch.float16 and sd["c.weight"].dtype == torch.bfloat16
    assert bytes(sd["a.comfy_quant"].tolist()) == b'{"format": "convrot_w4a4", "convrot_groupsize": 16}'
    assert bytes(sd["b.comfy_quant"].tolist()) == \
        b'{"format": "int8_tensorwise", "convrot": true, "convrot_groupsize": 64}'
    assert fmt.format_metadata(prec, native=True, source_metadata={"x": "y", "n": 3}) == {"x": "y"}


def test_legacy_layout(fmt):
    m = _module()
    sd, prec, _ = fmt.quantized_state_dict(m, native=False)
    assert not any(k.endswith("comfy_quant") for k in sd)
    assert sd["b.weight_scale"].shape == (4,)
    meta = fmt.format_metadata(prec, native=False)
    assert meta["convrot_w4a4"] == "2" and json.loads(meta["convrot_precision"]) == {"a": "int4", "b": "int8"}


@pytest.mark.parametrize("native_mode", [True, False])
def test_safetensors_roundtrip(fmt, tmp_path, native_mode):
    native = native_mode
    m = _module()
    path = str(tmp_path / "q.safetensors")
    counts = fmt.save_quantized(m, path, native=native, source_metadata={"modelspec.title": "t"})
    assert counts == {"int4": 1, "int8": 1, "tensors": 9 if native else 7, "dynamic_lora_layers": 1}
    sd, meta = fmt.load_quantized(path)
    ref, _, _ = fmt.quantized_state_dict(m, native=native)
    assert set(sd) == set(ref) and all(torch.equal(sd[k], ref[k]) and sd[k].dtype == ref[k].dtype for k in ref)
    assert meta["modelspec.title"] == "t" and (("convrot_w4a4" in meta) != native)
    # the same state gives the same tensor bytes and the same header (whose
    # metadata map safetensors may serialise in any key order)
    path2 = str(tmp_path / "q2.safetensors")
    fmt.save_quantized(m, path2, native=native, source_metadata={"modelspec.title": "t"})
    f1, f2 = _split(open(path, "rb").read()), _split(open(path2, "rb").read())
    assert f1[0] == f2[0] and f1[1] == f2[1]


def _split(raw):
    """(parsed JSON header, data bytes) of a safetensors file."""
    n = int.from_bytes(raw[:8], "little")
    return json.loads(raw[8:8 + n]), raw[8 + n:]
