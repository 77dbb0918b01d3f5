"""The names the reference's ComfyUI nodes import from this package exist, and
accept the arguments those nodes pass them (CPU only; the reference is not
imported: its import statements and call sites are listed here by hand).

Every import the reference's node files make into the backend:
  int4_loader.py:15          from .int4_ops import Int4ConvRotOps, _pick_groupsize, hip_backend_ready
  int4_ops.py:16-17          from . import _int4; from ._int4 import pick_groupsize
  int4_ops.py:340            from ._int4.int8_eager import quantize_convrot_w8a8_weight
  int4_ops.py:344            from ._int4 import quantize_convrot_w4a4_weight
  int4_ops.py:376,380        from ._int4 import convrot_w8a8_linear / convrot_w4a4_linear
  int4_sensitivity.py:43-46  from ._int4.eager import quantize_convrot_w4a4_weight, dequantize_convrot_w4a4_weight
  int4_sensitivity.py:67-70  from ._int4.int8_eager import quantize_convrot_w8a8_weight, dequantize_convrot_w8a8_weight
  int4_sensitivity.py:95-98  from ._int4 import convrot_w4a4_linear, convrot_w8a8_linear, quantize_convrot_w4a4_weight
                             from ._int4.int8_eager import quantize_convrot_w8a8_weight
"""
import importlib
import inspect

import pytest
import torch

from conftest import PKG_NAME, import_pkg
from fake_comfy import install_fake_comfy

IMPORTS = {
    "int4_ops": ["Int4ConvRotOps", "_pick_groupsize", "hip_backend_ready"],
    "_int4": ["pick_groupsize", "quantize_convrot_w4a4_weight", "convrot_w4a4_linear", "convrot_w8a8_linear",
              "dequantize_convrot_w4a4_weight", "is_available"],
    "_int4.int8_eager": ["quantize_convrot_w8a8_weight", "dequantize_convrot_w8a8_weight"],
    "_int4.eager": ["quantize_convrot_w4a4_weight", "dequantize_convrot_w4a4_weight"],
}


def _module(name):
    install_fake_comfy()
    import_pkg()
    return importlib.import_module(PKG_NAME + "." + name)


@pytest.mark.parametrize("mod", sorted(IMPORTS))
def test_every_imported_name_exists(mod):
    m = _module(mod)
    for name in IMPORTS[mod]:
        assert hasattr(m, name), f"{mod}.{name}"
    if mod == "int4_ops":
        assert m.Int4ConvRotOps is not None     # built against the comfy.ops stand-in


W = torch.zeros(4, 256)
Q = torch.zeros(4, 128, dtype=torch.int8)
S = torch.zeros(4)

# (module, function, args, kwargs) exactly as the reference's nodes call them
CALLS = [
    ("_int4", "quantize_convrot_w4a4_weight", (W,), {"convrot_groupsize": 256, "stochastic_rounding": 0}),  # int4_ops.py:347-349
    ("_int4.int8_eager", "quantize_convrot_w8a8_weight", (W,), {"convrot_groupsize": 256}),                # int4_ops.py:341-342
    ("_int4", "convrot_w8a8_linear", (W, Q, S), {"bias": None, "convrot_groupsize": 256}),                  # int4_ops.py:377-378
    ("_int4", "convrot_w4a4_linear", (W, Q, S), {"bias": None, "convrot_groupsize": 256}),                  # int4_ops.py:381-382
    ("_int4.eager", "quantize_convrot_w4a4_weight", (W,), {"convrot_groupsize": 256}),                      # int4_sensitivity.py:52-53
    ("_int4.eager", "dequantize_convrot_w4a4_weight", (Q, S),
     {"convrot_groupsize": 256, "output_dtype": torch.float32}),                                           # int4_sensitivity.py:54-55
    ("_int4.int8_eager", "quantize_convrot_w8a8_weight", (W,), {"convrot_groupsize": 256}),                # int4_sensitivity.py:76
    ("_int4.int8_eager", "dequantize_convrot_w8a8_weight", (Q, S),
     {"convrot_groupsize": 256, "output_dtype": torch.float32}),                                           # int4_sensitivity.py:77-78
    ("_int4", "quantize_convrot_w4a4_weight", (W,), {"convrot_groupsize": 256}),                            # int4_sensitivity.py:107
    ("_int4", "convrot_w4a4_linear", (W, Q, S), {"convrot_groupsize": 256}),                                # int4_sensitivity.py:108
    ("_int4.int8_eager", "quantize_convrot_w8a8_weight", (W, 256), {}),                                    # int4_sensitivity.py:109
    ("_int4", "convrot_w8a8_linear", (W, Q, S), {"convrot_groupsize": 256}),                                # int4_sensitivity.py:110
]


@pytest.mark.parametrize("mod,fn,args,kwargs", CALLS, ids=[f"{m}.{f}" for m, f, _, _ in CALLS])
def test_node_call_sites_bind(mod, fn, args, kwargs):
    sig = inspect.signature(getattr(_module(mod), fn))
    sig.bind(*args, **kwargs)


def test_eager_module_runs_the_gpu_quantizer_not_a_torch_restatement():
    """``_int4.eager`` hands out the package's kernel-backed functions."""
    eager, pkg = _module("_int4.eager"), _module("_int4")
    assert eager.quantize_convrot_w4a4_weight is pkg.quantize_convrot_w4a4_weight
    assert eager.dequantize_convrot_w4a4_weight is pkg.dequantize_convrot_w4a4_weight
    assert eager.validate_w4a4_shape is pkg.validate_w4a4_shape


def test_eager_module_validates_like_the_reference():
    """Argument errors raise the reference's ValueErrors before any device work
    (reference _int4/eager.py:82-89,130-131,180-189)."""
    eager = _module("_int4.eager")
    with pytest.raises(ValueError, match="linear_dtype"):
        eager.convrot_w4a4_linear(W, Q, S, linear_dtype="fp8")
    with pytest.raises(ValueError, match="quant_group_size"):
        eager.convrot_w4a4_linear(W, Q, S, quant_group_size=32)
    with pytest.raises(ValueError, match="does not match qweight"):
        eager.convrot_w4a4_linear(torch.zeros(4, 512), Q, S)
    with pytest.raises(ValueError, match="2D"):
        eager.quantize_convrot_w4a4_weight(torch.zeros(256))
    with pytest.raises(ValueError, match="not divisible by convrot_groupsize"):
        eager.quantize_convrot_w4a4_weight(torch.zeros(4, 320), convrot_groupsize=256)
    with pytest.raises(ValueError, match="quant_group_size"):
        eager.dequantize_convrot_w4a4_weight(Q, S, quant_group_size=128)
