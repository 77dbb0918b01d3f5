"""On-disk format of ConvRot-quantized diffusion models (.safetensors).

The layout the reference's Save node writes and its loader reads back without
re-quantizing (reference int4_save.py:1-16 format description, :97-158 the
writer; int4_ops.py:223-284 the prequantized load that
``Int4ConvRotOps.Linear._load_from_state_dict`` mirrors):

* int4 layer:  ``<key>.weight``        int8 [N, K/2]  two signed nibbles per byte
               ``<key>.weight_scale``  f32  [N]
* int8 layer:  ``<key>.weight``        int8 [N, K]    plain signed int8
               ``<key>.weight_scale``  f32  [N] (legacy) / [N, 1] (native)
* native mode: ``<key>.comfy_quant``   uint8 JSON tag per quantized layer:
  ``{"format": "convrot_w4a4", "convrot_groupsize": G}`` or
  ``{"format": "int8_tensorwise", "convrot": true, "convrot_groupsize": G}``
* legacy mode: header metadata ``convrot_w4a4 = "2"`` and
  ``convrot_precision = {layer: "int4" | "int8"}`` (JSON)
* everything else (bf16 layers, norms, biases -- fp16 on quantized layers)
  as the module holds it.

The packed codes and scales are the ones the load-time GPU quantizer produced
from the fp16 weight (int4_ops.py:339-350 semantics), which equal the
reference eager path's bit for bit, so a file written from this package holds
the same tensors as one written from the reference.  The names, dtypes, shapes
and tag strings are alike because they are the file format.  Writing uses
safetensors' ``save_file`` (what ``comfy.utils.save_torch_file`` calls).
"""
from __future__ import annotations

import json

import torch

FORMAT_TAG = "convrot_w4a4"
FORMAT_VERSION = "2"
PRECISION_TAG = "convrot_precision"


def _quant_tag(mode: str, groupsize: int) -> torch.Tensor:
    if mode == "int8":
        conf = {"format": "int8_tensorwise", "convrot": True, "convrot_groupsize": groupsize}
    else:
        conf = {"format": "convrot_w4a4", "convrot_groupsize": groupsize}
    return torch.tensor(list(json.dumps(conf).encode("utf-8")), dtype=torch.uint8)


def quantized_state_dict(module: torch.nn.Module, native: bool = True):
    """The tensors a save of ``module`` writes (reference int4_save.py:97-137).

    Returns (state dict of CPU tensors, {layer: "int4" | "int8"}, number of
    layers that carry a dynamic LoRA side path, which is not written)."""
    sd = {}
    for k, v in module.state_dict().items():
        if isinstance(v, torch.Tensor):
            sd[k] = v.detach().to("cpu").contiguous()
    precision = {}
    n_dyn = 0
    for name, sub in module.named_modules():
        if getattr(sub, "_dyn_lora", None):
            n_dyn += 1
        q = getattr(sub, "_q", None)
        if q is None:
            continue
        mode = getattr(sub, "_qmode", None) or "int4"
        gs = int(getattr(sub, "_qgs", None) or 256)
        scale = sub._qs.detach().float().to("cpu").contiguous()
        sd[name + ".weight"] = q.detach().to("cpu").contiguous()
        if native:
            if mode == "int8":
                scale = scale.reshape(-1, 1).contiguous()
            sd[name + ".comfy_quant"] = _quant_tag(mode, gs)
        sd[name + ".weight_scale"] = scale
        precision[name] = mode
    return sd, precision, n_dyn


def format_metadata(precision: dict, native: bool = True, source_metadata: dict | None = None) -> dict:
    """Header metadata (reference int4_save.py:146-153): the source file's
    string entries, plus the format markers in legacy mode."""
    meta = {k: v for k, v in (source_metadata or {}).items() if isinstance(k, str) and isinstance(v, str)}
    if not native:
        meta[FORMAT_TAG] = FORMAT_VERSION
        meta[PRECISION_TAG] = json.dumps(precision)
    return meta


def save_quantized(module: torch.nn.Module, path: str, native: bool = True,
                   source_metadata: dict | None = None) -> dict:
    """Write ``module``'s quantized state to ``path`` (.safetensors).  Returns
    {"int4": n, "int8": n, "tensors": n, "dynamic_lora_layers": n}."""
    from safetensors.torch import save_file

    sd, precision, n_dyn = quantized_state_dict(module, native)
    save_file(sd, path, metadata=format_metadata(precision, native, source_metadata))
    modes = list(precision.values())
    return {"int4": modes.count("int4"), "int8": modes.count("int8"), "tensors": len(sd),
            "dynamic_lora_layers": n_dyn}


def load_quantized(path: str):
    """(state dict, metadata) of a saved file, read with safetensors (nothing in
    the file is executed).  Legacy files need no metadata on load: int4 vs
    int8 follows from the stored column count (K/2 vs K)."""
    from safetensors import safe_open

    sd = {}
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        for k in f.keys():
            sd[k] = f.get_tensor(k)
    return sd, meta
