"""INT4 ConvRot-W4A4 custom operations for ComfyUI on AMD MI355X (gfx950).

``Int4ConvRotOps`` is the drop-in for the reference's class of the same name
(reference ``int4_ops.py:44-386``): a ``comfy.ops.manual_cast`` subclass whose
``Linear`` quantizes weights to packed int4 at load time (or loads prequantized
ones) and runs the forward through the gfx950 W4A4 kernels.  The class
attributes the loader sets, the per-layer attributes the Save node reads
(``_q``, ``_qs``, ``_qgs``, ``_qmode``, ``_dyn_lora``) and the
``_load_from_state_dict`` dispatch order (prequantized -> LoRA -> quantize ->
plain load) are those of the reference, so its loader and Save nodes use this
class unchanged.
"""
import json
import logging

import torch
import torch.nn as nn

_CK_OK = False
try:
    from . import _int4 as _ck
    from ._int4 import pick_groupsize as _pick_groupsize
    _CK_OK = True
except Exception as e:  # pragma: no cover - import guard keeps ComfyUI booting
    logging.error(f"INT4 ConvRot: gfx950 _int4 backend import failed: {e}")

    def _pick_groupsize(in_features):
        return None

try:
    from comfy.ops import manual_cast
    _COMFY_OPS = True
except Exception:  # pragma: no cover
    _COMFY_OPS = False

try:
    from comfy.weight_adapter.base import WeightAdapterBase as _WA_BASE
except Exception:  # pragma: no cover
    _WA_BASE = None

_KEY_PREFIXES = ("diffusion_model.", "model.diffusion_model.", "model.", "transformer.")


def hip_backend_ready() -> bool:
    return _CK_OK and _ck.is_available()


def _strip_prefix(key):
    if not isinstance(key, str):
        return key
    for p in _KEY_PREFIXES:
        if key.startswith(p):
            return key[len(p):]
    return key


def _patch_fields(patch):
    """(v, offset, function[, strength]) -> (v, offset, function, strength)."""
    if len(patch) == 4:
        return patch
    v, offset, function = patch
    return v, offset, function, 1.0


def _plain_lora(v, in_features, out_features):
    """(down, up, scale) of a plain LoRA adapter, or None.

    A plain LoRA (comfy's LoRAAdapter, ``name == "lora"``) holds
    ``weights = (up [N, r], down [r, K], alpha, mid, dora_scale, reshape)`` and
    its bypass adds ``multiplier * (alpha / r) * up(down(x))`` (reference
    int4_ops.py:181-192).  Adapters with a mid tensor, a DoRA scale, a reshape
    or shapes that do not fit the layer keep the generic ``h()`` side path."""
    if getattr(v, "name", None) != "lora":
        return None
    w = getattr(v, "weights", None)
    if not isinstance(w, (tuple, list)) or len(w) < 3:
        return None
    up, down, alpha = w[0], w[1], w[2]
    if any(len(w) > i and w[i] is not None for i in (3, 4, 5)):
        return None
    if not (isinstance(up, torch.Tensor) and isinstance(down, torch.Tensor)):
        return None
    if down.dim() != 2 or up.dim() != 2:
        return None
    r = down.shape[0]
    if down.shape[1] != in_features or up.shape != (out_features, r) or r == 0:
        return None
    a = float(alpha) if alpha is not None else float(r)
    return down, up, float(getattr(v, "multiplier", 1.0)) * a / r


def _parse_quant_tag(tag):
    """Decode a ComfyUI native ``<key>.comfy_quant`` uint8-JSON tag.

    Returns (accepted, groupsize or None).  Formats the kernels cannot run
    (e.g. fp8, or int8 that is not ConvRot-rotated) are refused."""
    conf = json.loads(bytes(tag.cpu().numpy().tolist()).decode("utf-8"))
    fmt = conf.get("format")
    if fmt not in ("convrot_w4a4", "int8_tensorwise"):
        return False, None
    if fmt == "int8_tensorwise" and not conf.get("convrot", False):
        return False, None
    return True, (int(conf.get("convrot_groupsize", 0)) or None)


if _COMFY_OPS and _CK_OK:

    class Int4ConvRotOps(manual_cast):
        """ComfyUI ops that quantize Linear weights to int4 ConvRot-W4A4."""

        excluded_names = []      # substrings of layer keys kept at bf16
        excluded_exact = set()   # exact normalized keys kept at bf16
        int8_exact = set()       # exact normalized keys quantized to int8
        enable = True            # master toggle
        min_in_features = 512    # narrower linears stay bf16

        lora_patches = {}        # {normalized_layer_key: [(v, offset, function, strength), ...]}
        lora_mode = "None"       # "None" (round) | "Stochastic" (stochastic int4 rounding)
        lora_dynamic = False     # keep LoRA as a forward-time side path on quantized layers
        skeleton_meta_init = False
        _applied_lora = set()
        _STOCHASTIC_SEED = 1234

        class Linear(manual_cast.Linear):
            def __init__(self, in_features, out_features, bias=True, device=None, dtype=None):
                if getattr(Int4ConvRotOps, "skeleton_meta_init", False):
                    # meta-device skeleton used only for LoRA key-map discovery
                    nn.Module.__init__(self)
                    self.in_features = in_features
                    self.out_features = out_features
                    kw = {"device": "meta"}
                    if dtype is not None:
                        kw["dtype"] = dtype
                    self.weight = nn.Parameter(torch.empty((out_features, in_features), **kw),
                                               requires_grad=False)
                    self.bias = (nn.Parameter(torch.empty((out_features,), **kw), requires_grad=False)
                                 if bias else None)
                else:
                    super().__init__(in_features, out_features, bias, device, dtype)
                self._q = None        # int8: packed [N, K/2] (int4) or plain [N, K] (int8)
                self._qs = None       # per-row scale f32 [N]
                self._qgs = None      # convrot groupsize
                self._qmode = None    # "int4" | "int8" | None (bf16)
                self._q6 = None       # int4 weight re-encoded for the bf6 matrix-core GEMM (load time)
                self._q8t = None      # int8 weight re-laid for the tile-major W8A8 GEMM (load time)
                self._dyn_lora = None
                self._dyn_fused = None   # (D, U) bf16: plain LoRAs fused into the GEMM epilogue
                self._dyn_rest = None    # adapters that keep the generic h() side path
                self.comfy_cast_weights = False

            _normalize_lora_key = staticmethod(_strip_prefix)

            @staticmethod
            def _format_lora_patches(patches):
                """-> (strength, v, key_strength, offset, function) tuples of comfy.lora."""
                out = []
                for p in patches or []:
                    v, offset, function, strength = _patch_fields(p)
                    out.append((strength, v, 1.0, offset, function))
                return out

            def _apply_lora(self, tensor, key):
                """Fold the LoRA patches registered for `key` into `tensor`."""
                if tensor is None or tensor.dtype == torch.int8 or not Int4ConvRotOps.lora_patches:
                    return tensor
                nk = _strip_prefix(key)
                patches = Int4ConvRotOps.lora_patches.get(nk)
                if not patches:
                    return tensor
                import comfy.lora
                import comfy.model_management
                dev = tensor.device
                if dev.type == "cpu" and torch.cuda.is_available():
                    dev = torch.device("cuda")
                t = tensor.to(device=dev, dtype=comfy.model_management.lora_compute_dtype(dev))
                merged = comfy.lora.calculate_weight(self._format_lora_patches(patches), t, key)
                Int4ConvRotOps._applied_lora.add(nk)
                return merged.to(dtype=tensor.dtype)

            @staticmethod
            def _dyn_capable(v):
                """True for adapters with an additive bypass h(x) (LoRA/LoHa/LoKr),
                false for raw diff/set patches, DoRA and OFT/BOFT."""
                if not hasattr(v, "weights") or not hasattr(v, "h"):
                    return False
                if _WA_BASE is not None and type(v).h is _WA_BASE.h:
                    return False
                w = getattr(v, "weights", None)
                is_dora = (getattr(v, "name", None) == "lora" and isinstance(w, (tuple, list))
                           and len(w) > 4 and w[4] is not None)
                return not is_dora

            def _prepare_dyn_adapters(self, patches):
                """Turn patches into forward-time bypass adapters (fp16 on the GPU).
                Returns None when one of them cannot run as a side path."""
                prepared = []
                for p in patches or []:
                    v, _offset, _function, strength = _patch_fields(p)
                    if not self._dyn_capable(v):
                        return None
                    w = getattr(v, "weights", None)
                    if isinstance(w, (tuple, list)):
                        v.weights = tuple(
                            t.to(device="cuda", dtype=torch.float16)
                            if isinstance(t, torch.Tensor) and t.is_floating_point() else t
                            for t in w)
                    # the attributes comfy's BypassForwardHook would set for a Linear
                    v.multiplier = float(strength)
                    v.is_conv = False
                    v.conv_dim = 0
                    v.kernel_size = (1,)
                    v.in_channels = None
                    v.out_channels = None
                    v.kw_dict = {}
                    prepared.append(v)
                return prepared

            def _set_dyn_lora(self, prepared):
                """Attach prepared adapters; the plain LoRAs among them are
                concatenated into one (D, U) pair that the W4A4 GEMM applies in
                its epilogue, the others keep their h() side path."""
                self._dyn_lora = prepared
                self._dyn_fused, self._dyn_rest = None, prepared
                plain = [_plain_lora(v, self.in_features, self.out_features) for v in prepared]
                if not any(p is not None for p in plain):
                    return
                try:
                    fused = _ck.fuse_lora_pairs([p for p in plain if p is not None])
                except Exception as e:
                    logging.warning(f"INT4 ConvRot: LoRA fusion failed, using the side path: {e}")
                    fused = None
                if fused is not None:
                    self._dyn_fused = fused
                    self._dyn_rest = [v for v, p in zip(prepared, plain) if p is None]

            def _apply_dyn_lora(self, x, out, adapters=None):
                """out + sum of the attached adapters' h(x) (already scaled)."""
                for v in (self._dyn_lora if adapters is None else adapters) or ():
                    try:
                        out = out + v.h(x, out)
                    except Exception as e:
                        logging.warning(f"INT4 ConvRot: dynamic LoRA side-path failed: {e}")
                return out

            @staticmethod
            def _exact_key(prefix):
                return _strip_prefix(prefix[:-1] if prefix.endswith(".") else prefix)

            def _should_quantize(self, prefix, w):
                if not Int4ConvRotOps.enable or w is None or w.dim() != 2:
                    return False
                if self.in_features < Int4ConvRotOps.min_in_features:
                    return False
                if _pick_groupsize(self.in_features) is None:
                    return False
                if any(n in prefix for n in (Int4ConvRotOps.excluded_names or [])):
                    return False
                return self._exact_key(prefix) not in Int4ConvRotOps.excluded_exact

            def _quant_mode(self, prefix):
                return "int8" if self._exact_key(prefix) in Int4ConvRotOps.int8_exact else "int4"

            def _take_bias(self, state_dict, prefix, dev):
                bkey = prefix + "bias"
                if bkey in state_dict:
                    self.bias = nn.Parameter(state_dict.pop(bkey).to(dev, torch.float16),
                                             requires_grad=False)

            def _attach_dyn_lora(self, wkey):
                nk = _strip_prefix(wkey)
                patches = Int4ConvRotOps.lora_patches.get(nk)
                if patches:
                    prepared = self._prepare_dyn_adapters(patches)
                    if prepared is not None:
                        self._set_dyn_lora(prepared)
                        Int4ConvRotOps._applied_lora.add(nk)

            def _load_prequantized(self, state_dict, prefix, wkey, skey, w):
                """Load a packed int4 (cols == K/2) or int8 (cols == K) ConvRot
                weight as stored (legacy header files or ComfyUI native files
                with a comfy_quant tag).  Returns True if consumed."""
                cols = w.shape[-1]
                if cols == self.in_features:
                    mode = "int8"
                elif cols * 2 == self.in_features:
                    mode = "int4"
                else:
                    return False
                qkey = prefix + "comfy_quant"
                gs = None
                tag = state_dict.get(qkey, None)
                if tag is not None:
                    try:
                        ok, gs = _parse_quant_tag(tag)
                        if not ok:
                            return False
                    except Exception:
                        gs = None
                if gs is None:
                    gs = _pick_groupsize(self.in_features)
                if gs is None:
                    return False
                dev = torch.device("cuda")
                self._q = w.to(dev).contiguous()
                self._qs = state_dict[skey].to(dev, torch.float32).reshape(-1).contiguous()
                self._qgs, self._qmode = gs, mode
                self._q6 = _ck.prepare_convrot_w4a4_weight_bf6(self._q) if mode == "int4" else None
                self._q8t = _ck.prepare_convrot_w8a8_weight_i8t(self._q) if mode == "int8" else None
                self.weight = None
                for k in (wkey, skey, qkey):
                    state_dict.pop(k, None)
                self._take_bias(state_dict, prefix, dev)
                if Int4ConvRotOps.lora_dynamic and Int4ConvRotOps.lora_patches:
                    self._attach_dyn_lora(wkey)
                return True

            def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict,
                                      missing_keys, unexpected_keys, error_msgs):
                wkey, skey = prefix + "weight", prefix + "weight_scale"
                w = state_dict.get(wkey, None)

                # (1) prequantized checkpoint
                if w is not None and w.dtype == torch.int8 and skey in state_dict:
                    try:
                        if self._load_prequantized(state_dict, prefix, wkey, skey, w):
                            return
                    except Exception as e:
                        logging.warning(f"INT4 ConvRot: prequant load failed for {prefix}, "
                                        f"falling back to bf16: {e}")

                # LoRA: dynamic side path for layers that will be quantized, else bake
                if Int4ConvRotOps.lora_patches:
                    nk = _strip_prefix(wkey)
                    wpatches = Int4ConvRotOps.lora_patches.get(nk)
                    prepared = None
                    if (Int4ConvRotOps.lora_dynamic and wpatches and w is not None
                            and w.dtype != torch.int8 and self._should_quantize(prefix, w)):
                        prepared = self._prepare_dyn_adapters(wpatches)
                    if prepared is not None:
                        self._set_dyn_lora(prepared)
                        Int4ConvRotOps._applied_lora.add(nk)
                    else:
                        if w is not None and w.dtype != torch.int8:
                            wp = self._apply_lora(w, wkey)
                            if wp is not w:
                                w = wp
                                state_dict[wkey] = w
                        bkey = prefix + "bias"
                        b = state_dict.get(bkey, None)
                        if b is not None:
                            bp = self._apply_lora(b, bkey)
                            if bp is not b:
                                state_dict[bkey] = bp

                # (2) quantize on the fly from an fp16 copy on the GPU
                if self._should_quantize(prefix, w):
                    dev = torch.device("cuda")
                    gs = _pick_groupsize(self.in_features)
                    mode = self._quant_mode(prefix)
                    try:
                        if mode == "int8":
                            from ._int4.int8_eager import quantize_convrot_w8a8_weight
                            qw, ws = quantize_convrot_w8a8_weight(w.to(dev, torch.float16), convrot_groupsize=gs)
                        else:
                            stoch = (Int4ConvRotOps._STOCHASTIC_SEED
                                     if Int4ConvRotOps.lora_mode == "Stochastic" else 0)
                            qw, ws = _ck.quantize_convrot_w4a4_weight(
                                w.to(dev, torch.float16), convrot_groupsize=gs, stochastic_rounding=stoch)
                        self._q, self._qs, self._qgs, self._qmode = qw, ws.float(), gs, mode
                        self._q6 = _ck.prepare_convrot_w4a4_weight_bf6(qw) if mode == "int4" else None
                        self._q8t = _ck.prepare_convrot_w8a8_weight_i8t(qw) if mode == "int8" else None
                        self.weight = None
                        state_dict.pop(wkey, None)
                        self._take_bias(state_dict, prefix, dev)
                        return
                    except Exception as e:
                        logging.warning(f"INT4 ConvRot: fell back to bf16 for {prefix}: {e}")

                # (3) plain load
                return super()._load_from_state_dict(
                    state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys, error_msgs)

            def forward(self, x):
                if self._q is None:
                    return self._apply_dyn_lora(x, super().forward(x))
                if self._q.device != x.device:
                    self._q = self._q.to(x.device)
                    self._qs = self._qs.to(x.device)
                    if self._q6 is not None:
                        self._q6 = self._q6.to(x.device)
                    if self._q8t is not None:
                        self._q8t = self._q8t.to(x.device)
                bias = self.bias
                if bias is not None and bias.device != x.device:
                    bias = bias.to(x.device)
                if self._qmode == "int8":
                    out = _ck.convrot_w8a8_linear(x, self._q, self._qs, bias=bias,
                                                  convrot_groupsize=self._qgs, qweight_i8t=self._q8t)
                    return self._apply_dyn_lora(x, out)
                fused = self._dyn_fused
                if fused is not None and fused[0].device != x.device:
                    fused = self._dyn_fused = (fused[0].to(x.device), fused[1].to(x.device))
                out = _ck.convrot_w4a4_linear(x, self._q, self._qs, bias=bias, convrot_groupsize=self._qgs,
                                              lora=fused, qweight_bf6=self._q6)
                return self._apply_dyn_lora(x, out, self._dyn_rest if fused is not None else None)

else:  # comfy.ops or the backend unavailable
    Int4ConvRotOps = None
