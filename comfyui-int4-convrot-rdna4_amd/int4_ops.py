"""INT4 ConvRot-W4A4 custom operations for ComfyUI on AMD MI355X (gfx950).

``Int4ConvRotOps`` is the drop-in for the reference's class of the same name
(reference ``int4_ops.py:44-386``).  What the interface fixes is kept: the
``comfy.ops.manual_cast`` base, the class attributes the loader sets
(``int4_loader.py:221-259``), the per-layer attributes the Save node reads
(``_q``, ``_qs``, ``_qgs``, ``_qmode``, ``_dyn_lora``; ``int4_save.py:110-130``),
the method names other code calls, and the order in which a layer's state is
resolved at load time:

  1. a prequantized weight (int8 tensor + ``weight_scale``) is taken as stored;
  2. LoRA patches for the layer either stay a forward-time bypass (dynamic mode,
     layers that will be quantized) or are folded into the float weight/bias;
  3. an eligible float weight is quantized on the GPU from its fp16 copy;
  4. anything else loads as a plain ``manual_cast`` layer.

The forward runs every quantized layer through the gfx950 kernels of
``_int4`` (one library call per linear); plain LoRA bypasses are concatenated
into one low-rank pair that the GEMM epilogue adds.
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

# container prefixes stripped from state-dict keys before they are matched
# against LoRA key maps and the loader's exact-key sets
_KEY_PREFIXES = ("diffusion_model.", "model.diffusion_model.", "model.", "transformer.")

# the attributes ComfyUI's BypassForwardHook gives an adapter wrapped around a
# Linear; h() reads them
_LINEAR_BYPASS_ATTRS = {"is_conv": False, "conv_dim": 0, "kernel_size": (1,), "in_channels": None,
                        "out_channels": None, "kw_dict": {}}


def hip_backend_ready() -> bool:
    return _CK_OK and _ck.is_available()


def _strip_prefix(key):
    if isinstance(key, str):
        for p in _KEY_PREFIXES:
            if key.startswith(p):
                return key[len(p):]
    return key


def _patch_fields(patch):
    """(v, offset, function[, strength]) -> (v, offset, function, strength)."""
    v, offset, function, *rest = patch
    return v, offset, function, (rest[0] if rest else 1.0)


def _has_additive_bypass(v) -> bool:
    """Whether adapter v adds a term h(x) to the layer output without needing
    the base weight: LoRA / LoHa / LoKr do; raw diff/set tuples, adapters
    that keep the base class's zero h() (OFT/BOFT) and DoRA (a LoRA with a
    dora_scale) do not."""
    if not (hasattr(v, "weights") and hasattr(v, "h")):
        return False
    if _WA_BASE is not None and type(v).h is _WA_BASE.h:
        return False
    w = v.weights
    dora = getattr(v, "name", None) == "lora" and isinstance(w, (tuple, list)) and len(w) > 4 \
        and w[4] is not None
    return not dora


def _arm_bypass(v, strength):
    """Make adapter v callable as a Linear bypass: its float tensors in fp16 on
    the GPU, and the attributes h() reads."""
    w = v.weights
    if isinstance(w, (tuple, list)):
        v.weights = tuple(t.to("cuda", torch.float16) if torch.is_tensor(t) and t.is_floating_point() else t
                          for t in w)
    v.multiplier = float(strength)
    for name, value in _LINEAR_BYPASS_ATTRS.items():
        setattr(v, name, value)
    return v


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


class _Keys:
    """The state-dict keys of one layer."""
    __slots__ = ("prefix", "weight", "scale", "bias", "tag")

    def __init__(self, prefix):
        self.prefix = prefix
        self.weight, self.scale = prefix + "weight", prefix + "weight_scale"
        self.bias, self.tag = prefix + "bias", prefix + "comfy_quant"


def _meta_skeleton(mod, in_features, out_features, bias, dtype):
    """A Linear with meta-device parameters: the loader builds the model this
    way only to discover the LoRA key map, so no storage is allocated."""
    nn.Module.__init__(mod)
    mod.in_features, mod.out_features = in_features, out_features
    spec = {"device": "meta"} if dtype is None else {"device": "meta", "dtype": dtype}
    shapes = [("weight", (out_features, in_features))] + ([("bias", (out_features,))] if bias else [])
    for name, shape in shapes:
        setattr(mod, name, nn.Parameter(torch.empty(shape, **spec), requires_grad=False))
    if not bias:
        mod.bias = None


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
                if Int4ConvRotOps.skeleton_meta_init:
                    _meta_skeleton(self, in_features, out_features, bias, dtype)
                else:
                    super().__init__(in_features, out_features, bias, device, dtype)
                # quantized storage (None: a plain layer); see the _q property
                self._q = self._qs = self._qgs = self._qmode = None
                self._q6 = None       # int4 weight as the bf6 GEMM's operand (made at load time)
                self._q8t = None      # int8 weight as the tile-major W8A8 GEMM's operand
                self._qshape = None   # shape stand-in of _q (meta device) for the linear's checks
                # dynamic LoRA: every attached adapter, the plain ones fused into one
                # (D, U) pair for the GEMM epilogue, and the rest (h() side path)
                self._dyn_lora = self._dyn_fused = self._dyn_rest = None
                self.comfy_cast_weights = False

            # One copy of a quantized weight stays on the device: the GEMM's
            # operand.  When that is the B6T (int4) or I8T (int8) tile layout,
            # `_q`, the checkpoint layout (packed int4 [N, K/2] or int8 [N, K])
            # that the Save node reads (int4_save.py:113-119), is decoded from it
            # on each read, bit for bit, on the operand's device; otherwise the
            # checkpoint layout is the operand itself (`_qpack`).
            @property
            def _q(self):
                if self._qpack is not None:
                    return self._qpack
                if self._q6 is not None:
                    return _ck.native.bf6_to_int4(self._q6, self.out_features, self.in_features)
                if self._q8t is not None:
                    return _ck.native.i8t_to_int8(self._q8t, self.out_features)
                return None

            @_q.setter
            def _q(self, value):
                self._qpack = value
                self._q6 = self._q8t = None

            _normalize_lora_key = staticmethod(_strip_prefix)

            @staticmethod
            def _format_lora_patches(patches):
                """-> the (strength, v, key_strength, offset, function) entries
                comfy.lora.calculate_weight takes."""
                return [(s, v, 1.0, off, fn) for v, off, fn, s in map(_patch_fields, patches or [])]

            @staticmethod
            def _patches_for(key):
                nk = _strip_prefix(key)
                return nk, Int4ConvRotOps.lora_patches.get(nk)

            def _apply_lora(self, tensor, key):
                """`tensor` with the LoRA patches registered for `key` folded in
                (the same tensor object when there are none)."""
                nk, patches = self._patches_for(key)
                if tensor is None or tensor.dtype == torch.int8 or not patches:
                    return tensor
                import comfy.lora
                import comfy.model_management
                dev = torch.device("cuda") if tensor.device.type == "cpu" and torch.cuda.is_available() \
                    else tensor.device
                work = tensor.to(dev, comfy.model_management.lora_compute_dtype(dev))
                baked = comfy.lora.calculate_weight(self._format_lora_patches(patches), work, key)
                Int4ConvRotOps._applied_lora.add(nk)
                return baked.to(tensor.dtype)

            _dyn_capable = staticmethod(_has_additive_bypass)

            def _prepare_dyn_adapters(self, patches):
                """The patches as armed bypass adapters, or None when one of them
                has no additive bypass (the layer then bakes instead)."""
                fields = [_patch_fields(p) for p in patches or []]
                if not all(_has_additive_bypass(v) for v, *_ in fields):
                    return None
                return [_arm_bypass(v, strength) for v, _, _, strength in fields]

            def _set_dyn_lora(self, prepared):
                """Attach prepared adapters; the plain LoRAs among them are
                concatenated into one (D, U) pair that the W4A4 GEMM applies in
                its epilogue, the others keep their h() side path."""
                self._dyn_lora = prepared
                self._dyn_fused, self._dyn_rest = None, prepared
                plain = [_plain_lora(v, self.in_features, self.out_features) for v in prepared]
                if all(p is None for p in plain):
                    return
                try:
                    fused = _ck.fuse_lora_pairs([p for p in plain if p is not None])
                except Exception as e:
                    logging.warning(f"INT4 ConvRot: LoRA fusion failed, using the side path: {e}")
                    fused = None
                if fused is not None:
                    self._dyn_fused = fused
                    self._dyn_rest = [v for v, p in zip(prepared, plain) if p is None]

            def _attach_dyn_lora(self, wkey, patches=None):
                """Attach the layer's patches as bypass adapters.  Returns False
                when they cannot all run that way."""
                nk, found = self._patches_for(wkey)
                patches = found if patches is None else patches
                prepared = self._prepare_dyn_adapters(patches) if patches else None
                if prepared is None:
                    return False
                self._set_dyn_lora(prepared)
                Int4ConvRotOps._applied_lora.add(nk)
                return True

            def _apply_dyn_lora(self, x, out, adapters=None):
                """out plus each adapter's bypass term h(x) (already scaled)."""
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
                ops = Int4ConvRotOps
                eligible = (ops.enable and w is not None and w.dim() == 2
                            and self.in_features >= ops.min_in_features
                            and _pick_groupsize(self.in_features) is not None
                            and self.in_features <= _ck.max_quant_k())
                if not eligible or any(n in prefix for n in ops.excluded_names or ()):
                    return False
                return self._exact_key(prefix) not in ops.excluded_exact

            def _quant_mode(self, prefix):
                return "int8" if self._exact_key(prefix) in Int4ConvRotOps.int8_exact else "int4"

            # -- load-time state ------------------------------------------------

            def _install(self, q, scale, groupsize, mode, state_dict, keys, consumed):
                """Take over quantized storage (on the GPU): the GEMM operand
                made from the checkpoint-layout codes `q` (which are dropped
                when the operand is a tile layout), the scales, and the bias in
                fp16; the `consumed` keys leave state_dict."""
                dev = torch.device("cuda")
                q = q.to(dev).contiguous()
                self._qs = scale.to(dev, torch.float32).reshape(-1).contiguous()
                self._qgs, self._qmode = groupsize, mode
                q6 = _ck.prepare_convrot_w4a4_weight_bf6(q) if mode == "int4" else None
                q8t = _ck.prepare_convrot_w8a8_weight_i8t(q) if mode == "int8" else None
                self._q = q if q6 is None and q8t is None else None
                self._q6, self._q8t = q6, q8t
                self._qshape = torch.empty(tuple(q.shape), dtype=torch.int8, device="meta")
                self.weight = None
                for k in consumed:
                    state_dict.pop(k, None)
                if keys.bias in state_dict:
                    self.bias = nn.Parameter(state_dict.pop(keys.bias).to(dev, torch.float16), requires_grad=False)

            def _load_prequantized(self, state_dict, prefix, wkey, skey, w):
                """Load a packed int4 (cols == K/2) or int8 (cols == K) ConvRot
                weight as stored (legacy header files or ComfyUI native files
                with a comfy_quant tag).  Returns True if consumed."""
                cols = w.shape[-1]
                mode = "int8" if cols == self.in_features else "int4" if 2 * cols == self.in_features else None
                if mode is None:
                    return False
                keys = _Keys(prefix)
                groupsize = None
                if keys.tag in state_dict:
                    try:
                        accepted, groupsize = _parse_quant_tag(state_dict[keys.tag])
                    except Exception:
                        accepted = True          # unreadable tag: decide from in_features
                    if not accepted:
                        return False
                groupsize = groupsize or _pick_groupsize(self.in_features)
                if groupsize is None:
                    return False
                if self.in_features > _ck.max_quant_k():
                    # rows too wide for the fused quantizer: keep the layer in bf16,
                    # from the stored codes (the reference rotates such rows with torch)
                    logging.warning(f"INT4 ConvRot: {prefix} has in_features {self.in_features} above "
                                    f"{_ck.max_quant_k()}; loading it dequantized in bf16")
                    from ._int4.int8_eager import dequantize_convrot_w8a8_weight
                    deq = (_ck.dequantize_convrot_w4a4_weight(w, state_dict[skey], groupsize) if mode == "int4" else
                           dequantize_convrot_w8a8_weight(w, state_dict[skey], groupsize))
                    state_dict[wkey] = deq.to(torch.bfloat16)
                    for k in (keys.scale, keys.tag):
                        state_dict.pop(k, None)
                    return False
                self._install(w, state_dict[skey], groupsize, mode, state_dict, keys,
                              (keys.weight, keys.scale, keys.tag))
                if Int4ConvRotOps.lora_dynamic and Int4ConvRotOps.lora_patches:
                    self._attach_dyn_lora(wkey)
                return True

            def _take_prequantized(self, state_dict, keys, w):
                if w is None or w.dtype != torch.int8 or keys.scale not in state_dict:
                    return False
                try:
                    return self._load_prequantized(state_dict, keys.prefix, keys.weight, keys.scale, w)
                except Exception as e:
                    logging.warning(f"INT4 ConvRot: prequant load failed for {keys.prefix}, "
                                    f"falling back to bf16: {e}")
                    return False

            def _route_lora(self, state_dict, keys, w):
                """Dynamic bypass for a layer about to be quantized, else fold
                the patches into the float weight and bias in state_dict.
                Returns the (possibly patched) weight."""
                if not Int4ConvRotOps.lora_patches:
                    return w
                _, patches = self._patches_for(keys.weight)
                floating = w is not None and w.dtype != torch.int8
                if (Int4ConvRotOps.lora_dynamic and patches and floating
                        and self._should_quantize(keys.prefix, w) and self._attach_dyn_lora(keys.weight, patches)):
                    return w
                for key, t in ((keys.weight, w if floating else None), (keys.bias, state_dict.get(keys.bias))):
                    patched = self._apply_lora(t, key)
                    if patched is not t:
                        state_dict[key] = patched
                return state_dict.get(keys.weight, w)

            def _quantize_on_load(self, state_dict, keys, w):
                if not self._should_quantize(keys.prefix, w):
                    if Int4ConvRotOps.enable and w is not None and self.in_features > _ck.max_quant_k():
                        logging.warning(f"INT4 ConvRot: {keys.prefix} stays bf16: in_features {self.in_features} "
                                        f"exceeds {_ck.max_quant_k()}, the widest row the gfx950 rotate+quantize "
                                        f"kernels take")
                    return False
                mode = self._quant_mode(keys.prefix)
                groupsize = _pick_groupsize(self.in_features)
                w16 = w.to("cuda", torch.float16)        # the loader's quantization input dtype
                try:
                    if mode == "int8":
                        from ._int4.int8_eager import quantize_convrot_w8a8_weight
                        q, s = quantize_convrot_w8a8_weight(w16, convrot_groupsize=groupsize)
                    else:
                        seed = Int4ConvRotOps._STOCHASTIC_SEED if Int4ConvRotOps.lora_mode == "Stochastic" else 0
                        q, s = _ck.quantize_convrot_w4a4_weight(w16, convrot_groupsize=groupsize,
                                                                stochastic_rounding=seed)
                    self._install(q, s, groupsize, mode, state_dict, keys, (keys.weight,))
                    return True
                except Exception as e:
                    logging.warning(f"INT4 ConvRot: fell back to bf16 for {keys.prefix}: {e}")
                    return False

            def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict,
                                      missing_keys, unexpected_keys, error_msgs):
                keys = _Keys(prefix)
                w = state_dict.get(keys.weight)
                if self._take_prequantized(state_dict, keys, w):
                    return
                w = state_dict.get(keys.weight)          # a too-wide prequantized weight comes back dequantized
                w = self._route_lora(state_dict, keys, w)
                if self._quantize_on_load(state_dict, keys, w):
                    return
                return super()._load_from_state_dict(
                    state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys, error_msgs)

            # -- forward ---------------------------------------------------------

            def _operand(self):
                """The quantized weight the GEMM reads (the one device copy)."""
                return self._q6 if self._q6 is not None else self._q8t if self._q8t is not None else self._qpack

            def _to_device(self, dev):
                """Move the quantized storage to `dev` once (the loader may keep
                layers elsewhere until the model runs)."""
                if self._operand().device == dev:
                    return
                self._qs = self._qs.to(dev)
                self._qpack = None if self._qpack is None else self._qpack.to(dev)
                self._q6 = None if self._q6 is None else self._q6.to(dev)
                self._q8t = None if self._q8t is None else self._q8t.to(dev)
                if self._dyn_fused is not None:
                    self._dyn_fused = tuple(t.to(dev) for t in self._dyn_fused)

            def forward(self, x):
                if self._qmode is None:
                    return self._apply_dyn_lora(x, super().forward(x))
                self._to_device(x.device)
                bias = self.bias if self.bias is None or self.bias.device == x.device else self.bias.to(x.device)
                # the checkpoint-layout codes when they are the operand, else their shape
                qw = self._qpack if self._qpack is not None else self._qshape
                if self._qmode == "int8":
                    y = _ck.convrot_w8a8_linear(x, qw, self._qs, bias=bias, convrot_groupsize=self._qgs,
                                                qweight_i8t=self._q8t)
                    return self._apply_dyn_lora(x, y)
                y = _ck.convrot_w4a4_linear(x, qw, self._qs, bias=bias, convrot_groupsize=self._qgs,
                                            lora=self._dyn_fused, qweight_bf6=self._q6)
                return self._apply_dyn_lora(x, y, None if self._dyn_fused is None else self._dyn_rest)

else:  # comfy.ops or the backend unavailable
    Int4ConvRotOps = None
