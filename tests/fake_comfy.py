"""A minimal stand-in for the parts of ComfyUI the Linear replacement imports
(``comfy.ops.manual_cast``) and for a plain LoRA weight adapter, so the
replacement's load and forward logic runs without ComfyUI installed."""
import sys
import types

import torch


def install_fake_comfy():
    if "comfy.ops" in sys.modules and getattr(sys.modules["comfy.ops"], "_FAKE", False):
        return
    comfy = types.ModuleType("comfy")
    ops = types.ModuleType("comfy.ops")
    ops._FAKE = True

    class manual_cast:
        class Linear(torch.nn.Linear):
            comfy_cast_weights = True

            def reset_parameters(self):
                return None

            def forward(self, x):
                w = self.weight.to(x.device, x.dtype)
                b = self.bias.to(x.device, x.dtype) if self.bias is not None else None
                return torch.nn.functional.linear(x, w, b)

    ops.manual_cast = manual_cast
    comfy.ops = ops
    sys.modules["comfy"] = comfy
    sys.modules["comfy.ops"] = ops


class FakeLoRA:
    """A plain LoRA adapter: weights = (up [N, r], down [r, K], alpha, mid,
    dora_scale, reshape); its bypass h() adds multiplier * alpha / r *
    up(down(x)), computed here in fp32."""
    name = "lora"

    def __init__(self, up, down, alpha=None, mid=None, dora_scale=None):
        self.weights = (up, down, alpha, mid, dora_scale, None)

    def h(self, x, base_out):
        up, down, alpha = self.weights[0], self.weights[1], self.weights[2]
        r = down.shape[0]
        s = (float(alpha) / r if alpha is not None else 1.0) * float(getattr(self, "multiplier", 1.0))
        y = (x.float() @ down.float().T) @ up.float().T
        return (y * s).to(base_out.dtype)


class FakeLoHa(FakeLoRA):
    """An adapter that is not a plain LoRA (keeps the generic h() path)."""
    name = "loha"
