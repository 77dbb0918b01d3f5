"""A synthetic Flux-style double-stream DiT stack: the workload that drives
``Int4ConvRotOps`` the way a ComfyUI diffusion model does (test and benchmark
helper, not part of the package).

Layer names follow the Flux 2 checkpoint keys so that the loader's skip list
for that model family applies unchanged (reference int4_loader.py:25-27): the
embedders (``img_in``, ``txt_in``, ``time_in``), the shared per-stream
modulation (``double_stream_modulation_img`` / ``_txt``) and ``final_layer``
stay bf16; the eight linears of every double block
(``{img,txt}_attn.{qkv,proj}``, ``{img,txt}_mlp.{0,2}``) are quantized.

Block (hidden H, ``heads`` heads of H/heads, MLP ratio 4, GELU-tanh MLP):

    per stream s in (img, txt), with (shift1, scale1, gate1, shift2, scale2, gate2) = mod_s
        x_s = LN(s) * (1 + scale1) + shift1
        q_s, k_s, v_s = split(s_attn.qkv(x_s)); q_s, k_s = RMSNorm(q_s), RMSNorm(k_s)
    a = attention over the joint sequence [txt; img]
    s = s + gate1 * s_attn.proj(a_s)
    s = s + gate2 * s_mlp(LN(s) * (1 + scale2) + shift2)

Attention is computed head-chunk by head-chunk with contiguous operands
(``q @ k^T`` from an explicitly transposed copy of k, softmax in fp32).  No
rotary embedding: it does not touch the linears.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

# Flux 2 skip list of the loader (reference int4_loader.py:25-27)
FLUX2_EXCLUDED = ['img_in', 'time_in', 'guidance_in', 'txt_in',
                  'double_stream_modulation_img', 'double_stream_modulation_txt',
                  'single_stream_modulation', 'final_layer']

QUANTIZED_SUFFIXES = ("img_attn.qkv", "img_attn.proj", "img_mlp.0", "img_mlp.2",
                      "txt_attn.qkv", "txt_attn.proj", "txt_mlp.0", "txt_mlp.2")


def _rms(x: torch.Tensor, scale: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * scale.float()).to(x.dtype)


def _modulate(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1]
    return F.layer_norm(x, (h,), eps=1e-6) * (1 + scale) + shift


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, head_chunk: int = 4) -> torch.Tensor:
    """softmax(q k^T / sqrt(d)) v for [1, heads, L, d] bf16 -> [1, L, heads * d]."""
    _, nh, L, d = q.shape
    out = torch.empty((nh, L, d), dtype=q.dtype, device=q.device)
    for h0 in range(0, nh, head_chunk):
        h1 = min(nh, h0 + head_chunk)
        qh = q[0, h0:h1].contiguous()
        kt = k[0, h0:h1].transpose(1, 2).contiguous()
        s = torch.matmul(qh, kt).float() * (1.0 / math.sqrt(d))
        p = torch.softmax(s, dim=-1).to(q.dtype)
        del s
        out[h0:h1] = torch.matmul(p, v[0, h0:h1].contiguous())
    return out.permute(1, 0, 2).reshape(1, L, nh * d)


class SelfAttention(nn.Module):
    def __init__(self, hidden, heads, ops, dtype, device):
        super().__init__()
        self.heads = heads
        self.qkv = ops.Linear(hidden, 3 * hidden, bias=True, dtype=dtype, device=device)
        self.norm = nn.Module()
        self.norm.query_norm = nn.Module()
        self.norm.key_norm = nn.Module()
        d = hidden // heads
        self.norm.query_norm.scale = nn.Parameter(torch.ones(d, dtype=dtype, device=device), requires_grad=False)
        self.norm.key_norm.scale = nn.Parameter(torch.ones(d, dtype=dtype, device=device), requires_grad=False)
        self.proj = ops.Linear(hidden, hidden, bias=True, dtype=dtype, device=device)

    def qkv_heads(self, x):
        B, L, H = x.shape
        qkv = self.qkv(x).view(B, L, 3, self.heads, H // self.heads).permute(2, 0, 3, 1, 4)
        q = _rms(qkv[0], self.norm.query_norm.scale)
        k = _rms(qkv[1], self.norm.key_norm.scale)
        return q, k, qkv[2]


class MLP(nn.Sequential):
    def __init__(self, hidden, mlp_hidden, ops, dtype, device):
        super().__init__(ops.Linear(hidden, mlp_hidden, bias=True, dtype=dtype, device=device),
                         nn.GELU(approximate="tanh"),
                         ops.Linear(mlp_hidden, hidden, bias=True, dtype=dtype, device=device))


class DoubleStreamBlock(nn.Module):
    def __init__(self, hidden, heads, mlp_ratio, ops, dtype, device):
        super().__init__()
        mh = int(hidden * mlp_ratio)
        self.img_attn = SelfAttention(hidden, heads, ops, dtype, device)
        self.img_mlp = MLP(hidden, mh, ops, dtype, device)
        self.txt_attn = SelfAttention(hidden, heads, ops, dtype, device)
        self.txt_mlp = MLP(hidden, mh, ops, dtype, device)

    def forward(self, img, txt, mod_img, mod_txt):
        iq, ik, iv = self.img_attn.qkv_heads(_modulate(img, mod_img[0], mod_img[1]))
        tq, tk, tv = self.txt_attn.qkv_heads(_modulate(txt, mod_txt[0], mod_txt[1]))
        a = attention(torch.cat((tq, iq), 2), torch.cat((tk, ik), 2), torch.cat((tv, iv), 2))
        lt = txt.shape[1]
        img = img + mod_img[2] * self.img_attn.proj(a[:, lt:])
        img = img + mod_img[5] * self.img_mlp(_modulate(img, mod_img[3], mod_img[4]))
        txt = txt + mod_txt[2] * self.txt_attn.proj(a[:, :lt])
        txt = txt + mod_txt[5] * self.txt_mlp(_modulate(txt, mod_txt[3], mod_txt[4]))
        return img, txt


class Embedder(nn.Module):
    """time_in: Linear(256, H) -> SiLU -> Linear(H, H)."""

    def __init__(self, in_dim, hidden, ops, dtype, device):
        super().__init__()
        self.in_layer = ops.Linear(in_dim, hidden, bias=True, dtype=dtype, device=device)
        self.out_layer = ops.Linear(hidden, hidden, bias=True, dtype=dtype, device=device)

    def forward(self, x):
        return self.out_layer(F.silu(self.in_layer(x)))


class Modulation(nn.Module):
    def __init__(self, hidden, ops, dtype, device):
        super().__init__()
        self.lin = ops.Linear(hidden, 6 * hidden, bias=True, dtype=dtype, device=device)

    def forward(self, vec):
        return self.lin(F.silu(vec))[:, None, :].chunk(6, dim=-1)


class FinalLayer(nn.Module):
    def __init__(self, hidden, out_channels, ops, dtype, device):
        super().__init__()
        self.linear = ops.Linear(hidden, out_channels, bias=True, dtype=dtype, device=device)

    def forward(self, x):
        return self.linear(F.layer_norm(x, (x.shape[-1],), eps=1e-6))


def timestep_embedding(t: torch.Tensor, dim: int = 256, max_period: float = 10000.0) -> torch.Tensor:
    half = dim // 2
    freqs = torch.exp(-math.log(max_period) * torch.arange(half, dtype=torch.float32, device=t.device) / half)
    args = 1000.0 * t.float()[:, None] * freqs[None]
    return torch.cat((torch.cos(args), torch.sin(args)), dim=-1)


class DoubleStreamDiT(nn.Module):
    def __init__(self, ops, depth=8, hidden=3072, heads=24, mlp_ratio=4.0, in_channels=64, context_dim=4096,
                 dtype=torch.bfloat16, device=None):
        super().__init__()
        self.img_in = ops.Linear(in_channels, hidden, bias=True, dtype=dtype, device=device)
        self.txt_in = ops.Linear(context_dim, hidden, bias=True, dtype=dtype, device=device)
        self.time_in = Embedder(256, hidden, ops, dtype, device)
        self.double_stream_modulation_img = Modulation(hidden, ops, dtype, device)
        self.double_stream_modulation_txt = Modulation(hidden, ops, dtype, device)
        self.double_blocks = nn.ModuleList(DoubleStreamBlock(hidden, heads, mlp_ratio, ops, dtype, device)
                                           for _ in range(depth))
        self.final_layer = FinalLayer(hidden, in_channels, ops, dtype, device)

    def forward(self, img, context, t):
        img = self.img_in(img)
        txt = self.txt_in(context)
        vec = self.time_in(timestep_embedding(t).to(img.dtype))
        mod_img = self.double_stream_modulation_img(vec)
        mod_txt = self.double_stream_modulation_txt(vec)
        for blk in self.double_blocks:
            img, txt = blk(img, txt, mod_img, mod_txt)
        return self.final_layer(img)


def linear_shapes(model: nn.Module):
    """{name: (in_features, out_features)} of every Linear-like module."""
    return {n: (m.in_features, m.out_features) for n, m in model.named_modules() if hasattr(m, "in_features")}


def is_quantized_name(name: str) -> bool:
    return name.startswith("double_blocks.") and name.split(".", 2)[2] in QUANTIZED_SUFFIXES


def state_dict_for(model: nn.Module, seed: int = 0, device="cpu", w_std=0.02, b_std=0.01):
    """Random-init weights of the model's architecture: Linear weights N(0, w_std),
    biases N(0, b_std), norm scales 1, all bf16, drawn in module order from one
    seeded generator on ``device``."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    sd = {}
    for name, m in model.named_modules():
        if hasattr(m, "in_features"):
            sd[name + ".weight"] = (torch.randn((m.out_features, m.in_features), generator=g, device=device)
                                    * w_std).to(torch.bfloat16)
            sd[name + ".bias"] = (torch.randn((m.out_features,), generator=g, device=device) * b_std
                                  ).to(torch.bfloat16)
    for name, p in model.named_parameters():
        if name.endswith(".scale"):
            sd[name] = torch.ones(p.shape, dtype=torch.bfloat16, device=device)
    return sd


def lora_patches_for(model: nn.Module, adapter_cls, rank=32, seed=1, std=0.02):
    """{normalized weight key: [(adapter, None, None, 1.0)]}: one rank-``rank``
    plain LoRA (alpha = rank, so scale 1) on every quantized linear."""
    g = torch.Generator()
    g.manual_seed(seed)
    out = {}
    for name, (k, n) in linear_shapes(model).items():
        if is_quantized_name(name):
            up = torch.randn((n, rank), generator=g) * std
            down = torch.randn((rank, k), generator=g) * std
            out[name + ".weight"] = [(adapter_cls(up, down, float(rank)), None, None, 1.0)]
    return out


def synthetic_inputs(n_img: int, n_txt: int, in_channels=64, context_dim=4096, seed=2, device="cpu"):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    img = torch.randn((1, n_img, in_channels), generator=g, device=device).to(torch.bfloat16)
    ctx = torch.randn((1, n_txt, context_dim), generator=g, device=device).to(torch.bfloat16)
    t = torch.full((1,), 0.5, device=device)
    return img, ctx, t


def quantized_work(n_img: int, n_txt: int, depth=8, hidden=3072, mlp_ratio=4.0, lora_rank=0):
    """Ops of the quantized linears of one forward: 2*M*N*K per linear
    (+ 2*M*R*(K+N) for the LoRA side path when ``lora_rank``)."""
    mh = int(hidden * mlp_ratio)
    kn = [(hidden, 3 * hidden), (hidden, hidden), (hidden, mh), (mh, hidden)]
    total = 0
    for M in (n_img, n_txt):
        for K, N in kn:
            total += 2 * M * N * K + (2 * M * lora_rank * (K + N) if lora_rank else 0)
    return depth * total


def build_int4_stack(Ops, adapter_cls=None, depth=8, n_lora_rank=32, seed=0, weight_device="cuda",
                     excluded=FLUX2_EXCLUDED, min_in_features=512, keep_reference=True, **kw):
    """The stack built and loaded through ``Ops`` (an Int4ConvRotOps class) the
    way the loader does it: class attributes set, modules constructed on the CPU
    without initialisation, then ``load_state_dict`` quantizes the eligible
    linears and attaches the dynamic LoRA adapters.  Returns (model on cuda,
    a copy of the bf16 state dict that was loaded or None, the LoRA patches,
    the keys whose patches were applied)."""
    model = DoubleStreamDiT(Ops, depth=depth, device="cpu", **kw)
    sd = state_dict_for(model, seed=seed, device=weight_device)
    ref_sd = {k: v.clone() for k, v in sd.items()} if keep_reference else None
    patches = lora_patches_for(model, adapter_cls, rank=n_lora_rank) if adapter_cls is not None else {}
    saved = (Ops.enable, list(Ops.excluded_names), set(Ops.excluded_exact), Ops.min_in_features,
             Ops.lora_patches, Ops.lora_dynamic, Ops.lora_mode)
    try:
        Ops.enable = True
        Ops.excluded_names = list(excluded)
        Ops.excluded_exact = set()
        Ops.min_in_features = int(min_in_features)
        Ops.lora_patches = patches
        Ops.lora_dynamic = bool(patches)
        Ops.lora_mode = "Dynamic" if patches else "None"
        Ops._applied_lora = set()
        model.load_state_dict(sd, strict=False)
        applied = set(Ops._applied_lora)
        del sd
    finally:
        (Ops.enable, Ops.excluded_names, Ops.excluded_exact, Ops.min_in_features,
         Ops.lora_patches, Ops.lora_dynamic, Ops.lora_mode) = saved
        Ops._applied_lora = set()
    model = model.to("cuda")
    return model, ref_sd, patches, applied
