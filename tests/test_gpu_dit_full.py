"""The DiT stack configuration at full size: 8 double-stream blocks, hidden
3072, 24 heads, MLP x4, 4096 image + 512 text tokens, a rank-32 dynamic LoRA
on every quantized linear, loaded through Int4ConvRotOps.

One forward runs with hooks on the eight quantized linears of a middle block
(image and text stream, each of qkv / proj / mlp up / mlp down).  For each
layer's real in-stack input and output:
  * the activation codes and scales equal the oracle's on sampled rows;
  * the whole output tensor equals the packed-operand int8-MFMA kernels (with
    the same LoRA term) fed the same input, bit for bit;
  * on sampled rows the output is within 1e-2 relative Frobenius of the eager
    bf16 chain plus the LoRA term, and within the elementwise bound of the f32
    epilogue plus the LoRA term."""
import numpy as np
import pytest
import torch

import dit_stack as ds
from fake_comfy import FakeLoRA, install_fake_comfy

pytestmark = pytest.mark.gpu

BF16 = 1
N_IMG, N_TXT, DEPTH, BLOCK = 4096, 512, 8, 3
KINDS = ("img_attn.qkv", "img_attn.proj", "img_mlp.0", "img_mlp.2",
         "txt_attn.qkv", "txt_attn.proj", "txt_mlp.0", "txt_mlp.2")


def bits(t):
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def bf16_f64(b):
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


@pytest.fixture(scope="module")
def captured(gpu):
    install_fake_comfy()
    from importlib import import_module, reload
    m = import_module("comfyui-int4-convrot-rdna4_amd.int4_ops")
    if m.Int4ConvRotOps is None:
        m = reload(m)
    print(f"building the {DEPTH}-block stack", flush=True)
    model, _, patches, applied = ds.build_int4_stack(m.Int4ConvRotOps, FakeLoRA, depth=DEPTH, keep_reference=False)
    assert applied == set(patches) and len(patches) == 8 * DEPTH
    img, ctx, t = ds.synthetic_inputs(N_IMG, N_TXT, device="cuda")
    mods = {k: dict(model.named_modules())[f"double_blocks.{BLOCK}.{k}"] for k in KINDS}
    seen, hooks = {}, []
    for k, mod in mods.items():
        hooks.append(mod.register_forward_hook(
            lambda _m, a, out, k=k: seen.__setitem__(k, (a[0].detach().clone(), out.detach().clone()))))
    try:
        with torch.no_grad():
            y = model(img, ctx, t)
        torch.cuda.synchronize()
    finally:
        for h in hooks:
            h.remove()
    assert y.shape == (1, N_IMG, 64) and torch.isfinite(y.float()).all()
    print("forward done", flush=True)
    return mods, seen


@pytest.mark.parametrize("kind", KINDS)
def test_full_stack_layer_in_context(captured, native, oracle, kind):
    mods, seen = captured
    mod = mods[kind]
    x, y = seen[kind]
    K, N = mod.in_features, mod.out_features
    x2 = x.reshape(-1, K).contiguous()
    y2 = y.reshape(-1, N)
    M = x2.shape[0]
    assert M == (N_IMG if kind.startswith("img") else N_TXT)
    print(f"layer {kind} M={M} K={K} N={N}", flush=True)
    D, U = mod._dyn_fused
    bias32 = mod.bias.float()
    # the whole tensor against the packed-operand kernels with the same LoRA term
    qx, xs = native.convrot_quant_int4(x2, mod._qgs)
    tl = native.lora_down(x2, D)
    ref = native.int4_convrot_gemm_lora(qx, mod._q, xs, mod._qs, bias32, tl, U, 1.0, native.EPI_BF16)
    assert torch.equal(y2.view(torch.int16), ref.view(torch.int16)), kind
    # sampled rows against the oracle
    rows = np.sort(np.random.RandomState(K + N + M).choice(M, 16, replace=False))
    xb = bits(x2[torch.from_numpy(rows).cuda()])
    packed, exs, _ = oracle.rotquant(xb, BF16, mod._qgs)
    assert np.array_equal(qx.cpu().numpy()[rows], packed) and np.array_equal(xs.cpu().numpy()[rows], exs), kind
    qw, ws, b = mod._q.cpu().numpy(), mod._qs.cpu().numpy(), bias32.cpu().numpy()
    acc = oracle.int_gemm(packed, qw)
    Dd, Ud = D.float().cpu().double().numpy(), U.float().cpu().double().numpy()
    tt = torch.from_numpy(bf16_f64(xb) @ Dd.T).float().to(torch.bfloat16).double().numpy()
    lora = tt @ Ud.T
    want = bf16_f64(oracle.epilogue_eager_bf16(acc, exs, ws, b)) + lora
    want_f32 = oracle.epilogue_f32(acc, exs, ws, b).astype(np.float64) + lora
    got = bf16_f64(bits(y2)[rows])
    err = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert err < 1e-2, (kind, err)
    tu = np.abs(tt) @ np.abs(Ud).T
    bound = 2.0 ** -8 * np.abs(want_f32) + (2.0 ** -7 + 2.0 ** -18) * tu + 1e-6
    assert np.all(np.abs(got - want_f32) <= bound), (kind, float(np.max(np.abs(got - want_f32) - bound)))
