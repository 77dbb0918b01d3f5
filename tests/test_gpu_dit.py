"""The synthetic double-stream DiT stack through Int4ConvRotOps on the GPU:
what the loader path selects and attaches (skip list, fp16 bias, fused
dynamic LoRA), every quantized linear checked in context against the oracle
(codes and scales bit-exact, outputs against the eager chain plus the LoRA
term), the whole forward without LoRA bit-identical to the same stack with
every quantized linear's output replaced by the oracle's, and run-to-run
determinism."""
import numpy as np
import pytest
import torch

import dit_stack as ds
from fake_comfy import FakeLoRA, install_fake_comfy

pytestmark = pytest.mark.gpu

BF16 = 1
F16 = 2
N_IMG, N_TXT = 128, 64
DEPTH = 2


def bits(t):
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def bf16_bits_to_f64(b):
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def unpack_f64(packed):
    p = packed.astype(np.int16) & 0xFF
    lo = ((p & 15) ^ 8) - 8
    hi = ((p >> 4) ^ 8) - 8
    return np.stack([lo, hi], -1).reshape(packed.shape[0], -1).astype(np.float64)


@pytest.fixture(scope="module")
def stack(gpu):
    install_fake_comfy()
    from importlib import import_module, reload
    m = import_module("comfyui-int4-convrot-rdna4_amd.int4_ops")
    if m.Int4ConvRotOps is None:
        m = reload(m)
    print(f"building the {DEPTH}-block stack", flush=True)
    model, ref_sd, patches, applied = ds.build_int4_stack(m.Int4ConvRotOps, FakeLoRA, depth=DEPTH)
    inputs = ds.synthetic_inputs(N_IMG, N_TXT, device="cuda")
    return model, ref_sd, patches, applied, inputs


def quantized_layers(model):
    return [(n, mod) for n, mod in model.named_modules() if hasattr(mod, "in_features") and ds.is_quantized_name(n)]


def test_loader_selection(stack):
    model, ref_sd, patches, applied, _ = stack
    n_q = 0
    for name, mod in model.named_modules():
        if not hasattr(mod, "in_features"):
            continue
        if ds.is_quantized_name(name):
            n_q += 1
            K, N = mod.in_features, mod.out_features
            assert mod._qmode == "int4" and mod.weight is None, name
            assert mod._q.shape == (N, K // 2) and mod._q.dtype == torch.int8
            assert mod._qs.shape == (N,) and mod._qs.dtype == torch.float32
            assert mod._qgs == 256 and mod._q6 is not None
            assert mod.bias.dtype == torch.float16, name          # the loader keeps biases in fp16
            D, U = mod._dyn_fused
            assert D.shape == (32, K) and U.shape == (N, 32) and mod._dyn_rest == []
        else:
            assert mod._q is None and mod.weight.dtype == torch.bfloat16, name
            assert torch.equal(mod.weight.cpu(), ref_sd[name + ".weight"].cpu())
    assert n_q == 8 * DEPTH
    assert applied == set(patches) and len(patches) == n_q


@pytest.mark.parametrize("name", ["double_blocks.0.img_attn.qkv", "double_blocks.1.txt_mlp.2"])
def test_weight_codes_match_oracle(stack, oracle, name):
    """Load-time quantization of the bf16 checkpoint weight (through fp16, as the
    Linear replacement does) is the oracle's, bit for bit."""
    model, ref_sd, *_ = stack
    mod = dict(model.named_modules())[name]
    w16 = ref_sd[name + ".weight"].to(torch.float16).cpu()
    qw, ws = oracle.quantize_weight(bits(w16), F16, 256)
    assert np.array_equal(mod._q.cpu().numpy(), qw)
    assert np.array_equal(mod._qs.cpu().numpy(), ws)


def oracle_linear(oracle, mod, x):
    """The oracle's output of a quantized linear for input x (bf16 [..., K]):
    eager bf16 chain of the exact integer GEMM, plus the fused LoRA term
    (t = bf16(x D^T), then t U^T) in fp64.  Returns (eager + lora, f32-epilogue
    + lora, sum |t| |U| per element) as float64 [M, N]."""
    K = mod.in_features
    xb = bits(x.reshape(-1, K))
    packed, xs, _ = oracle.rotquant(xb, BF16, mod._qgs)
    qw = mod._q.cpu().numpy()
    ws = mod._qs.cpu().numpy()
    bias = mod.bias.float().cpu().numpy()
    acc64 = unpack_f64(packed) @ unpack_f64(qw).T            # exact: |partial sums| < 2^53
    acc = acc64.astype(np.int32)
    rows = np.arange(0, acc.shape[0], 37)
    assert np.array_equal(acc[rows], oracle.int_gemm(packed[rows], qw))
    eager = bf16_bits_to_f64(oracle.epilogue_eager_bf16(acc, xs, ws, bias))
    f32 = oracle.epilogue_f32(acc, xs, ws, bias).astype(np.float64)
    D, U = (t.float().cpu().double().numpy() for t in mod._dyn_fused)
    t = torch.from_numpy(bf16_bits_to_f64(xb) @ D.T).float().to(torch.bfloat16).double().numpy()
    lora = t @ U.T
    return eager + lora, f32 + lora, np.abs(t) @ np.abs(U).T, (packed, xs)


def capture(model, fn):
    """Run fn() with forward hooks on every quantized linear; -> {name: (x, y)}."""
    seen, hooks = {}, []
    for n, mod in quantized_layers(model):
        hooks.append(mod.register_forward_hook(lambda m, a, out, n=n: seen.__setitem__(n, (a[0].detach().clone(), out.detach().clone()))))
    try:
        fn()
    finally:
        for h in hooks:
            h.remove()
    return seen


def test_every_linear_in_context(stack, native, oracle):
    model, _, _, _, (img, ctx, t) = stack
    with torch.no_grad():
        seen = capture(model, lambda: model(img, ctx, t))
    assert len(seen) == 8 * DEPTH
    for name, (x, y) in seen.items():
        mod = dict(model.named_modules())[name]
        print(f"layer {name} M={x.numel() // x.shape[-1]}", flush=True)
        want, want_f32, tu, (packed, xs) = oracle_linear(oracle, mod, x)
        # codes and scales of the layer's real activation, bit for bit
        q, s = native.convrot_quant_int4(x.reshape(-1, mod.in_features).contiguous(), mod._qgs)
        assert np.array_equal(q.cpu().numpy(), packed), name
        assert np.array_equal(s.cpu().numpy(), xs), name
        got = y.reshape(-1, mod.out_features).double().cpu().numpy()
        err = np.linalg.norm(got - want) / np.linalg.norm(want)
        assert err < 1e-2, (name, err)
        # against the f32 epilogue: half a bf16 ulp of the output (2^-8 relative),
        # one bf16 ulp of each t (2^-7 relative; the GPU's fp32 down projection
        # may round t the other way) and the fp32 sum of the rank terms
        bound = 2.0 ** -8 * np.abs(want_f32) + (2.0 ** -7 + 2.0 ** -18) * tu + 1e-6
        assert np.all(np.abs(got - want_f32) <= bound), (name, float(np.max(np.abs(got - want_f32) - bound)))


@pytest.fixture(scope="module")
def plain_stack(gpu):
    """The same stack (same weights) loaded without LoRA adapters."""
    install_fake_comfy()
    from importlib import import_module
    m = import_module("comfyui-int4-convrot-rdna4_amd.int4_ops")
    model, _, _, _ = ds.build_int4_stack(m.Int4ConvRotOps, None, depth=DEPTH, keep_reference=False)
    return model


def test_stack_bitexact_with_oracle_linears(plain_stack, stack, oracle):
    """The whole forward (no LoRA) with the kernels equals, bit for bit, the
    same forward with every quantized linear's output replaced by the oracle's
    (rotate+quantize of that run's own input, exact integer GEMM, the f32
    epilogue rounded once to bf16: the computation of the reference's HIP
    path).  The int4 quantizer is discontinuous, so a forward whose linears
    differ by rounding (e.g. the eager bf16 chain instead of the f32
    epilogue) flips codes in the next layer's activation and drifts by far
    more than the per-linear tolerance; only exact per-layer agreement
    composes, and that is what this checks end to end."""
    model = plain_stack
    img, ctx, t = stack[4]
    assert all(m._dyn_fused is None and m._dyn_lora is None for _, m in quantized_layers(model))

    def replace(mod, args, out):
        K, N = mod.in_features, mod.out_features
        xb = bits(args[0].reshape(-1, K))
        packed, xs, _ = oracle.rotquant(xb, BF16, mod._qgs)
        qw = mod._q.cpu().numpy()
        acc = (unpack_f64(packed) @ unpack_f64(qw).T).astype(np.int32)
        o = oracle.epilogue_f32(acc, xs, mod._qs.cpu().numpy(), mod.bias.float().cpu().numpy(), out_bf16=True)
        return torch.from_numpy(o.view(np.int16)).view(torch.bfloat16).to(out.device).reshape(out.shape)

    with torch.no_grad():
        y = model(img, ctx, t)
        hooks = [mod.register_forward_hook(replace) for _, mod in quantized_layers(model)]
        try:
            y_ref = model(img, ctx, t)
        finally:
            for h in hooks:
                h.remove()
    assert torch.isfinite(y.float()).all()
    assert torch.equal(y, y_ref), float((y.double() - y_ref.double()).norm() / y_ref.double().norm())


def test_forward_deterministic(stack):
    model, _, _, _, (img, ctx, t) = stack
    with torch.no_grad():
        a = model(img, ctx, t)
        b = model(img, ctx, t)
    assert a.shape == (1, N_IMG, 64) and a.dtype == torch.bfloat16
    assert torch.equal(a, b)
