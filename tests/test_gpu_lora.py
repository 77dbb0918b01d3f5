"""GPU checks of the fused dynamic-LoRA side path: the down projection, the
up projection inside each GEMM epilogue (against the bit-exact main epilogue
plus an fp64 closed form of the LoRA term), the linear entry point and the
Int4ConvRotOps forward with adapters attached."""
import numpy as np
import pytest
import torch

from fake_comfy import FakeLoHa, FakeLoRA, install_fake_comfy
from inputs import normal_bias, normal_weight, outlier_activations

pytestmark = pytest.mark.gpu


def cu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def f64(t):
    return t.detach().float().cpu().double().numpy()


def rand_bf16(shape, seed, std):
    rs = np.random.RandomState(seed)
    return torch.from_numpy((rs.standard_normal(shape) * std).astype(np.float32)).to(torch.bfloat16)


DOWN_CASES = [(1, 256, 32, torch.bfloat16), (31, 3072, 64, torch.bfloat16), (33, 2080, 96, torch.float16),
              (300, 3072, 128, torch.bfloat16), (4608, 3072, 128, torch.bfloat16), (100, 12288, 32, torch.float16),
              (7, 1040, 32, torch.bfloat16), (17, 528, 64, torch.bfloat16), (4096, 12288, 32, torch.bfloat16),
              (512, 3072, 32, torch.float16), (16, 16, 96, torch.bfloat16),
              # 128-row workgroups over k ranges of <= 384 (M >= 1024, K <= 3072, R <= 64)
              (4096, 3072, 32, torch.bfloat16), (1025, 3072, 64, torch.float16), (2000, 1040, 32, torch.bfloat16),
              (1024, 256, 32, torch.bfloat16), (1500, 3056, 64, torch.bfloat16)]


@pytest.mark.parametrize("M,K,R,dt", DOWN_CASES)
def test_lora_down_matches_fp64(native, gpu, M, K, R, dt):
    print(f"lora_down M={M} K={K} R={R} {dt}", flush=True)
    x = outlier_activations(M, K, seed=M + K, dtype=dt)
    D = rand_bf16((R, K), R + K, 0.05)
    t = native.lora_down(x.cuda(), D.cuda())
    assert t.shape == (M, R) and t.dtype == torch.bfloat16
    xd, Dd = f64(x), f64(D)
    ref = xd @ Dd.T
    mag = np.abs(xd) @ np.abs(Dd).T
    err = np.abs(f64(t) - ref)
    # bf16 rounding of t, fp32 accumulation, and (f16 input) the bf16 operand conversion
    bound = 2.0 ** -8 * np.abs(ref) + (2.0 ** -12 + (2.0 ** -9 if dt == torch.float16 else 0.0)) * mag
    assert np.all(err <= bound), float((err / np.maximum(bound, 1e-30)).max())
    assert np.linalg.norm(f64(t) - ref) / np.linalg.norm(ref) < 4e-3
    assert torch.equal(native.lora_down(x.cuda(), D.cuda()), t)     # fixed summation order


def rand_gemm(M, N, K, R, seed):
    rs = np.random.RandomState(seed)
    xp = rs.randint(-128, 128, size=(M, K // 2)).astype(np.int8)
    wp = rs.randint(-128, 128, size=(N, K // 2)).astype(np.int8)
    xs = rs.uniform(0.005, 0.05, size=M).astype(np.float32)
    ws = rs.uniform(0.005, 0.05, size=N).astype(np.float32)
    b = (rs.standard_normal(N) * 0.01).astype(np.float32)
    t = rand_bf16((M, R), seed + 1, 1.0)
    U = rand_bf16((N, R), seed + 2, 0.5)
    return xp, wp, xs, ws, b, t, U


GEMM_CASES = [(64, 48, 256, 32), (257, 300, 3072, 64), (33, 513, 2080, 96), (300, 256, 1024, 128),
              (4608, 3072, 3072, 128)]


@pytest.mark.parametrize("M,N,K,R", GEMM_CASES)
def test_gemm_lora_epilogues(native, oracle, gpu, M, N, K, R):
    print(f"gemm_lora M={M} N={N} K={K} R={R}", flush=True)
    xp, wp, xs, ws, b, t, U = rand_gemm(M, N, K, R, M + N + K + R)
    scale = 0.375
    rows = np.arange(M) if M <= 512 else np.random.RandomState(0).choice(M, 64, replace=False)
    acc = oracle.int_gemm(xp[rows], wp)
    main = oracle.epilogue_f32(acc, xs[rows], ws, b).astype(np.float64)
    td, Ud = f64(t)[rows], f64(U)
    lterm = scale * (td @ Ud.T)
    lmag = scale * (np.abs(td) @ np.abs(Ud).T)
    args = (cu(xp), cu(wp), cu(xs), cu(ws), cu(b), t.cuda(), U.cuda(), scale)

    f32 = native.int4_convrot_gemm_lora(*args, native.EPI_F32).cpu().double().numpy()[rows]
    want = main + lterm
    bound = 2.0 ** -23 * (np.abs(main) + np.abs(lterm)) + 2.0 ** -17 * lmag
    assert np.all(np.abs(f32 - want) <= bound)

    bf = native.int4_convrot_gemm_lora(*args, native.EPI_BF16).float().cpu().double().numpy()[rows]
    assert np.all(np.abs(bf - want) <= 2.0 ** -8 * np.abs(want) + bound)

    # eager bf16 chain: o4 (bit-exact chain) + bf16(scale * l), rounded to bf16
    o4 = oracle.bf16_to_f32(oracle.epilogue_eager_bf16(acc, xs[rows], ws, b)).astype(np.float32)
    lb = oracle.bf16_to_f32(oracle.f32_to_bf16(lterm.astype(np.float32)))
    exp = oracle.bf16_to_f32(oracle.f32_to_bf16((o4 + lb).astype(np.float32))).astype(np.float64)
    eg = native.int4_convrot_gemm_lora(*args, native.EPI_BF16_EAGER).float().cpu().double().numpy()[rows]
    diff = np.abs(eg - exp)
    assert np.all(diff <= 2.0 ** -7 * (np.abs(exp) + np.abs(lterm)) + 2.0 ** -16 * lmag)  # one bf16 step
    assert np.mean(diff == 0) > 0.99


def test_gemm_lora_zero_up_equals_plain_gemm(native, gpu):
    """U = 0 leaves every epilogue bit-identical to the plain GEMM."""
    M, N, K, R = 257, 300, 3072, 32
    xp, wp, xs, ws, b, t, U = rand_gemm(M, N, K, R, 11)
    U = torch.zeros_like(U)
    base = (cu(xp), cu(wp), cu(xs), cu(ws), cu(b))
    for epi in (native.EPI_F32, native.EPI_BF16, native.EPI_BF16_EAGER):
        a = native.int4_convrot_gemm_ex(*base, epi)
        c = native.int4_convrot_gemm_lora(*base, t.cuda(), U.cuda(), 1.0, epi)
        assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                           c.view(torch.int16) if c.dtype == torch.bfloat16 else c)


@pytest.mark.parametrize("M,N,K,G", [(77, 256, 3072, 256), (512, 3072, 3072, 256), (40, 200, 1088, 16),
                                     (1, 97, 128, 64), (257, 333, 2048, 256), (5, 1000, 12288, 256)])
def test_linear_with_fused_lora(backend, native, oracle, gpu, M, N, K, G):
    print(f"linear+lora M={M} N={N} K={K} G={G}", flush=True)
    x = outlier_activations(M, K, seed=M)
    w = normal_weight(N, K, seed=N)
    bias = normal_bias(N, seed=3)
    qw, ws = backend.quantize_convrot_w4a4_weight(w.cuda(), convrot_groupsize=G)
    rng = np.random.RandomState(K)
    pairs = []
    for r, s in ((16, 0.5), (48, 1.5)):
        down = torch.from_numpy((rng.standard_normal((r, K)) * 0.02).astype(np.float32))
        up = torch.from_numpy((rng.standard_normal((N, r)) * 0.1).astype(np.float32))
        pairs.append((down.cuda(), up.cuda(), s))
    D, U = backend.fuse_lora_pairs(pairs)
    assert D.shape == (64, K)
    xg = x.cuda()
    out = backend.convrot_w4a4_linear(xg, qw, ws, bias=bias.cuda(), convrot_groupsize=G, lora=(D, U))
    assert out.dtype == torch.bfloat16 and out.shape == (M, N)

    packed, xs, _ = oracle.rotquant(x.view(torch.int16).numpy().view(np.uint16), oracle.BF16, G)
    acc = oracle.int_gemm(packed, qw.cpu().numpy())
    main = oracle.epilogue_f32(acc, xs, ws.cpu().numpy(), bias.float().numpy()).astype(np.float64)
    xd = f64(x)
    lterm = sum(s * ((xd @ f64(d).T) @ f64(u).T) for d, u, s in pairs)
    ref = main + lterm
    got = f64(out)
    assert np.linalg.norm(lterm) > 0.3 * np.linalg.norm(main)          # the LoRA term matters
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-2
    assert np.linalg.norm((got - main) - lterm) / np.linalg.norm(lterm) < 1e-2
    # the same bits as the separate calls: the split down projection (whose
    # partials the linear sums inside its rotate+quant kernel) and the packed
    # GEMM with the LoRA epilogue
    tl = native.lora_down(xg, D)
    qx, xs2 = native.convrot_quant_int4(xg, G)
    sep = native.int4_convrot_gemm_lora(qx, qw, xs2, ws, bias.float().cuda(), tl, U, 1.0, native.EPI_BF16)
    assert torch.equal(out.view(torch.int16), sep.view(torch.int16))


def test_ops_forward_fused_and_side_path(backend, gpu):
    """Int4ConvRotOps.Linear with a plain LoRA (fused) and a LoHa-like adapter
    (h() side path): the forward equals the quantized layer without adapters
    plus every adapter's bypass term."""
    install_fake_comfy()
    from importlib import import_module, reload
    m = import_module("comfyui-int4-convrot-rdna4_amd.int4_ops")
    if m.Int4ConvRotOps is None:
        m = reload(m)
    Ops = m.Int4ConvRotOps
    M, N, K = 96, 512, 3072
    w, b = normal_weight(N, K, seed=21), normal_bias(N, seed=22)
    rng = np.random.RandomState(23)
    mk = lambda cls, r, alpha: cls(torch.from_numpy((rng.standard_normal((N, r)) * 0.1).astype(np.float32)),
                                   torch.from_numpy((rng.standard_normal((r, K)) * 0.02).astype(np.float32)),
                                   alpha)
    plain, other = mk(FakeLoRA, 16, 8.0), mk(FakeLoHa, 8, 8.0)

    base = Ops.Linear(K, N, bias=True)
    base.load_state_dict({"weight": w.clone(), "bias": b.clone()})
    assert base._qmode == "int4" and base._dyn_lora is None

    Ops.lora_patches = {"weight": [(plain, None, None, 0.8), (other, None, None, 1.0)]}
    Ops.lora_dynamic = True
    try:
        lin = Ops.Linear(K, N, bias=True)
        lin.load_state_dict({"weight": w.clone(), "bias": b.clone()})
    finally:
        Ops.lora_patches, Ops.lora_dynamic = {}, False
        Ops._applied_lora = set()
    assert lin._qmode == "int4" and lin._dyn_fused is not None and lin._dyn_rest == [other]
    assert torch.equal(lin._q, base._q)

    x = outlier_activations(M, K, seed=24).cuda()
    y = lin(x)
    y0 = base(x)
    want = y0.double() + plain.h(x, y0).double() + other.h(x, y0).double()
    err = (y.double() - want).norm() / want.norm()
    assert err < 1e-2, float(err)
    lora_part = (plain.h(x, y0) + other.h(x, y0)).double()
    assert ((y.double() - y0.double()) - lora_part).norm() / lora_part.norm() < 3e-2


@pytest.mark.parametrize("M,N,K,R", [(512, 3072, 3072, 32), (300, 1024, 12288, 64)])
def test_fused_lora_precision_vs_fp16_adapters(backend, native, gpu, M, N, K, R):
    """The fused side path rounds D, U * scale and t to bf16 (8 significant
    bits); the reference arms its adapters in fp16 (11 bits, int4_ops.py:
    165-168) and ComfyUI's h() computes from those (its rounding is not
    vendored).  Measured here: the fused LoRA term (f32 epilogue, with and
    without the adapter) against the fp64 closed form of the fp16 adapters,
    scale * (x @ D16^T) @ U16^T.  The bf16 roundings bound the error of each
    term by about 3 * 2^-9 of the magnitudes involved; the test holds the
    elementwise bound and reports the Frobenius error (below 1e-2 relative to
    the LoRA term, about 1e-3 of a typical LoRA term's own size per rounding)."""
    print(f"fused LoRA precision M={M} N={N} K={K} R={R}", flush=True)
    rs = np.random.RandomState(M + R)
    x = outlier_activations(M, K, seed=M + 1)
    qw, ws = backend.quantize_convrot_w4a4_weight(normal_weight(N, K, seed=N).cuda())
    w6 = backend.prepare_convrot_w4a4_weight_bf6(qw)
    down16 = torch.from_numpy((rs.standard_normal((R, K)) * 0.02).astype(np.float32)).to(torch.float16)
    up16 = torch.from_numpy((rs.standard_normal((N, R)) * 0.1).astype(np.float32)).to(torch.float16)
    scale = 0.8 * 16.0 / R                                   # strength * alpha / rank
    D, U = backend.fuse_lora_pairs([(down16.cuda(), up16.cuda(), scale)])
    xg = x.cuda()
    y_l = native.convrot_w4a4_linear_bf6(xg, w6, ws, None, D, U, 1.0, native.EPI_F32, 256, N)
    y_0 = native.convrot_w4a4_linear_bf6(xg, w6, ws, None, None, None, 1.0, native.EPI_F32, 256, N)
    ours = y_l.double().cpu().numpy() - y_0.double().cpu().numpy()
    xd = x.double().numpy()
    d16, u16 = down16.double().numpy(), up16.double().numpy()
    ref = scale * (xd @ d16.T) @ u16.T
    mag = scale * (np.abs(xd) @ np.abs(d16).T) @ np.abs(u16).T
    err = np.abs(ours - ref)
    # D, U*scale, t rounded to bf16 (2^-9 each), fp32 sums, and the f32 rounding of the two outputs
    ulp_y = np.spacing(np.maximum(np.abs(y_l.double().cpu().numpy()), np.abs(y_0.double().cpu().numpy())).astype(
        np.float32)).astype(np.float64)
    bound = 3.2 * 2.0 ** -9 * mag + 2 * ulp_y
    assert np.all(err <= bound), float((err / bound).max())
    rel = float(np.linalg.norm(ours - ref) / np.linalg.norm(ref))
    print(f"  relative Frobenius error of the fused LoRA term vs the fp16 closed form: {rel:.2e}", flush=True)
    assert rel < 1e-2
