"""GPU parity at the benchmark configurations, at their full sizes.

C1  the single linear (x bf16 [256, 3072] with outlier channels, W fp16
    [3072, 3072], fp16 bias) end to end through ``_int4.convrot_w4a4_linear``:
    bit-exact against the oracle's f32 epilogue, within 1e-2 relative
    Frobenius of the reference eager output (golden rows + SHA-pinned oracle),
    and, with linear_dtype="int8" (the reference's eager route), equal to the
    reference eager output bit for bit (its SHA-256 golden).
C2  the four Flux block linears at M = 4608 through ``Int4ConvRotOps.Linear``:
    sampled rows bit-exact against the oracle, the eager chain within 1e-2, and
    the whole tensor equal to the packed int8-MFMA kernels' output.
C4  the GEMM token sweep M in {1024 .. 16384} x (K, N) in {(3072, 3072),
    (3072, 12288), (12288, 3072), (3840, 15360)} with codes uniform in [-8, 7]:
    the bf6 GEMM's accumulators equal an exact fp32 GEMM of the codes over the
    whole tensor and the oracle on sampled rows; the bf16 epilogue matches the
    oracle on the sampled rows."""
import hashlib

import numpy as np
import pytest
import torch

from inputs import (bf16_bits, config1_bias, config1_weight, config1_x, normal_bias, normal_weight,
                    outlier_activations)

pytestmark = pytest.mark.gpu


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def u16(t):
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def bf16_f64(b):
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def rel_fro(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


# ----------------------------------------------------------------------------
# C1
# ----------------------------------------------------------------------------

def test_config1_linear_end_to_end(backend, native, oracle, goldens, gpu):
    print("config1 linear 256x3072->3072", flush=True)
    x, w, b = config1_x(), config1_weight(), config1_bias()
    qw, ws = backend.quantize_convrot_w4a4_weight(w.cuda())          # fp16, as the Linear loads it
    qw_np, ws_np = qw.cpu().numpy(), ws.cpu().numpy()
    assert sha(qw_np) == str(goldens["c1_qw_sha"])
    assert np.array_equal(ws_np, goldens["c1_wscale"])
    y = backend.convrot_w4a4_linear(x.cuda(), qw, ws, bias=b.cuda(), convrot_groupsize=256)
    assert y.dtype == torch.bfloat16 and y.shape == (256, 3072)
    # bit-exact: the oracle's codes, exact accumulators, the f32 epilogue rounded once
    qx, xs, _ = oracle.rotquant(bf16_bits(x), oracle.BF16, 256)
    assert np.array_equal(qx, goldens["c1_qact"]) and np.array_equal(xs, goldens["c1_xscale"])
    acc = oracle.int_gemm(qx, qw_np)
    want = oracle.epilogue_f32(acc, xs, ws_np, b.float().numpy(), out_bf16=True)
    assert np.array_equal(u16(y), want)
    # the packed-operand C-ABI kernels give the same bits
    q2, s2 = native.convrot_quant_int4(x.cuda(), 256)
    y2 = native.int4_convrot_gemm(q2, qw, s2, ws, b.float().cuda(), torch.bfloat16)
    assert np.array_equal(u16(y2), want)
    # against the reference eager output: its first 32 rows are a golden, the
    # whole tensor is the oracle's eager chain, SHA-pinned to the reference's
    eager = oracle.linear_eager(bf16_bits(x), oracle.BF16, qw_np, ws_np, b.float().numpy(), 256)
    assert sha(eager) == str(goldens["c1_y_sha"])
    assert np.array_equal(eager[:32], goldens["c1_y_rows32"])
    err = rel_fro(bf16_f64(u16(y)), bf16_f64(eager))
    assert err <= 1e-2, err
    # linear_dtype="int8": the reference's eager route, reproduced bit for bit
    y8 = backend.convrot_w4a4_linear(x.cuda(), qw, ws, bias=b.cuda(), convrot_groupsize=256, linear_dtype="int8")
    assert sha(u16(y8)) == str(goldens["c1_y_sha"])
    # and on the packed int8-MFMA path (K % 128 == 0 is not needed there)
    y8p = native.int4_convrot_gemm_ex(q2, qw, s2, ws, b.float().cuda(), native.EPI_BF16_EAGER)
    assert sha(u16(y8p)) == str(goldens["c1_y_sha"])


def test_config1_linear_f32_activations(backend, oracle, gpu):
    """f32 x: the eager route and the default epilogue are the same fp32
    chain; both equal the oracle's eager f32 output bit for bit."""
    x = config1_x().float()
    qw, ws = backend.quantize_convrot_w4a4_weight(config1_weight().cuda())
    b = config1_bias()
    want = oracle.linear_eager(x.numpy(), oracle.F32, qw.cpu().numpy(), ws.cpu().numpy(), b.float().numpy(), 256)
    for ld in ("int4", "int8"):
        y = backend.convrot_w4a4_linear(x.cuda(), qw, ws, bias=b.cuda(), linear_dtype=ld)
        assert y.dtype == torch.float32
        assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32)), ld


# ----------------------------------------------------------------------------
# C2
# ----------------------------------------------------------------------------

FLUX_LINEARS = [("qkv", 3072, 9216), ("proj", 3072, 3072), ("mlp_up", 3072, 12288), ("mlp_down", 12288, 3072)]


@pytest.fixture(scope="module")
def ops_cls(gpu):
    from fake_comfy import install_fake_comfy
    install_fake_comfy()
    from importlib import import_module, reload
    m = import_module("comfyui-int4-convrot-rdna4_amd.int4_ops")
    if m.Int4ConvRotOps is None:
        m = reload(m)
    return m.Int4ConvRotOps


@pytest.mark.parametrize("name,K,N", FLUX_LINEARS)
def test_config2_flux_linear(ops_cls, native, oracle, gpu, name, K, N):
    M = 4608
    print(f"config2 {name} {M}x{K}->{N}", flush=True)
    lin = ops_cls.Linear(K, N, bias=True)
    w = normal_weight(N, K, seed=K + N).to(torch.bfloat16)     # a bf16 checkpoint weight
    b = normal_bias(N, seed=N + 1).to(torch.bfloat16)
    lin.load_state_dict({"weight": w, "bias": b})
    assert lin._qmode == "int4" and lin._q6 is not None
    lin = lin.cuda()
    x = outlier_activations(M, K, seed=M + K).cuda()
    with torch.no_grad():
        y = lin(x)
    assert y.shape == (M, N) and y.dtype == torch.bfloat16
    bias32 = lin.bias.float()
    # the whole tensor against the packed-operand int8-MFMA kernels
    qx, xs = native.convrot_quant_int4(x, 256)
    y2 = native.int4_convrot_gemm(qx, lin._q, xs, lin._qs, bias32, torch.bfloat16)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
    # sampled rows against the oracle: codes, scales, f32 epilogue bit-exact
    rows = np.sort(np.random.RandomState(K + N).choice(M, 16, replace=False))
    xb = bf16_bits(x[torch.from_numpy(rows).cuda()].cpu())
    eqx, exs, _ = oracle.rotquant(xb, oracle.BF16, 256)
    assert np.array_equal(qx.cpu().numpy()[rows], eqx) and np.array_equal(xs.cpu().numpy()[rows], exs)
    qw, ws = lin._q.cpu().numpy(), lin._qs.cpu().numpy()
    acc = oracle.int_gemm(eqx, qw)
    want = oracle.epilogue_f32(acc, exs, ws, bias32.cpu().numpy(), out_bf16=True)
    got = u16(y)[rows]
    assert np.array_equal(got, want)
    eager = oracle.epilogue_eager_bf16(acc, exs, ws, bias32.cpu().numpy())
    assert rel_fro(bf16_f64(got), bf16_f64(eager)) <= 1e-2


# ----------------------------------------------------------------------------
# C4
# ----------------------------------------------------------------------------

SWEEP_KN = [(3072, 3072), (3072, 12288), (12288, 3072), (3840, 15360)]
SWEEP_M = [1024, 2048, 4608, 8192, 16384]


def unpack_codes(p):
    p = p.to(torch.int32)
    return torch.stack([(p << 28) >> 28, (p << 24) >> 28], -1).reshape(p.shape[0], -1).float()


@pytest.mark.parametrize("K,N", SWEEP_KN)
@pytest.mark.parametrize("M", SWEEP_M)
def test_config4_token_sweep(native, oracle, gpu, M, K, N):
    print(f"config4 sweep {M}x{K}->{N}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(M * 7 + K + N)
    xp = torch.randint(-128, 128, (M, K // 2), generator=g, device="cuda", dtype=torch.int32).to(torch.int8)
    wp = torch.randint(-128, 128, (N, K // 2), generator=g, device="cuda", dtype=torch.int32).to(torch.int8)
    xs = torch.empty(M, device="cuda").uniform_(0.005, 0.05, generator=g)
    ws = torch.empty(N, device="cuda").uniform_(0.005, 0.05, generator=g)
    b = (torch.randn(N, generator=g, device="cuda") * 0.01)
    a6, w6 = native.int4_to_bf6(xp), native.int4_to_bf6(wp)
    acc = native.int4_gemm_acc_bf6(a6, w6, M, N)
    # exact fp32 GEMM of the codes: every partial sum is an integer below 2^24
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False     # restored below: later tests keep their setting
    try:
        ref = (unpack_codes(xp) @ unpack_codes(wp).T).to(torch.int32)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev
    assert torch.equal(acc, ref)
    del ref
    out = native.int4_convrot_gemm_bf6(a6, w6, xs, ws, b, native.EPI_BF16)
    rows = np.sort(np.random.RandomState(M + N).choice(M, 6, replace=False))
    ri = torch.from_numpy(rows).cuda()
    xp_r, wp_np = xp[ri].cpu().numpy(), wp.cpu().numpy()
    eacc = oracle.int_gemm(xp_r, wp_np)
    assert np.array_equal(acc[ri].cpu().numpy(), eacc)
    want = oracle.epilogue_f32(eacc, xs[ri].cpu().numpy(), ws.cpu().numpy(), b.cpu().numpy(), out_bf16=True)
    assert np.array_equal(u16(out[ri]), want)
