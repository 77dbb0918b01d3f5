"""GPU parity of the W8A8 (int8) tier: the fused rotate + int8 quantizer
bit-exact against the oracle and the reference goldens, the int8 GEMM's int32
accumulators and epilogues bit-exact, the linear and the int8 layers of
Int4ConvRotOps (quantized on load or prequantized)."""
import hashlib
import importlib

import numpy as np
import pytest
import torch

from bf6_format import i8t_np
from inputs import (bf16_bits, clamp_rows8, config1_weight, edge_cases, normal_bias, normal_weight,
                    outlier_activations, small_w8a8_case)

pytestmark = pytest.mark.gpu

DT_OF = {torch.bfloat16: 1, torch.float16: 2, torch.float32: 0}


def np_of(t):
    t = t.detach().cpu()
    return t.numpy() if t.dtype == torch.float32 else t.contiguous().view(torch.int16).numpy().view(np.uint16)


def cu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


QUANT_CASES = [(1, 256, 256, torch.bfloat16), (7, 80, 16, torch.bfloat16), (33, 192, 64, torch.bfloat16),
               (300, 3072, 256, torch.bfloat16), (64, 12288, 256, torch.bfloat16), (5, 16384, 256, torch.bfloat16),
               (3, 32768, 256, torch.bfloat16), (65, 3072, 256, torch.float16), (17, 512, 64, torch.float32),
               (4608, 3072, 256, torch.bfloat16)]


@pytest.mark.parametrize("M,K,G,dt", QUANT_CASES)
def test_quant_int8_matches_oracle(native, oracle, gpu, M, K, G, dt):
    print(f"quant8 M={M} K={K} G={G} {dt}", flush=True)
    x = outlier_activations(M, K, seed=M + K, student_t=(K == 3072), dtype=dt)
    q, s = native.convrot_quant_int8(x.cuda(), G)
    rows = np.arange(M) if M <= 512 else np.random.RandomState(0).choice(M, 64, replace=False)
    qo, so, _ = oracle.rotquant8(np_of(x)[rows], DT_OF[dt], G)
    assert np.array_equal(q.cpu().numpy()[rows], qo)
    assert np.array_equal(s.cpu().numpy()[rows], so)


@pytest.mark.parametrize("name", list(edge_cases().keys()))
def test_quant_int8_edge_goldens(native, oracle, goldens, gpu, name):
    xe, G = edge_cases()[name]
    q, s = native.convrot_quant_int8(xe.cuda(), G)
    if xe.dtype == torch.float32:     # torch's fp32 rotation is not correctly rounded: compare to the oracle
        qo, so, _ = oracle.rotquant8(np_of(xe), 0, G)
        assert np.array_equal(q.cpu().numpy(), qo) and np.array_equal(s.cpu().numpy(), so)
    else:
        assert np.array_equal(q.cpu().numpy(), goldens[f"i8_edge_{name}_q"])
        assert np.array_equal(s.cpu().numpy(), goldens[f"i8_edge_{name}_s"])


def test_quant_int8_largest_quotient(native, goldens, gpu):
    q, s = native.convrot_quant_int8(clamp_rows8().cuda(), 16)
    assert np.array_equal(q.cpu().numpy(), goldens["i8_maxq_q"])
    assert np.array_equal(s.cpu().numpy(), goldens["i8_maxq_s"])


def test_weight_int8_config1_golden(backend, goldens, gpu):
    i8 = importlib.import_module(backend.__name__ + ".int8_eager")
    qw, ws = i8.quantize_convrot_w8a8_weight(config1_weight().cuda(), convrot_groupsize=256)
    qw = qw.cpu().numpy()
    assert np.array_equal(qw[:64], goldens["i8_c1_qw_rows64"])
    assert sha(qw) == str(goldens["i8_c1_qw_sha"])
    assert np.array_equal(ws.cpu().numpy(), goldens["i8_c1_wscale"])


ACC_SHAPES = [(1, 1, 16), (3, 5, 48), (64, 48, 256), (300, 200, 160), (257, 513, 1024), (100, 300, 3840),
              (16, 700, 80), (512, 256, 12288), (31, 33, 4112), (5, 9, 64), (12, 70, 128), (40, 33, 192)]


@pytest.mark.parametrize("M,N,K", ACC_SHAPES)
def test_int8_acc_bitexact(native, oracle, gpu, M, N, K):
    rs = np.random.RandomState(M + N + K)
    X = rs.randint(-128, 128, size=(M, K)).astype(np.int8)
    W = rs.randint(-128, 128, size=(N, K)).astype(np.int8)
    acc = native.int8_gemm_acc(cu(X), cu(W)).cpu().numpy()
    assert np.array_equal(acc, oracle.int8_gemm(X, W))


def test_int8_acc_extremes(native, gpu):
    """|acc| = 128^2 K = 2^27 at K = 8192 (all -128): exact int32, beyond fp32 integers."""
    M, N, K = 256, 256, 8192
    X = torch.full((M, K), -128, dtype=torch.int8, device="cuda")
    W = torch.full((N, K), -128, dtype=torch.int8, device="cuda")
    W[1::2] = 127
    acc = native.int8_gemm_acc(X, W)
    assert torch.all(acc[:, 0::2] == 128 * 128 * K) and torch.all(acc[:, 1::2] == -128 * 127 * K)


def test_int8_acc_full_size(native, gpu):
    M, N, K = 4608, 3072, 3072
    g = torch.Generator(device="cuda").manual_seed(5)
    X = torch.randint(-127, 128, (M, K), generator=g, device="cuda", dtype=torch.int8)
    W = torch.randint(-127, 128, (N, K), generator=g, device="cuda", dtype=torch.int8)
    acc = native.int8_gemm_acc(X, W)
    ref = (X.double() @ W.double().T).to(torch.int32)       # exact: |acc| < 2^53
    assert torch.equal(acc, ref)


@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("M,N,K", [(64, 48, 256), (257, 300, 3072), (33, 513, 1040)])
def test_int8_epilogues_bitexact(native, oracle, gpu, M, N, K, bias):
    rs = np.random.RandomState(3 * M + N)
    X = rs.randint(-127, 128, size=(M, K)).astype(np.int8)
    W = rs.randint(-127, 128, size=(N, K)).astype(np.int8)
    xs = rs.uniform(0.005, 0.05, size=M).astype(np.float32)
    ws = rs.uniform(0.005, 0.05, size=N).astype(np.float32)
    b = (rs.standard_normal(N) * 0.01).astype(np.float32) if bias else None
    acc = oracle.int8_gemm(X, W)
    args = (cu(X), cu(W), cu(xs), cu(ws), cu(b) if bias else None)
    f32 = native.int8_convrot_gemm(*args, torch.float32).cpu().numpy()
    assert np.array_equal(f32.view(np.uint32), oracle.epilogue_f32(acc, xs, ws, b).view(np.uint32))
    bf = np_of(native.int8_convrot_gemm(*args, torch.bfloat16))
    assert np.array_equal(bf, oracle.epilogue_f32(acc, xs, ws, b, out_bf16=True))


def test_linear_w8a8_golden(backend, oracle, goldens, gpu):
    """The whole W8A8 linear against the reference eager output (K = 512: its
    fp32 matmul is exact) and the oracle."""
    i8 = importlib.import_module(backend.__name__ + ".int8_eager")
    x, w, b = small_w8a8_case()
    qw, ws = i8.quantize_convrot_w8a8_weight(w.cuda(), convrot_groupsize=256)
    assert np.array_equal(qw.cpu().numpy(), goldens["i8_lin_qw"])
    y = backend.convrot_w8a8_linear(x.cuda(), qw, ws, bias=b.cuda(), convrot_groupsize=256)
    assert y.dtype == torch.bfloat16 and y.shape == (64, 96)
    assert np.array_equal(np_of(y), goldens["i8_lin_y"])


@pytest.mark.parametrize("M,N,K", [(256, 3072, 3072), (77, 640, 12288), (4608, 3072, 3072)])
def test_linear_w8a8_matches_oracle(backend, oracle, gpu, M, N, K):
    print(f"w8a8 linear M={M} N={N} K={K}", flush=True)
    i8 = importlib.import_module(backend.__name__ + ".int8_eager")
    x = outlier_activations(M, K, seed=M + 1)
    w, b = normal_weight(N, K, seed=N + 2), normal_bias(N, seed=N + 3)
    qw, ws = i8.quantize_convrot_w8a8_weight(w.cuda(), convrot_groupsize=256)
    y = backend.convrot_w8a8_linear(x.cuda().reshape(1, M, K), qw, ws, bias=b.cuda(), convrot_groupsize=256)
    assert y.shape == (1, M, N)
    rows = np.arange(M) if M <= 256 else np.random.RandomState(1).choice(M, 48, replace=False)
    want = oracle.linear_w8a8(np_of(x)[rows], oracle.BF16, qw.cpu().numpy(), ws.cpu().numpy(),
                              b.float().numpy(), 256)
    assert np.array_equal(np_of(y[0])[rows], want)
    # and against the unquantized product (the int8 tier's accuracy)
    ref = x.float() @ w.float().T + b.float()
    err = float((y[0].float().cpu() - ref).norm() / ref.norm())
    assert err < 0.02, err


def test_dequantize_w8a8_roundtrip(backend, gpu):
    i8 = importlib.import_module(backend.__name__ + ".int8_eager")
    w = normal_weight(64, 512, seed=31)
    qw, ws = i8.quantize_convrot_w8a8_weight(w.cuda(), convrot_groupsize=64)
    deq = i8.dequantize_convrot_w8a8_weight(qw, ws, convrot_groupsize=64).cpu()
    # per-row error below half a step in the rotated basis (orthogonal rotation keeps the norm)
    err = (deq - w.float()).norm(dim=1)
    assert torch.all(err <= 0.5 * ws.cpu() * (512 ** 0.5) * 1.01)


def _ops():
    from fake_comfy import install_fake_comfy
    install_fake_comfy()
    m = importlib.import_module("comfyui-int4-convrot-rdna4_amd.int4_ops")
    if m.Int4ConvRotOps is None:
        m = importlib.reload(m)
    return m.Int4ConvRotOps


# ---------------------------------------------------------------------------
# I8T: the tile-major int8 operand layout of the W8A8 GEMM (the linear's path
# when K % 64 == 0)
# ---------------------------------------------------------------------------

I8T_QUANT_CASES = [(1, 256, 256, torch.bfloat16), (33, 192, 64, torch.bfloat16), (300, 3072, 256, torch.bfloat16),
                   (257, 12288, 256, torch.bfloat16), (65, 3072, 256, torch.float16), (17, 512, 64, torch.float32),
                   (8, 64, 16, torch.bfloat16)]


@pytest.mark.parametrize("M,K,G,dt", I8T_QUANT_CASES)
def test_quant_int8_i8t_layout(native, gpu, M, K, G, dt):
    x = outlier_activations(M, K, seed=M + K, dtype=dt).cuda()
    q, s = native.convrot_quant_int8(x, G)
    q8t, s8t = native.convrot_quant_int8_i8t(x, G)
    assert torch.equal(s8t, s)
    want = i8t_np(q.cpu().numpy())
    assert np.array_equal(q8t.cpu().numpy(), want)
    assert np.array_equal(native.int8_to_i8t(q).cpu().numpy(), want)


I8T_GEMM_SHAPES = [(64, 48, 256), (257, 300, 3072), (33, 513, 1088), (512, 256, 64), (300, 700, 12288),
                   (20, 40, 128), (70, 90, 192)]   # one to three 64-k blocks


@pytest.mark.parametrize("M,N,K", I8T_GEMM_SHAPES)
def test_int8_i8t_gemm_bitexact(native, oracle, gpu, M, N, K):
    rs = np.random.RandomState(7 * M + N + K)
    X = rs.randint(-128, 128, size=(M, K)).astype(np.int8)
    W = rs.randint(-128, 128, size=(N, K)).astype(np.int8)
    xs = rs.uniform(0.005, 0.05, size=M).astype(np.float32)
    ws = rs.uniform(0.005, 0.05, size=N).astype(np.float32)
    b = (rs.standard_normal(N) * 0.01).astype(np.float32)
    a8t, w8t = native.int8_to_i8t(cu(X)), native.int8_to_i8t(cu(W))
    acc = oracle.int8_gemm(X, W)
    got = native.int8_convrot_gemm_i8t(a8t, w8t, None, None, None, native.EPI_ACC, M, N).cpu().numpy()
    assert np.array_equal(got, acc)
    f32 = native.int8_convrot_gemm_i8t(a8t, w8t, cu(xs), cu(ws), cu(b), native.EPI_F32, M, N).cpu().numpy()
    assert np.array_equal(f32.view(np.uint32), oracle.epilogue_f32(acc, xs, ws, b).view(np.uint32))
    bf = np_of(native.int8_convrot_gemm_i8t(a8t, w8t, cu(xs), cu(ws), None, native.EPI_BF16, M, N))
    assert np.array_equal(bf, oracle.epilogue_f32(acc, xs, ws, None, out_bf16=True))


def test_int8_i8t_gemm_full_size_matches_row_major(native, gpu):
    M, N, K = 4608, 3072, 3072
    g = torch.Generator(device="cuda").manual_seed(6)
    X = torch.randint(-127, 128, (M, K), generator=g, device="cuda", dtype=torch.int8)
    W = torch.randint(-127, 128, (N, K), generator=g, device="cuda", dtype=torch.int8)
    xs = torch.rand(M, generator=g, device="cuda") * 0.01
    ws = torch.rand(N, generator=g, device="cuda") * 0.01
    b = torch.rand(N, generator=g, device="cuda") * 0.01
    ref = native.int8_convrot_gemm(X, W, xs, ws, b, torch.bfloat16)
    got = native.int8_convrot_gemm_i8t(native.int8_to_i8t(X), native.int8_to_i8t(W), xs, ws, b,
                                       native.EPI_BF16, M, N)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_linear_w8a8_i8t_and_row_major_paths_agree(backend, native, gpu):
    """K % 64 == 0 takes the I8T path; the same linear through the row-major
    kernels gives the same bits."""
    M, N, K = 129, 384, 3072
    x = outlier_activations(M, K, seed=61).cuda()
    w = normal_weight(N, K, seed=62, dtype=torch.float16).cuda()
    b = normal_bias(N, seed=63).cuda()
    int8_eager = importlib.import_module("comfyui-int4-convrot-rdna4_amd._int4.int8_eager")
    qw, ws = int8_eager.quantize_convrot_w8a8_weight(w, 256)
    assert backend.i8t_path_ok(K)
    y = backend.convrot_w8a8_linear(x, qw, ws, bias=b, convrot_groupsize=256,
                                    qweight_i8t=backend.prepare_convrot_w8a8_weight_i8t(qw))
    qa, xs = native.convrot_quant_int8(x, 256)
    ref = native.int8_convrot_gemm(qa, qw, xs, ws, b, torch.bfloat16)
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))


def test_ops_int8_layer_quantized_on_load(backend, oracle, gpu):
    Ops = _ops()
    M, N, K = 96, 640, 3072
    w, b = normal_weight(N, K, seed=41, dtype=torch.bfloat16), normal_bias(N, seed=42)
    Ops.int8_exact = {"blk.lin"}
    try:
        lin = Ops.Linear(K, N, bias=True)
        lin.load_state_dict({"weight": w.clone(), "bias": b.clone()}, strict=False)
        # the exact key is the prefix the loader passes: emulate it through a parent module
        parent = torch.nn.Module()
        parent.blk = torch.nn.Module()
        parent.blk.lin = Ops.Linear(K, N, bias=True)
        parent.load_state_dict({"blk.lin.weight": w.clone(), "blk.lin.bias": b.clone()})
    finally:
        Ops.int8_exact = set()
    assert lin._qmode == "int4"
    m = parent.blk.lin
    assert m._qmode == "int8" and m._q.shape == (N, K) and m._q.dtype == torch.int8 and m._q6 is None
    assert m._q8t is not None and m._q8t.shape == ((N + 255) // 256 * 256, K)
    qw, ws = oracle.quantize_weight8(np_of(w.to(torch.float16)), oracle.F16, 256)
    assert np.array_equal(m._q.cpu().numpy(), qw) and np.array_equal(m._qs.cpu().numpy(), ws)
    x = outlier_activations(M, K, seed=43)
    y = m(x.cuda())
    want = oracle.linear_w8a8(np_of(x), oracle.BF16, qw, ws, m.bias.float().cpu().numpy(), 256)
    assert np.array_equal(np_of(y), want)


def test_ops_int8_prequantized_load(backend, oracle, gpu):
    """A ComfyUI-native int8 ConvRot layer (int8 [N, K] weight, [N, 1] scale,
    comfy_quant tag) loads as stored and runs the W8A8 path."""
    import json
    Ops = _ops()
    M, N, K = 40, 256, 1024
    w = normal_weight(N, K, seed=51)
    qw, ws = oracle.quantize_weight8(np_of(w), oracle.F16, 256)
    tag = torch.tensor(list(json.dumps({"format": "int8_tensorwise", "convrot": True,
                                        "convrot_groupsize": 256}).encode()), dtype=torch.uint8)
    lin = Ops.Linear(K, N, bias=False)
    lin.load_state_dict({"weight": torch.from_numpy(qw), "weight_scale": torch.from_numpy(ws).reshape(N, 1),
                         "comfy_quant": tag}, strict=False)
    assert lin._qmode == "int8" and lin._qgs == 256
    x = outlier_activations(M, K, seed=52)
    y = lin(x.cuda())
    assert np.array_equal(np_of(y), oracle.linear_w8a8(np_of(x), oracle.BF16, qw, ws, None, 256))
