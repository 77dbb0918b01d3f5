"""Seeded sweep of ragged linear shapes through the Linear's forward path
(convrot_w4a4_linear: fused rotate+quantize, GEMM, dequant epilogue), bf16, f16
and f32 activations, with and without bias, rows of 64 to 12288 elements.  Every bit equals the oracle's: the
weight quantizer's codes and scales, then rotate+quantize of x, the integer
GEMM and the f32 epilogue.  K multiples of 128 take the bf6 GEMM, the other
multiples of 64 the int8-MFMA GEMM (groupsize 256 or 64 as picked from K)."""
import numpy as np
import pytest
import torch

from inputs import bf16_bits, normal_bias, normal_weight, outlier_activations

pytestmark = pytest.mark.gpu


def _shapes(n=32, seed=2024):
    rs = np.random.RandomState(seed)
    out = []
    for i in range(n):
        M = int(rs.choice([1, 2, 3, 7, 31, 33, 64, 100, 255, 257, 300, 513]))
        N = int(rs.randint(1, 700))
        K = 64 * int(rs.randint(1, 49))          # 64 .. 3072
        out.append((M, N, K, "bf16" if i % 3 else "f32", bool(rs.randint(2))))
    return out


@pytest.mark.parametrize("M,N,K,dt,has_bias", _shapes())
def test_linear_sweep_vs_oracle(backend, oracle, gpu, M, N, K, dt, has_bias):
    print(f"linear sweep M={M} N={N} K={K} {dt} bias={has_bias}", flush=True)
    G = backend.pick_groupsize(K)
    # f32 activations hold bf16-grid values: every fp64 group sum is exact
    x = outlier_activations(M, K, seed=7 * M + K, dtype=torch.bfloat16)
    w = normal_weight(N, K, seed=N + K)
    b = normal_bias(N, seed=N) if has_bias else None

    qw, ws = backend.quantize_convrot_w4a4_weight(w.cuda(), convrot_groupsize=G)
    eqw, ews = oracle.quantize_weight(w.view(torch.int16).numpy().view(np.uint16), oracle.F16, G)
    assert np.array_equal(qw.cpu().numpy(), eqw)
    assert np.array_equal(ws.cpu().numpy().view(np.uint32), ews.view(np.uint32))

    xin = x if dt == "bf16" else x.float()
    y = backend.convrot_w4a4_linear(xin.cuda(), qw, ws, bias=None if b is None else b.cuda(), convrot_groupsize=G)
    assert y.shape == (M, N) and y.dtype == xin.dtype

    if dt == "bf16":
        eqx, exs, _ = oracle.rotquant(bf16_bits(x), oracle.BF16, G)
    else:
        eqx, exs, _ = oracle.rotquant(x.float().numpy(), oracle.F32, G)
    acc = oracle.int_gemm(eqx, eqw)
    bias32 = None if b is None else b.float().numpy()
    if dt == "bf16":
        want = oracle.epilogue_f32(acc, exs, ews, bias32, out_bf16=True)
        assert np.array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16), want)
    else:
        want = oracle.epilogue_f32(acc, exs, ews, bias32, out_bf16=False)
        assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))


def _long_shapes(n=12, seed=2025):
    rs = np.random.RandomState(seed)
    out = []
    for i in range(n):
        M = int(rs.choice([300, 513, 1025, 2049]))
        N = int(rs.randint(1, 1500))
        K = 128 * int(rs.randint(33, 97))        # 4224 .. 12288: the 256 x 256 kernel, split or not
        out.append((M, N, K, bool(rs.randint(2))))
    # enough 256 x 256 tiles that the host rule runs them unsplit
    return out + [(4099, 1301, 4224, True), (3000, 2000, 6144, False), (4097, 3001, 8320, True)]


@pytest.mark.parametrize("M,N,K,has_bias", _long_shapes())
def test_linear_sweep_long_rows_vs_oracle(backend, native, oracle, gpu, M, N, K, has_bias):
    """Long rows (K > 4096) and up to 2049 tokens: the 256 x 256 kernel with and
    without its k-split on ragged shapes.  Codes, scales and sampled output rows
    bit-exact against the oracle."""
    print(f"linear sweep long M={M} N={N} K={K} bias={has_bias} nsplit={native.choose_nsplit_bf6(M, N, K)}", flush=True)
    G = backend.pick_groupsize(K)
    x = outlier_activations(M, K, seed=11 * M + K, dtype=torch.bfloat16)
    w = normal_weight(N, K, seed=3 * N + K)
    b = normal_bias(N, seed=N + 1) if has_bias else None
    qw, ws = backend.quantize_convrot_w4a4_weight(w.cuda(), convrot_groupsize=G)
    y = backend.convrot_w4a4_linear(x.cuda(), qw, ws, bias=None if b is None else b.cuda(), convrot_groupsize=G)
    assert y.shape == (M, N) and y.dtype == torch.bfloat16
    rows = np.concatenate([np.random.RandomState(M + N).choice(M, 12, replace=False), [0, M - 1]])
    eqx, exs, _ = oracle.rotquant(bf16_bits(x[rows]), oracle.BF16, G)
    eqw, ews = oracle.quantize_weight(w.view(torch.int16).numpy().view(np.uint16), oracle.F16, G)
    assert np.array_equal(qw.cpu().numpy(), eqw)
    acc = oracle.int_gemm(eqx, eqw)
    want = oracle.epilogue_f32(acc, exs, ews, None if b is None else b.float().numpy(), out_bf16=True)
    assert np.array_equal(y.cpu()[rows].view(torch.int16).numpy().view(np.uint16), want)


F16_SHAPES = [(1, 64, 64, True), (257, 129, 192, False), (33, 200, 256, True), (300, 1000, 3072, False),
              (513, 777, 4224, True), (2049, 1500, 12288, False), (4099, 1301, 4224, True)]


@pytest.mark.parametrize("M,N,K,has_bias", F16_SHAPES)
def test_linear_f16_activations_vs_oracle(backend, native, oracle, gpu, M, N, K, has_bias):
    """fp16 activations and an fp16 bias (as the loader keeps it): the output is the
    f32 epilogue cast to fp16, as the reference's native path returns it.  The
    int8 GEMM (K = 192), the 128 x 128 kernel and the 256 x 256 kernel split and
    unsplit; codes, scales and sampled output rows bit-exact against the oracle."""
    print(f"linear f16 M={M} N={N} K={K} bias={has_bias}", flush=True)
    G = backend.pick_groupsize(K)
    x = outlier_activations(M, K, seed=5 * M + K, dtype=torch.float16)
    w = normal_weight(N, K, seed=N + 2 * K)
    b = normal_bias(N, seed=N + 3).to(torch.float16) if has_bias else None
    qw, ws = backend.quantize_convrot_w4a4_weight(w.cuda(), convrot_groupsize=G)
    y = backend.convrot_w4a4_linear(x.cuda(), qw, ws, bias=None if b is None else b.cuda(), convrot_groupsize=G)
    assert y.shape == (M, N) and y.dtype == torch.float16
    rows = np.unique(np.concatenate([np.random.RandomState(M + K).choice(M, min(M, 12), replace=False), [0, M - 1]]))
    eqx, exs, _ = oracle.rotquant(x[rows].view(torch.int16).numpy().view(np.uint16), oracle.F16, G)
    eqw, ews = oracle.quantize_weight(w.view(torch.int16).numpy().view(np.uint16), oracle.F16, G)
    assert np.array_equal(qw.cpu().numpy(), eqw)
    acc = oracle.int_gemm(eqx, eqw)
    want = oracle.epilogue_f32(acc, exs, ews, None if b is None else b.float().numpy(), out_bf16=False)
    got = y.cpu()[torch.from_numpy(rows)].numpy()
    assert np.array_equal(got.view(np.uint16), want.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("M,N,K,has_bias", F16_SHAPES)
def test_linear_genuine_f32_activations_vs_oracle(backend, native, oracle, gpu, M, N, K, has_bias):
    """f32 activations with full 24-bit significands (the sweep above keeps f32
    values on the bf16 grid): f32 output bit-exact on sampled rows against the
    eager quantizer, the integer GEMM and the f32 epilogue applied to the
    kernel's fp64 rotation restated on the CPU."""
    from fp64_rotation import rotate_fp64_kernel_order
    print(f"linear f32 M={M} N={N} K={K} bias={has_bias}", flush=True)
    G = backend.pick_groupsize(K)
    x = outlier_activations(M, K, seed=9 * M + K, dtype=torch.float32)
    w = normal_weight(N, K, seed=N + 5 * K)
    b = normal_bias(N, seed=N + 4) if has_bias else None
    qw, ws = backend.quantize_convrot_w4a4_weight(w.cuda(), convrot_groupsize=G)
    y = backend.convrot_w4a4_linear(x.cuda(), qw, ws, bias=None if b is None else b.cuda(), convrot_groupsize=G)
    assert y.shape == (M, N) and y.dtype == torch.float32
    rows = np.unique(np.concatenate([np.random.RandomState(M + 2 * K).choice(M, min(M, 12), replace=False), [0, M - 1]]))
    xr = rotate_fp64_kernel_order(x[torch.from_numpy(rows)].contiguous().numpy(), G, oracle.F32)
    eqx, exs, _ = oracle.quant_rows(xr, oracle.F32)
    eqw, ews = oracle.quantize_weight(w.view(torch.int16).numpy().view(np.uint16), oracle.F16, G)
    assert np.array_equal(qw.cpu().numpy(), eqw)
    acc = oracle.int_gemm(eqx, eqw)
    want = oracle.epilogue_f32(acc, exs, ews, None if b is None else b.float().numpy(), out_bf16=False)
    assert np.array_equal(y.cpu()[torch.from_numpy(rows)].numpy().view(np.uint32), want.view(np.uint32))
