"""Seeded sweep of ragged shapes through the W8A8 tier's linear
(convrot_w8a8_linear: fused rotate + int8 quantize, int8 GEMM, dequant
epilogue), bf16 and f32 activations, with and without bias.  Every bit equals
the oracle's: the weight quantizer's int8 codes and scales, then the whole
linear (rotate + quantize x, exact int32 GEMM, f32 epilogue).  K multiples of
64 take the tile-major I8T GEMM, the other multiples of 16 the row-major int8
GEMM; the groupsize is the largest of 256 / 64 / 16 dividing K."""
import importlib

import numpy as np
import pytest
import torch

from inputs import bf16_bits, normal_bias, normal_weight, outlier_activations

pytestmark = pytest.mark.gpu


def _shapes(n=24, seed=4096):
    rs = np.random.RandomState(seed)
    out = []
    for i in range(n):
        M = int(rs.choice([1, 5, 16, 33, 100, 257, 511]))
        N = int(rs.randint(1, 600))
        K = 16 * int(rs.randint(1, 193))         # 16 .. 3072
        out.append((M, N, K, "bf16" if i % 3 else "f32", bool(rs.randint(2))))
    return out


@pytest.mark.parametrize("M,N,K,dt,has_bias", _shapes())
def test_w8a8_linear_sweep_vs_oracle(backend, oracle, gpu, M, N, K, dt, has_bias):
    print(f"w8a8 linear sweep M={M} N={N} K={K} {dt} bias={has_bias}", flush=True)
    i8 = importlib.import_module(backend.__name__ + ".int8_eager")
    G = backend.pick_groupsize(K)
    # f32 activations hold bf16-grid values: every fp64 group sum is exact
    x = outlier_activations(M, K, seed=3 * M + K, dtype=torch.bfloat16)
    w = normal_weight(N, K, seed=N + 2 * K)
    b = normal_bias(N, seed=N + 1) if has_bias else None

    qw, ws = i8.quantize_convrot_w8a8_weight(w.cuda(), convrot_groupsize=G)
    eqw, ews = oracle.quantize_weight8(w.view(torch.int16).numpy().view(np.uint16), oracle.F16, G)
    assert np.array_equal(qw.cpu().numpy(), eqw)
    assert np.array_equal(ws.cpu().numpy().view(np.uint32), ews.view(np.uint32))

    xin = x if dt == "bf16" else x.float()
    y = backend.convrot_w8a8_linear(xin.cuda(), qw, ws, bias=None if b is None else b.cuda(), convrot_groupsize=G)
    assert y.shape == (M, N) and y.dtype == xin.dtype

    bias32 = None if b is None else b.float().numpy()
    if dt == "bf16":
        want = oracle.linear_w8a8(bf16_bits(x), oracle.BF16, eqw, ews, bias32, G, out_bf16=True)
        assert np.array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16), want)
    else:
        want = oracle.linear_w8a8(x.float().numpy(), oracle.F32, eqw, ews, bias32, G, out_bf16=False)
        assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))


W8A8_TYPED = [(300, 700, 3072, torch.float32, True), (2049, 1000, 12288, torch.float16, False),
              (513, 257, 4096, torch.float32, False), (1025, 640, 1040, torch.float16, True),
              (33, 100, 9216, torch.float32, True), (4099, 384, 3072, torch.float16, True)]


@pytest.mark.parametrize("M,N,K,dt,has_bias", W8A8_TYPED)
def test_w8a8_linear_f32_f16_long_rows(backend, oracle, gpu, M, N, K, dt, has_bias):
    """Genuine f32 activations (24-bit significands, not bf16-grid values) and
    f16 activations, rows of up to 12288: sampled output rows equal the oracle's
    int8 quantizer, exact int32 GEMM and f32 epilogue applied to the kernel's
    fp64 rotation restated on the CPU (f16 output: that epilogue cast to f16)."""
    from fp64_rotation import rotate_fp64_kernel_order
    print(f"w8a8 linear {dt} M={M} N={N} K={K} bias={has_bias}", flush=True)
    i8 = importlib.import_module(backend.__name__ + ".int8_eager")
    G = backend.pick_groupsize(K)
    code = oracle.F32 if dt == torch.float32 else oracle.F16
    x = outlier_activations(M, K, seed=M + 2 * K, dtype=dt)
    w = normal_weight(N, K, seed=N + 3 * K)
    b = normal_bias(N, seed=N + 2) if has_bias else None
    qw, ws = i8.quantize_convrot_w8a8_weight(w.cuda(), convrot_groupsize=G)
    eqw, ews = oracle.quantize_weight8(w.view(torch.int16).numpy().view(np.uint16), oracle.F16, G)
    assert np.array_equal(qw.cpu().numpy(), eqw)
    y = backend.convrot_w8a8_linear(x.cuda(), qw, ws, bias=None if b is None else b.cuda(), convrot_groupsize=G)
    assert y.shape == (M, N) and y.dtype == dt
    rows = np.unique(np.concatenate([np.random.RandomState(K).choice(M, min(M, 12), replace=False), [0, M - 1]]))
    xs_host = x[torch.from_numpy(rows)].contiguous()
    xb = xs_host.numpy() if dt == torch.float32 else xs_host.view(torch.int16).numpy().view(np.uint16)
    q8, sx = oracle.quant_rows8(rotate_fp64_kernel_order(xb, G, code), code)
    acc = oracle.int8_gemm(q8, eqw)
    want = oracle.epilogue_f32(acc, sx, ews, None if b is None else b.float().numpy(), out_bf16=False)
    got = y.cpu()[torch.from_numpy(rows)].numpy()
    if dt == torch.float32:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    else:
        assert np.array_equal(got.view(np.uint16), want.astype(np.float16).view(np.uint16))
