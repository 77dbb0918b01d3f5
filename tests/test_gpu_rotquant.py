"""GPU parity of the fused rotate+quantize kernel against the oracle and the
reference goldens: packed codes and scales bit-exact."""
import numpy as np
import pytest
import torch

from inputs import (WIDE_SPAN_CASES, bf16_bits, config1_x, edge_cases, outlier_activations, stochastic_weight_case,
                    wide_span_rows, wide_span_rows_typed)

pytestmark = pytest.mark.gpu

DT = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def host_bits(t):
    t = t.detach().cpu().contiguous()
    return t.numpy() if t.dtype == torch.float32 else t.view(torch.int16).numpy().view(np.uint16)


def gpu_quant(native, x, G):
    q, s = native.convrot_quant_int4(x.cuda(), G)
    torch.cuda.synchronize()
    return q.cpu().numpy(), s.cpu().numpy()


def assert_same(oracle, x, G, q, s):
    eq, es, _ = oracle.rotquant(host_bits(x), DT[x.dtype], G)
    bad_rows = np.nonzero((q != eq).any(axis=1) | (s != es))[0]
    assert len(bad_rows) == 0, f"{len(bad_rows)} rows differ, first {bad_rows[:5]}"


def test_config1_matches_goldens(native, oracle, goldens, gpu):
    x = config1_x()
    q, s = gpu_quant(native, x, 256)
    assert np.array_equal(q, goldens["c1_qact"])
    assert np.array_equal(s, goldens["c1_xscale"])


SHAPES = [
    (1, 3072, 256), (3, 256, 256), (257, 3072, 256), (64, 12288, 256), (33, 3840, 256),
    (16, 192, 64), (5, 64, 64), (16, 80, 16), (8, 16, 16), (9, 4096, 16), (11, 4096, 64),
    (7, 5120, 256), (12, 768, 256), (40, 32768, 256), (2, 32768, 64),
]


@pytest.mark.parametrize("M,K,G", SHAPES)
def test_shapes_bf16(native, oracle, gpu, M, K, G):
    x = outlier_activations(M, K, seed=M * 31 + K + G)
    q, s = gpu_quant(native, x, G)
    assert_same(oracle, x, G, q, s)


@pytest.mark.parametrize("M,K,G", [(19, 3072, 256), (8, 192, 64), (6, 80, 16), (130, 12288, 256), (300, 9216, 256)])
def test_shapes_f16(native, oracle, gpu, M, K, G):
    x = outlier_activations(M, K, seed=K + G, dtype=torch.float16, scale=8.0)
    q, s = gpu_quant(native, x, G)
    assert_same(oracle, x, G, q, s)


@pytest.mark.parametrize("M,K,G", [(19, 3072, 256), (8, 192, 64), (6, 80, 16), (40, 12288, 256), (600, 9216, 64)])
def test_shapes_f32(native, oracle, gpu, M, K, G):
    # f32 values on a bf16 grid: every group sum is exact in fp64, so the
    # correctly rounded rotation is what both sides compute
    x = outlier_activations(M, K, seed=K, dtype=torch.bfloat16).float()
    q, s = gpu_quant(native, x, G)
    assert_same(oracle, x, G, q, s)


@pytest.mark.parametrize("name", list(edge_cases().keys()))
def test_edge_cases_match_goldens(native, oracle, goldens, gpu, name):
    x, G = edge_cases()[name]
    q, s = gpu_quant(native, x, G)
    assert np.array_equal(q, goldens[f"edge_{name}_q"])
    if x.dtype != torch.float32:
        assert np.array_equal(s, goldens[f"edge_{name}_s"])
    assert_same(oracle, x, G, q, s)


def test_stochastic_weight_rounding(native, oracle, goldens, gpu):
    w = stochastic_weight_case()
    gen = torch.Generator(device="cpu")
    gen.manual_seed(1234)
    noise = torch.rand(w.shape, dtype=torch.float16, generator=gen)
    q, s = native.convrot_quant_int4_stochastic(w.cuda(), 256, noise.cuda())
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), goldens["stoch_q"])
    assert np.array_equal(s.cpu().numpy(), goldens["stoch_s"])


@pytest.mark.parametrize("K", [3072, 12288])
def test_full_size_sampled_rows(native, oracle, gpu, K):
    """The rotate+quant configuration at full size, 16384 x {3072, 12288}
    heavy-tailed (Student-t outlier channel) activations: every row is
    independent, so a sample of rows checked against the oracle pins the
    full-size launch.  The B6T output the linear uses decodes to the packed
    codes on every row, and its scales are the same."""
    M = 16384
    print(f"rotquant full size {M}x{K} Student-t", flush=True)
    x = outlier_activations(M, K, seed=123 + K, student_t=True)
    xg = x.cuda()
    q, s = native.convrot_quant_int4(xg, 256)
    q2, s2 = native.convrot_quant_int4(xg, 256)
    torch.cuda.synchronize()
    assert torch.equal(q, q2) and torch.equal(s, s2)          # deterministic
    rows = np.random.RandomState(0).choice(M, 48, replace=False)
    rows = np.concatenate([rows, [0, M - 1]])
    xs = x[rows]
    eq, es, _ = oracle.rotquant(host_bits(xs), 1, 256)
    assert np.array_equal(q.cpu().numpy()[rows], eq)
    assert np.array_equal(s.cpu().numpy()[rows], es)
    # properties over all rows: codes in [-7, 7], the absmax code is +-7
    codes = torch.stack([(q.to(torch.int32) << 28) >> 28, (q.to(torch.int32) << 24) >> 28], -1)
    assert int(codes.abs().max()) == 7
    assert bool((codes.abs().amax(dim=(1, 2)) == 7).all())
    a6, s6 = native.convrot_quant_bf6(xg, 256)
    assert torch.equal(s6, s)
    assert torch.equal(native.bf6_to_int4(a6, M, K), q)


@pytest.mark.parametrize("M,K", [(20000, 3072), (9000, 5120), (16500, 256)])
def test_persistent_rows_sampled(native, oracle, gpu, M, K):
    """More rows than resident waves: every wave walks several rows."""
    x = outlier_activations(M, K, seed=M + K)
    q, s = native.convrot_quant_int4(x.cuda(), 256)
    torch.cuda.synchronize()
    rows = np.concatenate([np.random.RandomState(2).choice(M, 40, replace=False), [0, 1, M - 2, M - 1]])
    eq, es, _ = oracle.rotquant(host_bits(x[rows]), 1, 256)
    assert np.array_equal(q.cpu().numpy()[rows], eq)
    assert np.array_equal(s.cpu().numpy()[rows], es)


# Every launch shape of the row-split kernel: W waves per row x P passes per
# wave (K = 1024 .. 11264 gives 1x1, 2x1, 4x1, 3x2, 2x3, 4x2, 3x3, 4x3), rows
# whose last wave or last pass starts past the row end (5120, 7168, 10240,
# 11264), lanes past the row end (640, 1152, 2176), and workgroups walking
# several rows (M above the resident grid).
ROW_SPLIT_SHAPES = [(300, 1024, 256), (1500, 2048, 256), (700, 4096, 256), (3000, 5120, 256),
                    (90, 6144, 256), (1300, 7168, 256), (64, 8192, 256), (2100, 9216, 256),
                    (33, 10240, 256), (1700, 11264, 256), (500, 640, 64), (2600, 1152, 64), (77, 2176, 64)]


@pytest.mark.parametrize("M,K,G", ROW_SPLIT_SHAPES)
def test_row_split_launch_shapes(native, oracle, gpu, M, K, G):
    """Packed int4 and int8 codes against the oracle (sampled rows); the B6T and
    I8T layouts against those codes (all rows)."""
    print(f"row-split M={M} K={K} G={G}", flush=True)
    from bf6_format import decode_b6t, i8t_np, unpack_int4
    x = outlier_activations(M, K, seed=M + 7 * K)
    xg = x.cuda()
    q, s = native.convrot_quant_int4(xg, G)
    a6, s6 = native.convrot_quant_bf6(xg, G)
    q8, s8 = native.convrot_quant_int8(xg, G)
    q8t, s8t = native.convrot_quant_int8_i8t(xg, G)
    torch.cuda.synchronize()
    rows = np.arange(M) if M <= 128 else np.concatenate(
        [np.random.RandomState(K).choice(M, 48, replace=False), [0, 1, M - 2, M - 1]])
    eq, es, _ = oracle.rotquant(host_bits(x[rows]), 1, G)
    assert np.array_equal(q.cpu().numpy()[rows], eq)
    assert np.array_equal(s.cpu().numpy()[rows], es)
    eq8, es8, _ = oracle.rotquant8(host_bits(x[rows]), 1, G)
    assert np.array_equal(q8.cpu().numpy()[rows], eq8)
    assert np.array_equal(s8.cpu().numpy()[rows], es8)
    assert torch.equal(s6.view(torch.int32), s.view(torch.int32))
    assert torch.equal(s8t.view(torch.int32), s8.view(torch.int32))
    assert np.array_equal(decode_b6t(a6.cpu().numpy(), M), unpack_int4(q.cpu().numpy()))
    assert np.array_equal(q8t.cpu().numpy(), i8t_np(q8.cpu().numpy()))


WIDE_SPAN_GPU = [(k, M, K, G) for k in ("mixed", "pairs", "ties")
                 for M, K, G in [(64, 256, 256), (96, 3072, 256), (40, 12288, 256), (64, 3072, 64), (32, 1024, 16)]]


@pytest.mark.parametrize("kind,M,K,G", WIDE_SPAN_GPU + list(WIDE_SPAN_CASES))
def test_wide_span_groups_vs_fp64_restatement(native, oracle, gpu, kind, M, K, G):
    """Groups spanning far more than the 36 binades of exact fp64 partial sums,
    where the kernel's rotation rounds: its int4 codes (packed and B6T), int8
    codes and row scales equal the eager quantizers applied to the fp64
    rotation restated operation for operation (tests/fp64_rotation.py), bit for
    bit.  On the "ties" rows that rotation differs from the exact one on about
    5% of the rotated values, so the int8 codes pin the kernel's summation order."""
    from bf6_format import decode_b6t, unpack_int4
    from fp64_rotation import rotate_fp64_kernel_order
    print(f"wide span {kind} M={M} K={K} G={G}", flush=True)
    x = wide_span_rows(M, K, G, M + K + G, kind)
    xr = rotate_fp64_kernel_order(host_bits(x), G)
    eq, es, _ = oracle.quant_rows(xr, DT[torch.bfloat16])
    eq8, es8 = oracle.quant_rows8(xr, DT[torch.bfloat16])
    q, s = gpu_quant(native, x, G)
    assert np.array_equal(q, eq) and np.array_equal(s.view(np.uint32), es.view(np.uint32))
    q8, s8 = native.convrot_quant_int8(x.cuda(), G)
    assert np.array_equal(q8.cpu().numpy(), eq8) and np.array_equal(s8.cpu().numpy().view(np.uint32), es8.view(np.uint32))
    if K % 128 == 0:
        a6, s6 = native.convrot_quant_bf6(x.cuda(), G)
        assert np.array_equal(s6.cpu().numpy().view(np.uint32), s.view(np.uint32))
        assert np.array_equal(decode_b6t(a6.cpu().numpy(), M), unpack_int4(q))


@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
@pytest.mark.parametrize("kind,M,K,G", [(k, M, K, G) for k in ("mixed", "pairs", "ties")
                                        for M, K, G in [(64, 3072, 256), (40, 12288, 256), (32, 1024, 16), (48, 3072, 64)]])
def test_wide_span_f32_f16_vs_fp64_restatement(native, oracle, gpu, dt, kind, M, K, G):
    """Genuine f32 inputs (24-bit significands; fp64 partial sums round beyond a
    20-binade span) and f16 inputs over the whole f16 range (always exact in
    fp64): int4 codes (packed and B6T), int8 codes and row scales equal the eager
    quantizers applied to the restated fp64 rotation, bit for bit."""
    from bf6_format import decode_b6t, unpack_int4
    from fp64_rotation import rotate_fp64_kernel_order
    print(f"wide span {dt} {kind} M={M} K={K} G={G}", flush=True)
    x = wide_span_rows_typed(M, K, G, M + K + G, kind, dt)
    xr = rotate_fp64_kernel_order(host_bits(x), G, DT[dt])
    eq, es, _ = oracle.quant_rows(xr, DT[dt])
    eq8, es8 = oracle.quant_rows8(xr, DT[dt])
    q, s = gpu_quant(native, x, G)
    assert np.array_equal(q, eq) and np.array_equal(s.view(np.uint32), es.view(np.uint32))
    q8, s8 = native.convrot_quant_int8(x.cuda(), G)
    assert np.array_equal(q8.cpu().numpy(), eq8) and np.array_equal(s8.cpu().numpy().view(np.uint32), es8.view(np.uint32))
    if K % 128 == 0:
        a6, s6 = native.convrot_quant_bf6(x.cuda(), G)
        assert np.array_equal(s6.cpu().numpy().view(np.uint32), s.view(np.uint32))
        assert np.array_equal(decode_b6t(a6.cpu().numpy(), M), unpack_int4(q))
