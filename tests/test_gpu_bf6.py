"""GPU parity of the bf6 GEMM path: the int4 -> B6 operand conversion, the
exact int32 accumulators on the bf6 matrix cores, every epilogue bit-exact
against the oracle and against the int8-MFMA kernels, the fused LoRA term."""
import numpy as np
import pytest
import torch

from bf6_format import decode_b6t, unpack_int4

pytestmark = pytest.mark.gpu


def rand_case(M, N, K, seed):
    rs = np.random.RandomState(seed)
    xp = rs.randint(-128, 128, size=(M, K // 2)).astype(np.int8)    # every nibble, -8 included
    wp = rs.randint(-128, 128, size=(N, K // 2)).astype(np.int8)
    xs = rs.uniform(0.005, 0.05, size=M).astype(np.float32)
    ws = rs.uniform(0.005, 0.05, size=N).astype(np.float32)
    b = (rs.standard_normal(N) * 0.01).astype(np.float32)
    return xp, wp, xs, ws, b


def cu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("rows,K", [(1, 128), (37, 256), (300, 3072), (64, 12288)])
def test_int4_to_bf6_roundtrip(native, gpu, rows, K):
    print(f"int4_to_bf6 rows={rows} K={K}", flush=True)
    p = np.random.RandomState(rows + K).randint(-128, 128, size=(rows, K // 2)).astype(np.int8)
    b6 = native.int4_to_bf6(cu(p)).cpu().numpy()
    assert b6.shape == ((rows + 255) // 256 * 256, K * 3 // 4)
    assert np.array_equal(decode_b6t(b6, rows), unpack_int4(p))


def test_bf6_codes_of_every_nibble(native, gpu):
    """Each int4 value -8..7 at each position of a group maps to its value."""
    K = 128
    rows = 16
    codes = (np.arange(rows * K) % 16 - 8).reshape(rows, K)
    lo = codes[:, 0::2] & 15
    hi = codes[:, 1::2] & 15
    p = (lo | (hi << 4)).astype(np.uint8).view(np.int8)
    b6 = native.int4_to_bf6(cu(p)).cpu().numpy()
    assert np.array_equal(decode_b6t(b6, rows), codes)


ACC_SHAPES = [(1, 1, 128), (3, 5, 256), (64, 48, 256), (256, 256, 3072), (300, 200, 1024),
              (257, 513, 1024), (512, 256, 12288), (100, 300, 3840), (16, 700, 128), (33, 1000, 2048)]


@pytest.mark.parametrize("M,N,K", ACC_SHAPES)
def test_bf6_acc_bitexact(native, oracle, gpu, M, N, K):
    print(f"bf6 acc M={M} N={N} K={K}", flush=True)
    xp, wp, *_ = rand_case(M, N, K, M + N + K)
    a6, w6 = native.int4_to_bf6(cu(xp)), native.int4_to_bf6(cu(wp))
    acc = native.int4_gemm_acc_bf6(a6, w6, M, N).cpu().numpy()
    assert np.array_equal(acc, oracle.int_gemm(xp, wp))


def test_bf6_acc_extremes(native, oracle, gpu):
    """All codes -8 (products 64) at K = 12288: |acc| = 786432, the largest
    partial sums the format allows at this K, still exact in fp32."""
    M, N, K = 64, 64, 12288
    xp = np.full((M, K // 2), -120, dtype=np.int8)           # 0x88: both nibbles -8
    wp = np.full((N, K // 2), -120, dtype=np.int8)
    wp[1::2] = 0x77                                          # alternate rows: both nibbles +7
    a6, w6 = native.int4_to_bf6(cu(xp)), native.int4_to_bf6(cu(wp))
    acc = native.int4_gemm_acc_bf6(a6, w6, M, N).cpu().numpy()
    assert np.array_equal(acc, oracle.int_gemm(xp, wp))
    assert acc[0, 0] == 64 * K and acc[0, 1] == -56 * K


@pytest.mark.parametrize("M,N,K", [(2048, 4096, 256), (2049, 4096, 256), (2048, 4097, 384), (512, 640, 4096),
                                   (512, 640, 4224), (1025, 4000, 128)])
def test_bf6_tile_choice_boundaries(native, oracle, gpu, M, N, K):
    """Shapes on either side of the 128 x 128 / 256 x 256 kernel choice (512
    quarter tiles; K 4096 / 4224) and of its split choice: the accumulators
    equal the int8-MFMA kernel's everywhere and the oracle's on sampled rows."""
    print(f"bf6 boundary M={M} N={N} K={K} nsplit={native.choose_nsplit_bf6(M, N, K)}", flush=True)
    xp, wp, *_ = rand_case(M, N, K, M + N + K)
    xg, wg = cu(xp), cu(wp)
    acc6 = native.int4_gemm_acc_bf6(native.int4_to_bf6(xg), native.int4_to_bf6(wg), M, N)
    acc8 = native.int4_gemm_acc(xg, wg)
    assert torch.equal(acc6, acc8)
    rows = np.concatenate([np.random.RandomState(K).choice(M, 6, replace=False), [0, M - 1]])
    assert np.array_equal(acc6.cpu().numpy()[rows], oracle.int_gemm(xp[rows], wp))


@pytest.mark.parametrize("M,N,K", [(4608, 3072, 3072), (1024, 3072, 12288)])
def test_bf6_acc_bitexact_large(native, oracle, gpu, M, N, K):
    print(f"bf6 acc large M={M} N={N} K={K}", flush=True)
    xp, wp, *_ = rand_case(M, N, K, 7)
    xg, wg = cu(xp), cu(wp)
    acc6 = native.int4_gemm_acc_bf6(native.int4_to_bf6(xg), native.int4_to_bf6(wg), M, N)
    acc8 = native.int4_gemm_acc(xg, wg)
    assert torch.equal(acc6, acc8)
    rows = np.random.RandomState(1).choice(M, 8, replace=False)
    assert np.array_equal(acc6.cpu().numpy()[rows], oracle.int_gemm(xp[rows], wp))


@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("M,N,K", [(64, 48, 256), (257, 300, 3072), (33, 513, 1024)])
def test_bf6_epilogues_bitexact(native, oracle, gpu, M, N, K, bias):
    xp, wp, xs, ws, b = rand_case(M, N, K, 3 * M + N)
    b = b if bias else None
    acc = oracle.int_gemm(xp, wp)
    a6, w6 = native.int4_to_bf6(cu(xp)), native.int4_to_bf6(cu(wp))
    args = (a6, w6, cu(xs), cu(ws), cu(b) if bias else None)
    f32 = native.int4_convrot_gemm_bf6(*args, native.EPI_F32).cpu().numpy()
    assert np.array_equal(f32.view(np.uint32), oracle.epilogue_f32(acc, xs, ws, b).view(np.uint32))
    bf = native.int4_convrot_gemm_bf6(*args, native.EPI_BF16).cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bf, oracle.epilogue_f32(acc, xs, ws, b, out_bf16=True))
    eg = native.int4_convrot_gemm_bf6(*args, native.EPI_BF16_EAGER).cpu().view(torch.int16).numpy()
    assert np.array_equal(eg.view(np.uint16), oracle.epilogue_eager_bf16(acc, xs, ws, b))


@pytest.mark.parametrize("M,N,K,R", [(64, 48, 256, 32), (257, 300, 3072, 96), (4608, 3072, 3072, 128),
                                     (77, 301, 128, 32), (300, 77, 384, 32), (4097, 3000, 3072, 32),
                                     (513, 9216, 3072, 32), (100, 200, 256, 128), (2049, 4000, 128, 32),
                                     (2049, 4000, 256, 32), (2300, 3700, 384, 32), (2049, 4000, 384, 64)])
def test_bf6_lora_equals_int8_path(native, gpu, M, N, K, R):
    """Same accumulators, same epilogue, same LoRA MFMA: outputs identical to
    the int8-MFMA kernel's for every epilogue.  Grids of at most 512 128 x 128
    tiles with K <= 4096 run the quarter-tile kernel, the rest the 256 x 256
    one; there, rank 32 with a bf16 output stages t / U in LDS during the last
    blocks (one 128-k block, two, three; ragged M and N: the staged rows past
    M / N repeat the last one)."""
    print(f"bf6 lora M={M} N={N} K={K} R={R}", flush=True)
    xp, wp, xs, ws, b = rand_case(M, N, K, M + R)
    rs = np.random.RandomState(R)
    t = torch.from_numpy(rs.standard_normal((M, R)).astype(np.float32)).to(torch.bfloat16).cuda()
    U = torch.from_numpy((rs.standard_normal((N, R)) * 0.3).astype(np.float32)).to(torch.bfloat16).cuda()
    xg, wg = cu(xp), cu(wp)
    a6, w6 = native.int4_to_bf6(xg), native.int4_to_bf6(wg)
    for epi in (native.EPI_F32, native.EPI_BF16, native.EPI_BF16_EAGER):
        o8 = native.int4_convrot_gemm_lora(xg, wg, cu(xs), cu(ws), cu(b), t, U, 0.7, epi)
        o6 = native.int4_convrot_gemm_bf6_lora(a6, w6, cu(xs), cu(ws), cu(b), t, U, 0.7, epi)
        v = (lambda o: o.view(torch.int16) if o.dtype == torch.bfloat16 else o.view(torch.int32))
        assert torch.equal(v(o6), v(o8)), epi


QUANT_CASES = [(1, 128, 16, torch.bfloat16), (37, 256, 256, torch.bfloat16), (300, 3072, 256, torch.bfloat16),
               (4608, 3072, 256, torch.bfloat16), (257, 12288, 256, torch.bfloat16), (64, 1024, 64, torch.bfloat16),
               (19, 3072, 256, torch.float16), (33, 640, 64, torch.float32), (513, 5120, 256, torch.bfloat16)]


@pytest.mark.parametrize("M,K,G,dt", QUANT_CASES)
def test_quant_bf6_equals_int4_quantizer(native, gpu, M, K, G, dt):
    """The fused quantizer into B6T writes the same codes and scales as the
    packed-int4 quantizer (whose parity with the oracle is tested separately),
    and zero codes in the padding rows."""
    print(f"quant_bf6 M={M} K={K} G={G} {dt}", flush=True)
    from inputs import outlier_activations
    x = outlier_activations(M, K, seed=M + K + G, student_t=True, dtype=dt).cuda()
    a6, s6 = native.convrot_quant_bf6(x, G)
    q, s = native.convrot_quant_int4(x, G)
    assert torch.equal(s6.view(torch.int32), s.view(torch.int32))
    assert np.array_equal(decode_b6t(a6.cpu().numpy(), M), unpack_int4(q.cpu().numpy()))


def test_quant_bf6_zero_rows_and_repeat(native, gpu):
    """All-zero rows (clamped scale) and a second call on a recycled buffer."""
    x = torch.zeros(300, 256, dtype=torch.bfloat16, device="cuda")
    x[5] = 1.0
    a, s = native.convrot_quant_bf6(x, 256)
    q, s4 = native.convrot_quant_int4(x, 256)
    assert torch.equal(s, s4)
    assert np.array_equal(decode_b6t(a.cpu().numpy(), 300), unpack_int4(q.cpu().numpy()))


@pytest.mark.parametrize("M,N,K,G,lora", [(77, 256, 3072, 256, False), (4608, 3072, 3072, 256, False),
                                          (300, 520, 1024, 64, True), (64, 3072, 12288, 256, False),
                                          (129, 384, 3072, 256, True)])
def test_linear_bf6_bit_identical_to_int8_path(backend, native, gpu, M, N, K, G, lora):
    """convrot_w4a4_linear on the bf6 GEMM (prepared weight) returns exactly
    the int8-MFMA path's output, LoRA term included."""
    print(f"linear bf6 M={M} N={N} K={K} lora={lora}", flush=True)
    from inputs import normal_bias, normal_weight, outlier_activations
    x = outlier_activations(M, K, seed=M).cuda()
    qw, ws = backend.quantize_convrot_w4a4_weight(normal_weight(N, K, seed=N).cuda(), convrot_groupsize=G)
    bias = normal_bias(N, seed=5).cuda()
    w6 = backend.prepare_convrot_w4a4_weight_bf6(qw)
    assert w6 is not None and w6.shape == (native.bf6_rows(N), K * 3 // 4)
    fused = None
    if lora:
        rng = np.random.RandomState(K)
        d = torch.from_numpy((rng.standard_normal((32, K)) * 0.02).astype(np.float32)).cuda()
        u = torch.from_numpy((rng.standard_normal((N, 32)) * 0.1).astype(np.float32)).cuda()
        fused = backend.fuse_lora_pairs([(d, u, 0.5)])
    y6 = backend.convrot_w4a4_linear(x, qw, ws, bias=bias, convrot_groupsize=G, lora=fused, qweight_bf6=w6)
    y6b = backend.convrot_w4a4_linear(x, qw, ws, bias=bias, convrot_groupsize=G, lora=fused)   # on-the-fly weight
    qa, xs = native.convrot_quant_int4(x, G)
    if lora:
        t = native.lora_down(x, fused[0])
        y8 = native.int4_convrot_gemm_lora(qa, qw, xs, ws, bias, t, fused[1], 1.0, native.EPI_BF16)
    else:
        y8 = native.int4_convrot_gemm(qa, qw, xs, ws, bias, torch.bfloat16)
    assert torch.equal(y6.view(torch.int16), y8.view(torch.int16))
    assert torch.equal(y6b.view(torch.int16), y8.view(torch.int16))
