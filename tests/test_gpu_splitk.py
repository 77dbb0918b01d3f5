"""GPU parity of the split-K bf6 GEMM: for every split count the accumulators
equal the oracle's and every epilogue (with and without the LoRA term) is
bit-identical to the unsplit kernel's, on full and ragged tile grids."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def cu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def operands(native, M, N, K, seed):
    rs = np.random.RandomState(seed)
    xp = rs.randint(-128, 128, size=(M, K // 2)).astype(np.int8)
    wp = rs.randint(-128, 128, size=(N, K // 2)).astype(np.int8)
    xs = rs.uniform(0.005, 0.05, size=M).astype(np.float32)
    ws = rs.uniform(0.005, 0.05, size=N).astype(np.float32)
    b = (rs.standard_normal(N) * 0.01).astype(np.float32)
    return xp, wp, native.int4_to_bf6(cu(xp)), native.int4_to_bf6(cu(wp)), cu(xs), cu(ws), cu(b)


# Grids of at most 512 quarter tiles take the small-tile kernel (128 x 128, or
# 128 x 192 where the split quarter tiles would exceed the CUs: 1024 x 3072 in
# two), whose splits are reduced in the kernel by the last split of each tile;
# larger grids take the 256 x 256 partial kernel and the reduce kernel (the
# last case).
SPLIT_CASES = [(512, 3072, 12288, [2, 5, 6, 16, 96]), (300, 700, 1024, [2, 3, 8]), (1024, 3072, 3072, [2, 4, 24]),
               (64, 256, 256, [2]), (257, 513, 3840, [7, 30]), (640, 13312, 2048, [2, 4])]


@pytest.mark.parametrize("M,N,K,splits", SPLIT_CASES)
def test_splitk_acc_exact(native, oracle, gpu, M, N, K, splits):
    print(f"splitk acc M={M} N={N} K={K}", flush=True)
    xp, wp, a6, w6, *_ = operands(native, M, N, K, M + N + K)
    base = native.int4_gemm_acc_bf6(a6, w6, M, N, nsplit=1)
    rows = np.arange(M) if M <= 300 else np.random.RandomState(2).choice(M, 24, replace=False)
    assert np.array_equal(base.cpu().numpy()[rows], oracle.int_gemm(xp[rows], wp))
    for s in splits:
        acc = native.int4_gemm_acc_bf6(a6, w6, M, N, nsplit=s)
        assert torch.equal(acc, base), s


@pytest.mark.parametrize("M,N,K,splits", SPLIT_CASES[:3])
def test_splitk_epilogues_identical(native, gpu, M, N, K, splits):
    _, _, a6, w6, xs, ws, b = operands(native, M, N, K, 7 * M + K)
    for epi in (native.EPI_F32, native.EPI_BF16, native.EPI_BF16_EAGER):
        for bias in (b, None):
            base = native.int4_convrot_gemm_bf6(a6, w6, xs, ws, bias, epi, nsplit=1)
            for s in splits:
                out = native.int4_convrot_gemm_bf6(a6, w6, xs, ws, bias, epi, nsplit=s)
                assert torch.equal(out.view(torch.int16) if out.dtype == torch.bfloat16 else out.view(torch.int32),
                                   base.view(torch.int16) if base.dtype == torch.bfloat16 else base.view(torch.int32)), (epi, s)


@pytest.mark.parametrize("R", [32, 64, 128])
def test_splitk_lora_identical(native, gpu, R):
    M, N, K = 512, 3072, 12288
    _, _, a6, w6, xs, ws, b = operands(native, M, N, K, R)
    g = torch.Generator(device="cuda").manual_seed(R)
    t = torch.randn((M, R), generator=g, device="cuda").to(torch.bfloat16)
    U = (torch.randn((N, R), generator=g, device="cuda") * 0.1).to(torch.bfloat16)
    for epi in (native.EPI_F32, native.EPI_BF16):
        base = native.int4_convrot_gemm_bf6_lora(a6, w6, xs, ws, b, t, U, 0.75, epi, nsplit=1)
        for s in (3, 8):
            out = native.int4_convrot_gemm_bf6_lora(a6, w6, xs, ws, b, t, U, 0.75, epi, nsplit=s)
            assert torch.equal(out, base), (epi, s)


def test_auto_split_linear_matches_unsplit(backend, native, gpu):
    """convrot_w4a4_linear at a small-M shape (where the library splits) is
    bit-identical to the same product forced unsplit."""
    from inputs import normal_bias, normal_weight, outlier_activations
    M, N, K = 512, 3072, 12288
    assert native.choose_nsplit_bf6(M, N, K) > 1
    x = outlier_activations(M, K, seed=3).cuda()
    qw, ws = backend.quantize_convrot_w4a4_weight(normal_weight(N, K, seed=4).cuda())
    b = normal_bias(N, seed=5).cuda()
    y = backend.convrot_w4a4_linear(x, qw, ws, bias=b)
    a6, xs = native.convrot_quant_bf6(x, 256)
    y1 = native.int4_convrot_gemm_bf6(a6, backend.prepare_convrot_w4a4_weight_bf6(qw), xs, ws, b,
                                      native.EPI_BF16, nsplit=1)
    assert torch.equal(y, y1)


def test_split_counters_left_zero(native, gpu):
    """Every split call leaves the counter region of its workspace zero, also
    across shapes and split counts sharing the stream's workspace, and a
    second run of each split equals the first."""
    st = native._stream(torch.device("cuda"))
    first = {}
    for M, N, K, s in [(512, 3072, 12288, 6), (300, 700, 1024, 3), (512, 3072, 12288, 4), (1024, 3072, 3072, 2),
                       (300, 700, 1024, 3), (512, 3072, 12288, 6)]:
        _, _, a6, w6, xs, ws, b = operands(native, M, N, K, M + K)
        out = native.int4_convrot_gemm_bf6(a6, w6, xs, ws, b, native.EPI_F32, nsplit=s)
        key = (M, N, K, s)
        if key in first:
            assert torch.equal(out, first[key]), key
        first[key] = out
        wsb = native._workspaces[(torch.cuda.current_device(), st)]
        assert int(wsb[:native.SPLIT_COUNTER_BYTES].count_nonzero()) == 0, key


# Small grids whose 128 x 128 tiles exceed the CUs run 128 x 192 tiles (6 waves,
# 64-row operand units): full tiles, ragged M and N, and an edge tile whose last
# B unit lies past the padded rows (9000 x 449: units re-read the last one).
WIDE_CASES = [(512, 12288, 3072), (2048, 3072, 3072), (500, 9000, 1024), (9000, 449, 1024)]


@pytest.mark.parametrize("M,N,K", WIDE_CASES)
def test_wide_small_tile_acc_exact(native, oracle, gpu, M, N, K):
    print(f"128x192 acc M={M} N={N} K={K}", flush=True)
    assert native.gemm_tile_bf6(M, N, K) == (128, 192)
    xp, wp, a6, w6, *_ = operands(native, M, N, K, 3 * M + N)
    acc = native.int4_gemm_acc_bf6(a6, w6, M, N, nsplit=1)
    rs = np.random.RandomState(M + N)
    rows = np.unique(np.concatenate([rs.choice(M, 20, replace=False), [0, M - 1]]))
    cols = np.unique(np.concatenate([rs.choice(N, min(N, 400), replace=False), [0, N - 1]]))
    ref = oracle.int_gemm(xp[rows], wp[cols])
    assert np.array_equal(acc.cpu().numpy()[np.ix_(rows, cols)], ref)
    assert torch.equal(acc, native.int4_gemm_acc_bf6(a6, w6, M, N, nsplit=2))   # 128 x 128, split


@pytest.mark.parametrize("M,N,K", WIDE_CASES)
def test_wide_small_tile_epilogues_match_quarter_tiles(native, gpu, M, N, K):
    """Every epilogue, with and without bias, equals the 128 x 128 kernel's
    bits (its split form, which equals its unsplit form)."""
    print(f"128x192 epilogues M={M} N={N} K={K}", flush=True)
    _, _, a6, w6, xs, ws, b = operands(native, M, N, K, M + 5 * N)
    for epi in (native.EPI_F32, native.EPI_BF16, native.EPI_BF16_EAGER):
        for bias in (b, None):
            out = native.int4_convrot_gemm_bf6(a6, w6, xs, ws, bias, epi, nsplit=1)
            ref = native.int4_convrot_gemm_bf6(a6, w6, xs, ws, bias, epi, nsplit=2)
            assert torch.equal(out.view(torch.int16) if out.dtype == torch.bfloat16 else out.view(torch.int32),
                               ref.view(torch.int16) if ref.dtype == torch.bfloat16 else ref.view(torch.int32)), epi


@pytest.mark.parametrize("R", [32, 64, 128])
def test_wide_small_tile_lora_matches_quarter_tiles(native, gpu, R):
    M, N, K = 500, 9000, 1024
    assert native.gemm_tile_bf6(M, N, K) == (128, 192)
    _, _, a6, w6, xs, ws, b = operands(native, M, N, K, R + 1)
    g = torch.Generator(device="cuda").manual_seed(R)
    t = torch.randn((M, R), generator=g, device="cuda").to(torch.bfloat16)
    U = (torch.randn((N, R), generator=g, device="cuda") * 0.1).to(torch.bfloat16)
    for epi in (native.EPI_F32, native.EPI_BF16, native.EPI_BF16_EAGER):
        out = native.int4_convrot_gemm_bf6_lora(a6, w6, xs, ws, b, t, U, 0.75, epi, nsplit=1)
        ref = native.int4_convrot_gemm_bf6_lora(a6, w6, xs, ws, b, t, U, 0.75, epi, nsplit=2)
        assert torch.equal(out, ref), (epi, R)


# k-split on 128 x 192 tiles (grids whose split quarter tiles would exceed the
# CUs), full and ragged, one with the last B unit past the padded rows
WIDE_SPLIT_CASES = [(1024, 3072, 3072, 2), (1000, 3000, 8192, 2), (5000, 449, 2048, 2)]


@pytest.mark.parametrize("M,N,K,s", WIDE_SPLIT_CASES)
def test_wide_small_tile_split_exact(native, oracle, gpu, M, N, K, s):
    print(f"128x192 split {s} M={M} N={N} K={K}", flush=True)
    assert native.gemm_tile_bf6(M, N, K, s) == (128, 192)
    xp, wp, a6, w6, xs, ws, b = operands(native, M, N, K, M + N + s)
    acc = native.int4_gemm_acc_bf6(a6, w6, M, N, nsplit=s)
    rs = np.random.RandomState(K)
    rows = np.unique(np.concatenate([rs.choice(M, 16, replace=False), [0, M - 1]]))
    assert np.array_equal(acc.cpu().numpy()[rows], oracle.int_gemm(xp[rows], wp))
    assert torch.equal(acc, native.int4_gemm_acc_bf6(a6, w6, M, N, nsplit=1))
    for epi in (native.EPI_F32, native.EPI_BF16, native.EPI_BF16_EAGER):
        out = native.int4_convrot_gemm_bf6(a6, w6, xs, ws, b, epi, nsplit=s)
        ref = native.int4_convrot_gemm_bf6(a6, w6, xs, ws, b, epi, nsplit=1)
        assert torch.equal(out.view(torch.int16) if out.dtype == torch.bfloat16 else out.view(torch.int32),
                           ref.view(torch.int16) if ref.dtype == torch.bfloat16 else ref.view(torch.int32)), epi
    g = torch.Generator(device="cuda").manual_seed(s)
    t = torch.randn((M, 32), generator=g, device="cuda").to(torch.bfloat16)
    U = (torch.randn((N, 32), generator=g, device="cuda") * 0.1).to(torch.bfloat16)
    out = native.int4_convrot_gemm_bf6_lora(a6, w6, xs, ws, b, t, U, 0.5, native.EPI_BF16, nsplit=s)
    ref = native.int4_convrot_gemm_bf6_lora(a6, w6, xs, ws, b, t, U, 0.5, native.EPI_BF16, nsplit=1)
    assert torch.equal(out, ref)
