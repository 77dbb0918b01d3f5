"""GPU parity of the W4A4 GEMM: int32 accumulators bit-exact, every epilogue
bit-exact against the oracle, and against the reference int4_linear goldens."""
import numpy as np
import pytest
import torch

from inputs import small_linear_case

pytestmark = pytest.mark.gpu


def rand_case(M, N, K, seed):
    rs = np.random.RandomState(seed)
    xp = rs.randint(-128, 128, size=(M, K // 2)).astype(np.int8)    # all nibbles incl. -8
    wp = rs.randint(-128, 128, size=(N, K // 2)).astype(np.int8)
    xs = rs.uniform(0.005, 0.05, size=M).astype(np.float32)
    ws = rs.uniform(0.005, 0.05, size=N).astype(np.float32)
    b = (rs.standard_normal(N) * 0.01).astype(np.float32)
    return xp, wp, xs, ws, b


def cu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


# K = 128 / 384 run the pipelined kernel with one / three 128-k blocks (copies
# past the last block clamped), K % 128 != 0 the register-staged one
ACC_SHAPES = [(1, 1, 32), (3, 5, 64), (64, 48, 256), (256, 256, 3072), (300, 200, 160),
              (257, 513, 1024), (512, 256, 12288), (100, 300, 3840), (16, 700, 96), (9, 17, 128), (40, 260, 384)]


@pytest.mark.parametrize("M,N,K", ACC_SHAPES)
def test_acc_bitexact(native, oracle, gpu, M, N, K):
    xp, wp, *_ = rand_case(M, N, K, M + N + K)
    acc = native.int4_gemm_acc(cu(xp), cu(wp)).cpu().numpy()
    assert np.array_equal(acc, oracle.int_gemm(xp, wp))


@pytest.mark.parametrize("M,N,K", [(4608, 3072, 3072), (1024, 3072, 12288)])
def test_acc_bitexact_large(native, oracle, gpu, M, N, K):
    """Full Flux-sized shapes against an exact fp32 GEMM of the codes
    (|acc| <= 64 K < 2^24, so fp32 accumulation is exact in any order)."""
    xp, wp, *_ = rand_case(M, N, K, 7)
    xg, wg = cu(xp), cu(wp)
    acc = native.int4_gemm_acc(xg, wg)
    unpack = lambda p: torch.stack([(p.to(torch.int32) << 28) >> 28, (p.to(torch.int32) << 24) >> 28],
                                   -1).reshape(p.shape[0], -1).float()
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False     # restored below: later tests keep their setting
    try:
        ref = (unpack(xg) @ unpack(wg).T).to(torch.int32)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev
    assert torch.equal(acc, ref)
    rows = np.random.RandomState(1).choice(M, 8, replace=False)
    assert np.array_equal(acc.cpu().numpy()[rows], oracle.int_gemm(xp[rows], wp))


@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("M,N,K", [(64, 48, 256), (257, 300, 3072), (33, 513, 1024)])
def test_epilogues_bitexact(native, oracle, gpu, M, N, K, bias):
    xp, wp, xs, ws, b = rand_case(M, N, K, 3 * M + N)
    b = b if bias else None
    acc = oracle.int_gemm(xp, wp)
    args = (cu(xp), cu(wp), cu(xs), cu(ws), cu(b) if bias else None)
    f32 = native.int4_convrot_gemm(*args, torch.float32).cpu().numpy()
    assert np.array_equal(f32.view(np.uint32), oracle.epilogue_f32(acc, xs, ws, b).view(np.uint32))
    bf = native.int4_convrot_gemm(*args, torch.bfloat16).cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bf, oracle.epilogue_f32(acc, xs, ws, b, out_bf16=True))
    eg = native.int4_convrot_gemm_ex(*args, native.EPI_BF16_EAGER).cpu().view(torch.int16).numpy()
    assert np.array_equal(eg.view(np.uint16), oracle.epilogue_eager_bf16(acc, xs, ws, b))


def test_int4_linear_goldens(native, goldens, gpu):
    xp, wp, xs, ws, bias = small_linear_case()
    args = (xp.cuda(), wp.cuda(), xs.cuda(), ws.cuda())
    eg = native.int4_convrot_gemm_ex(*args, bias.float().cuda(), native.EPI_BF16_EAGER)
    assert np.array_equal(eg.cpu().view(torch.int16).numpy().view(np.uint16), goldens["lin_bf16"])
    eg = native.int4_convrot_gemm_ex(*args, None, native.EPI_BF16_EAGER)
    assert np.array_equal(eg.cpu().view(torch.int16).numpy().view(np.uint16), goldens["lin_bf16_nobias"])
    f32 = native.int4_convrot_gemm(*args, bias.float().cuda(), torch.float32)
    assert np.array_equal(f32.cpu().numpy(), goldens["lin_f32"])


def test_bf16_output_close_to_eager_chain(native, oracle, gpu):
    """The default bf16 epilogue (fp32 chain, one rounding) vs the eager bf16
    chain: within the 1e-2 relative Frobenius bound."""
    xp, wp, xs, ws, b = rand_case(512, 384, 3072, 99)
    acc = oracle.int_gemm(xp, wp)
    ref = oracle.bf16_to_f32(oracle.epilogue_eager_bf16(acc, xs, ws, b)).astype(np.float64)
    out = native.int4_convrot_gemm(cu(xp), cu(wp), cu(xs), cu(ws), cu(b), torch.bfloat16)
    got = out.float().cpu().numpy().astype(np.float64)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-2


# the reference's split-K export: pipelined kernel (K % 128 == 0) and the
# register-staged one (K % 128 != 0), nsplit below, at and above the k-block count
SPLITK_CASES = [(64, 256, 3072, [1, 2, 8, 24, 40]), (300, 200, 160, [1, 2, 3]), (257, 513, 12288, [3, 8, 96]),
                (8, 1000, 3840, [2, 7, 30]), (512, 3072, 12288, [8])]


@pytest.mark.parametrize("M,N,K,splits", SPLITK_CASES)
def test_reference_splitk_bitexact(native, oracle, gpu, M, N, K, splits):
    """ck_int4_convrot_gemm_splitk: the zeroed f32 accumulator ends up holding
    fl32(fl32(acc * xs) * ws) for every nsplit: against the oracle's epilogue
    (sampled rows) and bit-identical to the unsplit f32 epilogue without bias;
    bias + cast afterwards (as the reference's caller does) gives the unsplit
    bf16 output."""
    print(f"ck splitk M={M} N={N} K={K}", flush=True)
    xp, wp, xs, ws, b = rand_case(M, N, K, 11 * M + K)
    args = (cu(xp), cu(wp), cu(xs), cu(ws))
    base = native.int4_convrot_gemm(*args, None, torch.float32)
    rows = np.arange(M) if M <= 300 else np.random.RandomState(5).choice(M, 16, replace=False)
    ref = oracle.epilogue_f32(oracle.int_gemm(xp[rows], wp), xs[rows], ws, None)
    assert np.array_equal(base.cpu().numpy()[rows].view(np.uint32), ref.view(np.uint32))
    for s in splits:
        acc = native.int4_convrot_gemm_splitk(*args, s)
        assert torch.equal(acc.view(torch.int32), base.view(torch.int32)), s
    bf = (acc + cu(b)).to(torch.bfloat16)
    unsplit = native.int4_convrot_gemm(*args, cu(b), torch.bfloat16)
    assert torch.equal(bf.view(torch.int16), unsplit.view(torch.int16))
