"""Pins for the CPU oracle: golden vectors written by the reference eager path,
closed forms, brute force and the exact integer accumulator."""
import hashlib

import numpy as np
import pytest
import torch

from inputs import (bf16_bits, clamp_rows8, config1_bias, config1_weight, config1_x, edge_cases,
                    hadamard_np, small_linear_case, small_w8a8_case, stochastic_weight_case, tie_rows8)

DT_OF = {torch.bfloat16: 1, torch.float16: 2, torch.float32: 0}


def np_of(t):
    return t.numpy() if t.dtype == torch.float32 else t.contiguous().view(torch.int16).numpy().view(np.uint16)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# ----------------------------------------------------------------------------
# golden vectors (reference eager path)
# ----------------------------------------------------------------------------

def test_golden_config1_activation(oracle, goldens):
    x = bf16_bits(config1_x())
    packed, xs, xr = oracle.rotquant(x, oracle.BF16, 256)
    assert np.array_equal(packed, goldens["c1_qact"])
    assert np.array_equal(xs, goldens["c1_xscale"])
    # the rotation is correctly rounded; torch's CPU bf16 matmul agrees except
    # at rare near-ties decided by its fp32 accumulation order
    diff = np.nonzero(xr != goldens["c1_xr"])
    assert len(diff[0]) <= 4
    for m, k in zip(*diff):
        a = oracle.bf16_to_f32(np.array([xr[m, k]]))[0]
        b = oracle.bf16_to_f32(np.array([goldens["c1_xr"][m, k]]))[0]
        assert abs(int(xr[m, k]) - int(goldens["c1_xr"][m, k])) == 1, (m, k, a, b)


def test_golden_config1_weight(oracle, goldens):
    w = np_of(config1_weight())
    qw, ws = oracle.quantize_weight(w, oracle.F16, 256)
    assert np.array_equal(qw[:256], goldens["c1_qw_rows256"])
    assert sha(qw) == str(goldens["c1_qw_sha"])
    assert np.array_equal(ws, goldens["c1_wscale"])


def test_golden_config1_linear(oracle, goldens):
    x = bf16_bits(config1_x())
    qw, ws = oracle.quantize_weight(np_of(config1_weight()), oracle.F16, 256)
    y = oracle.linear_eager(x, oracle.BF16, qw, ws, config1_bias().float().numpy(), 256)
    assert np.array_equal(y[:32], goldens["c1_y_rows32"])
    assert sha(y) == str(goldens["c1_y_sha"])


@pytest.mark.parametrize("name", list(edge_cases().keys()))
def test_golden_edge_cases(oracle, goldens, name):
    xe, G = edge_cases()[name]
    dt = DT_OF[xe.dtype]
    packed, s, xr = oracle.rotquant(np_of(xe), dt, G)
    assert np.array_equal(packed, goldens[f"edge_{name}_q"])
    if dt == oracle.F32:
        # torch's fp32 accumulation is not correctly rounded: xr (and the absmax
        # element) may differ in the last bits; the oracle is the exact value
        gxr = goldens[f"edge_{name}_xr"]
        # fp32 accumulation error of a 256-term sum, relative to the row magnitude
        err = np.abs(xr.astype(np.float64) - gxr) / np.abs(xr).max(axis=1, keepdims=True)
        assert err.max() <= 256 * 2.0 ** -24
        sd = np.abs(s.view(np.int32).astype(np.int64) - goldens[f"edge_{name}_s"].view(np.int32))
        assert sd.max() <= 16
    else:
        assert np.array_equal(xr, goldens[f"edge_{name}_xr"])
        assert np.array_equal(s, goldens[f"edge_{name}_s"])


def test_golden_stochastic_weight(oracle, goldens):
    w = np_of(stochastic_weight_case())
    gen = torch.Generator(device="cpu")
    gen.manual_seed(1234)
    noise = np_of(torch.rand(w.shape, dtype=torch.float16, generator=gen))
    q, s = oracle.quantize_weight(w, oracle.F16, 256, noise)
    assert np.array_equal(q, goldens["stoch_q"])
    assert np.array_equal(s, goldens["stoch_s"])


def test_golden_weight_g64_and_dequant(oracle, goldens):
    w = np_of(stochastic_weight_case())
    q, s = oracle.quantize_weight(w, oracle.F16, 64)
    assert np.array_equal(q, goldens["w64_q"]) and np.array_equal(s, goldens["w64_s"])
    deq = oracle.dequantize_weight(q, s, 64)
    np.testing.assert_allclose(deq, goldens["w64_deq"], rtol=0, atol=1e-6)


def test_golden_int4_linear(oracle, goldens):
    xp, wp, xs, ws, bias = small_linear_case()
    acc = oracle.int_gemm(xp.numpy(), wp.numpy())
    b = bias.float().numpy()
    assert np.array_equal(oracle.epilogue_eager_bf16(acc, xs.numpy(), ws.numpy(), b), goldens["lin_bf16"])
    assert np.array_equal(oracle.epilogue_eager_bf16(acc, xs.numpy(), ws.numpy(), None),
                          goldens["lin_bf16_nobias"])
    assert np.array_equal(oracle.epilogue_f32(acc, xs.numpy(), ws.numpy(), b), goldens["lin_f32"])


def test_golden_codec(oracle, goldens):
    allb = np.arange(-128, 128).astype(np.int8).reshape(1, 256)
    assert np.array_equal(oracle.unpack(allb), goldens["codec_unpack_all"])
    assert np.array_equal(oracle.pack(np.array([[1, -1, -8, 7, 0, -7, 3, 5]])), goldens["codec_pack_pairs"])


# ----------------------------------------------------------------------------
# closed forms and brute force
# ----------------------------------------------------------------------------

@pytest.mark.parametrize("G", [4, 16, 64, 256])
def test_hadamard_identities(oracle, G):
    H = oracle.hadamard(G).astype(np.float64)
    assert np.array_equal(H, H.T)                                  # symmetric
    np.testing.assert_array_equal(H @ H, np.eye(G))                # involution (exact in fp64)
    assert np.all(np.abs(np.abs(H) - 1 / np.sqrt(G)) == 0)
    np.testing.assert_array_equal(H, hadamard_np(G))               # kron construction
    # H4 v = (sum v) 1 - 2 reverse(v)
    v = np.arange(1.0, 5.0)
    np.testing.assert_array_equal(oracle.hadamard(4).astype(np.float64) * 2 @ v, v.sum() - 2 * v[::-1])


def test_hadamard_rejects_bad_sizes(oracle):
    for g in (2, 8, 32, 48):
        with pytest.raises(ValueError):
            oracle.hadamard(g)


def test_codec_known_answers_and_roundtrip(oracle):
    assert oracle.pack(np.array([[1, -1]])).view(np.uint8)[0, 0] == 0xF1
    assert oracle.pack(np.array([[-8, 7]])).view(np.uint8)[0, 0] == 0x78
    allb = np.arange(256).astype(np.uint8).view(np.int8).reshape(1, 256)
    assert np.array_equal(oracle.pack(oracle.unpack(allb)), allb)


@pytest.mark.parametrize("dt,G", [(1, 256), (1, 64), (1, 16), (2, 256), (0, 64)])
def test_rotation_fp64_path_equals_exact_accumulator(oracle, dt, G):
    rs = np.random.RandomState(dt * 100 + G)
    f = (rs.standard_normal((3, 2 * G)) * np.exp(rs.uniform(-4, 4, (3, 2 * G)))).astype(np.float32)
    x = f if dt == 0 else (oracle.f32_to_bf16(f) if dt == 1 else f.astype(np.float16).view(np.uint16))
    xr = oracle.rotate(x, dt, G)
    xrf = oracle.to_f32(xr, dt)
    for m in range(3):
        for col in rs.choice(2 * G, 12, replace=False):
            assert oracle.rotate_one_exact(x, dt, G, m, col) == xrf[m, col]


def test_rotation_matches_fraction_arithmetic(oracle):
    from fractions import Fraction
    rs = np.random.RandomState(3)
    G = 16
    f = (rs.standard_normal((2, G)) * np.exp(rs.uniform(-30, 30, (2, G)))).astype(np.float32)
    x = oracle.f32_to_bf16(f)
    xf = oracle.bf16_to_f32(x).astype(np.float64)
    H = hadamard_np(G) * 4  # +-1 entries
    xr = oracle.bf16_to_f32(oracle.rotate(x, oracle.BF16, G))
    for m in range(2):
        for j in range(G):
            exact = sum(Fraction(float(xf[m, i])) * int(H[i, j]) for i in range(G)) / 4
            # correctly rounded bf16 of `exact`: compare with neighbours
            got = Fraction(float(xr[m, j]))
            bits = int(oracle.f32_to_bf16(np.array([xr[m, j]], dtype=np.float32))[0])
            up = Fraction(float(oracle.bf16_to_f32(np.array([bits + 1], dtype=np.uint16))[0]))
            dn = Fraction(float(oracle.bf16_to_f32(np.array([bits - 1], dtype=np.uint16))[0]))
            if got > 0:
                assert abs(exact - got) <= abs(exact - up) and abs(exact - got) <= abs(exact - dn)
            elif got < 0:
                assert abs(exact - got) <= abs(exact - up) and abs(exact - got) <= abs(exact - dn)


def _bf16(v):
    return float(torch.tensor(v, dtype=torch.float32).to(torch.bfloat16).float())


def test_quantizer_brute_force_small(oracle):
    """Each code from the eager formula evaluated by hand in exact rationals +
    explicit bf16 roundings (no shared code with the oracle)."""
    rs = np.random.RandomState(11)
    for trial in range(20):
        row = oracle.f32_to_bf16((rs.standard_normal(16) * (0.1 + trial)).astype(np.float32))
        _, s, codes = oracle.quant_rows(row.reshape(1, 16), oracle.BF16)
        vals = oracle.bf16_to_f32(row).astype(np.float64)
        a = max(np.abs(vals).max(), _bf16(1e-10))
        sc = _bf16(np.float32(a) / np.float32(7.0))
        assert s[0] == sc
        for k in range(16):
            t = _bf16(np.float32(vals[k]) / np.float32(sc))
            q = int(np.clip(np.round(t), -7, 7))          # numpy rounds half to even
            assert codes[0, k] == q


def test_quantizer_ties_round_half_even(oracle):
    # row with absmax 7 -> s = 1: x/s lands exactly on half-integers
    vals = np.array([7.0, 0.5, 1.5, 2.5, 3.5, 4.5, 5.5, 6.5, -0.5, -1.5, -2.5, -3.5, -4.5, -5.5, -6.5, 0.0],
                    dtype=np.float32)
    _, s, codes = oracle.quant_rows(oracle.f32_to_bf16(vals).reshape(1, 16), oracle.BF16)
    assert s[0] == 1.0
    assert codes[0].tolist() == [7, 0, 2, 2, 4, 4, 6, 6, 0, -2, -2, -4, -4, -6, -6, 0]


def test_bf16_quotient_never_a_rounding_midpoint():
    """For bf16 xr and s (8-bit significands mx, ms) the quotient mx/ms * 2^d
    is never an odd 9-bit dyadic (a bf16 rounding midpoint), and its distance
    to one is at least 2^-17 relative.  This is what lets the kernel replace
    the IEEE division by a multiply with fl32(1/s).  Exhaustive over all
    significand pairs."""
    from fractions import Fraction
    mids = [Fraction(p, 256) for p in range(257, 512, 2)]   # midpoints in [1, 2)
    worst = Fraction(1)
    for mx in range(128, 256):
        for ms in range(128, 256):
            q = Fraction(mx, ms)
            while q < 1:
                q *= 2
            while q >= 2:
                q /= 2
            # nearest midpoint in [1, 2)
            k = min(range(len(mids)), key=lambda i: abs(mids[i] - q))
            d = abs(mids[k] - q) / q
            assert d != 0
            worst = min(worst, d)
    assert worst >= Fraction(1, 2 ** 17)


def test_all_zero_row_scale(oracle):
    _, s, codes = oracle.quant_rows(np.zeros((1, 16), dtype=np.uint16), oracle.BF16)
    assert s[0] == _bf16(np.float32(_bf16(1e-10)) / np.float32(7.0))
    assert not codes.any()
    # f16: the 1e-10 clamp underflows to 0 -> s = 0, codes 0 (0/0)
    _, s, codes = oracle.quant_rows(np.zeros((1, 16), dtype=np.uint16), oracle.F16)
    assert s[0] == 0.0 and not codes.any()


def test_int_gemm_matches_numpy(oracle):
    rs = np.random.RandomState(4)
    xp = rs.randint(-128, 128, size=(7, 48)).astype(np.int8)
    wp = rs.randint(-128, 128, size=(5, 48)).astype(np.int8)
    ref = oracle.unpack(xp).astype(np.int64) @ oracle.unpack(wp).astype(np.int64).T
    assert np.array_equal(oracle.int_gemm(xp, wp), ref)


def test_eager_chain_vs_torch_ops(oracle):
    """epilogue_eager_bf16 against the same chain evaluated with torch bf16 ops."""
    rs = np.random.RandomState(9)
    acc = rs.randint(-50000, 50000, size=(6, 5)).astype(np.int32)
    xs = rs.uniform(0.005, 0.05, 6).astype(np.float32)
    ws = rs.uniform(0.005, 0.05, 5).astype(np.float32)
    b = (rs.standard_normal(5) * 0.01).astype(np.float32)
    t = torch.from_numpy(acc).to(torch.bfloat16)
    t = t * torch.from_numpy(xs).reshape(-1, 1).to(torch.bfloat16)
    t = t * torch.from_numpy(ws).reshape(1, -1).to(torch.bfloat16)
    t = t + torch.from_numpy(b).to(torch.bfloat16).reshape(1, -1)
    assert np.array_equal(oracle.epilogue_eager_bf16(acc, xs, ws, b), np_of(t))


# ----------------------------------------------------------------------------
# W8A8 tier (int8_eager.py)
# ----------------------------------------------------------------------------

def test_golden_int8_config1(oracle, goldens):
    q, s, _ = oracle.rotquant8(bf16_bits(config1_x()), oracle.BF16, 256)
    assert np.array_equal(q[:32], goldens["i8_c1_q_rows32"])
    assert sha(q) == str(goldens["i8_c1_q_sha"])
    assert np.array_equal(s, goldens["i8_c1_s"])
    qw, ws = oracle.quantize_weight8(np_of(config1_weight()), oracle.F16, 256)
    assert np.array_equal(qw[:64], goldens["i8_c1_qw_rows64"])
    assert sha(qw) == str(goldens["i8_c1_qw_sha"])
    assert np.array_equal(ws, goldens["i8_c1_wscale"])


@pytest.mark.parametrize("name", list(edge_cases().keys()))
def test_golden_int8_edge_cases(oracle, goldens, name):
    xe, G = edge_cases()[name]
    dt = DT_OF[xe.dtype]
    q, s, xr = oracle.rotquant8(np_of(xe), dt, G)
    if dt == oracle.F32:
        # torch's fp32 rotation is not correctly rounded (the absmax element may
        # differ in its last bits), so compare the quantizer on torch's own xr
        xr_t = torch.from_numpy(goldens[f"edge_{name}_xr"])
        q, s = oracle.quant_rows8(np_of(xr_t), dt)
    assert np.array_equal(q, goldens[f"i8_edge_{name}_q"])
    assert np.array_equal(s, goldens[f"i8_edge_{name}_s"])


def test_golden_int8_ties_and_largest_quotient(oracle, goldens):
    q, s = oracle.quant_rows8(np_of(tie_rows8()), oracle.BF16)
    assert np.array_equal(q, goldens["i8_ties_q"]) and np.array_equal(s, goldens["i8_ties_s"])
    q, s, _ = oracle.rotquant8(np_of(clamp_rows8()), oracle.BF16, 16)
    assert np.array_equal(q, goldens["i8_maxq_q"]) and np.array_equal(s, goldens["i8_maxq_s"])
    assert q[0, 0] == 126 and q[1, 0] == -126 and s[0] == 1.0078125


def test_golden_int8_linear(oracle, goldens):
    """K = 512: the eager fp32 matmul of int8 codes is exact, so the eager
    output equals the exact-product epilogue bit for bit."""
    x, w, b = small_w8a8_case()
    qw, ws = oracle.quantize_weight8(np_of(w), oracle.F16, 256)
    assert np.array_equal(qw, goldens["i8_lin_qw"]) and np.array_equal(ws, goldens["i8_lin_ws"])
    y = oracle.linear_w8a8(np_of(x), oracle.BF16, qw, ws, b.float().numpy(), 256)
    assert np.array_equal(y, goldens["i8_lin_y"])


def test_int8_quantizer_brute_force_small(oracle):
    """Codes from the eager formula by hand (explicit bf16 roundings, numpy's
    half-to-even round), independent of the oracle's code."""
    rs = np.random.RandomState(12)
    for trial in range(20):
        row = oracle.f32_to_bf16((rs.standard_normal(32) * (0.01 + 3 * trial)).astype(np.float32))
        q, s = oracle.quant_rows8(row.reshape(1, 32), oracle.BF16)
        vals = oracle.bf16_to_f32(row).astype(np.float64)
        a = max(np.abs(vals).max(), _bf16(1e-10))
        sc = _bf16(np.float32(a) / np.float32(127.0))
        assert s[0] == sc
        for k in range(32):
            t = _bf16(np.float32(vals[k]) / np.float32(sc))
            assert q[0, k] == int(np.clip(np.round(t), -127, 127))


def test_int8_quantizer_properties(oracle):
    """Every code within half a step (plus the bf16 quotient rounding) of
    xr / s; the absmax element at +-126 or +-127 (a / s lies in [126.5, 127.25]
    since s = RNE(a / 127) is within 2^-8 of a / 127); odd symmetry; codes in
    [-127, 127]."""
    rs = np.random.RandomState(13)
    x = oracle.f32_to_bf16((rs.standard_t(3, size=(64, 512)) * 2).astype(np.float32))
    q, s = oracle.quant_rows8(x, oracle.BF16)
    v = oracle.bf16_to_f32(x).astype(np.float64)
    z = v / s[:, None].astype(np.float64)
    assert np.all(np.abs(q - z) <= 0.5 + np.abs(z) * 2.0 ** -8)
    qmax = np.abs(q.astype(np.int32)).max(axis=1)
    assert np.all(qmax >= 126) and qmax.max() <= 127 and (qmax == 127).any()
    qn, sn = oracle.quant_rows8(x ^ np.uint16(0x8000), oracle.BF16)
    assert np.array_equal(qn, -q) and np.array_equal(sn, s)


def test_int8_zero_rows(oracle):
    q, s = oracle.quant_rows8(np.zeros((1, 16), dtype=np.uint16), oracle.BF16)
    assert s[0] == _bf16(np.float32(_bf16(1e-10)) / np.float32(127.0)) and not q.any()
    q, s = oracle.quant_rows8(np.zeros((1, 16), dtype=np.uint16), oracle.F16)
    assert s[0] == 0.0 and not q.any()


def test_int8_gemm_matches_numpy(oracle):
    rs = np.random.RandomState(14)
    X = rs.randint(-128, 128, size=(9, 4096)).astype(np.int8)
    W = rs.randint(-128, 128, size=(7, 4096)).astype(np.int8)
    W[0] = -128
    X[0] = -128                                   # |acc| = 2^26: beyond fp32's exact integers
    acc = oracle.int8_gemm(X, W)
    assert np.array_equal(acc, X.astype(np.int64) @ W.astype(np.int64).T)
    assert acc[0, 0] == 128 * 128 * 4096


# ----------------------------------------------------------------------------
# torch restatement of the eager path (the CPU baseline of bench.py)
# ----------------------------------------------------------------------------

def test_torch_eager_reproduces_reference_config1(goldens, oracle):
    """The torch restatement runs the reference's torch operations: on the
    config-1 linear it gives the reference eager output bit for bit (SHA-256
    golden), the reference's activation codes and scales, and the fp16 weight
    codes; its codec inverts the C oracle's on every byte."""
    from oracle import torch_eager as te
    x, w, b = config1_x(), config1_weight(), config1_bias()
    qw, ws = te.quantize_weight(w, 256)
    assert sha(qw.numpy()) == str(goldens["c1_qw_sha"])
    assert np.array_equal(ws.numpy(), goldens["c1_wscale"])
    qx, xs = te.quantize_rows(te.rotate(x, 256))
    assert np.array_equal(qx.numpy(), goldens["c1_qact"]) and np.array_equal(xs.numpy(), goldens["c1_xscale"])
    stages = {}
    y = te.linear(x, qw, ws, b, 256, stage_seconds=stages)
    assert sha(np_of(y)) == str(goldens["c1_y_sha"])
    assert set(stages) == {"rotate", "quantize_pack", "gemm_epilogue"}
    allb = torch.arange(-128, 128, dtype=torch.int32).to(torch.int8).reshape(2, 128)
    assert np.array_equal(te.unpack(allb).numpy(), oracle.unpack(allb.numpy()))
    assert torch.equal(te.pack(te.unpack(allb)), allb)


def test_torch_eager_hadamard_is_an_involution():
    from oracle import torch_eager as te
    for G in (16, 64, 256):
        h = te.block_hadamard(G, torch.float64)
        assert torch.equal(h, h.T)
        assert torch.allclose(h @ h, torch.eye(G, dtype=torch.float64), atol=0, rtol=0)
    with pytest.raises(ValueError):
        te.block_hadamard(32, torch.float32)
