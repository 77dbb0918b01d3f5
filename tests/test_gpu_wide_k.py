"""GPU parity of rows wider than 12288 on the product path (the 8- and 16-wave
rotate+quantize instances, K up to 32768) and of the operand decoders that
give back the checkpoint layout from a layer's one device copy.

* cr_bf6_to_int4 / cr_i8t_to_int8 invert cr_int4_to_bf6 / cr_int8_to_i8t bit
  for bit (every nibble, ragged row counts, K up to 32768), and decode the
  activation quantizer's B6T output to the packed quantizer's codes;
* the B6T, I8T and packed quantizers at K in (12288, 32768] (8 waves x 2 or 3
  passes, 16 waves x 2; ragged last passes at K = 13824) equal the oracle on
  sampled rows, for bf16, f16 and f32 inputs;
* the W4A4 linear on the bf6 GEMM and the W8A8 linear on the I8T GEMM at
  K = 13824 and 16384 (Wan-class and 4x4096 FFN down projections), with and
  without the fused LoRA, equal the oracle's linear on sampled rows."""
import numpy as np
import pytest
import torch

from bf6_format import unpack_int4
from inputs import normal_bias, normal_weight, outlier_activations

pytestmark = pytest.mark.gpu

DT = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def host_bits(t):
    t = t.detach().cpu().contiguous()
    return t.numpy() if t.dtype == torch.float32 else t.view(torch.int16).numpy().view(np.uint16)


def cu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("rows,K", [(1, 128), (37, 256), (300, 3072), (64, 12288), (513, 32768)])
def test_bf6_to_int4_inverts_int4_to_bf6(native, gpu, rows, K):
    print(f"bf6_to_int4 rows={rows} K={K}", flush=True)
    p = np.random.RandomState(rows + K).randint(-128, 128, size=(rows, K // 2)).astype(np.int8)
    back = native.bf6_to_int4(native.int4_to_bf6(cu(p)), rows, K)
    assert back.shape == (rows, K // 2) and back.dtype == torch.int8
    assert np.array_equal(back.cpu().numpy(), p)


@pytest.mark.parametrize("rows,K", [(1, 64), (300, 3072), (513, 32768)])
def test_i8t_to_int8_inverts_int8_to_i8t(native, gpu, rows, K):
    print(f"i8t_to_int8 rows={rows} K={K}", flush=True)
    q = np.random.RandomState(rows + K).randint(-128, 128, size=(rows, K)).astype(np.int8)
    back = native.i8t_to_int8(native.int8_to_i8t(cu(q)), rows)
    assert np.array_equal(back.cpu().numpy(), q)


def test_bf6_to_int4_of_activation_codes(native, gpu):
    """The activation quantizer's B6T output (zero codes may carry a sign)
    decodes to the packed quantizer's bytes."""
    x = outlier_activations(700, 3072, seed=11, student_t=True).cuda()
    x[3] = 0.0
    a6, _ = native.convrot_quant_bf6(x, 256)
    q, _ = native.convrot_quant_int4(x, 256)
    assert torch.equal(native.bf6_to_int4(a6, 700, 3072), q)


WIDE = [(300, 13824, torch.bfloat16), (77, 16384, torch.bfloat16), (513, 24576, torch.bfloat16),
        (40, 32768, torch.bfloat16), (129, 16384, torch.float16), (33, 20480, torch.float32),
        (2600, 16384, torch.bfloat16)]


@pytest.mark.parametrize("M,K,dt", WIDE)
def test_wide_quantizers_vs_oracle(native, oracle, gpu, M, K, dt):
    print(f"wide quantizers M={M} K={K} {dt}", flush=True)
    x = outlier_activations(M, K, seed=M + K, student_t=True, dtype=dt)
    if dt == torch.float32:
        x = x.to(torch.bfloat16).float()         # values on a bf16 grid: exact group sums in fp64
    xg = x.cuda()
    a6, s6 = native.convrot_quant_bf6(xg, 256)
    q, s = native.convrot_quant_int4(xg, 256)
    q8t, s8 = native.convrot_quant_int8_i8t(xg, 256)
    q8, s8r = native.convrot_quant_int8(xg, 256)
    torch.cuda.synchronize()
    assert torch.equal(s6, s) and torch.equal(native.bf6_to_int4(a6, M, K), q)
    assert torch.equal(s8, s8r) and torch.equal(native.i8t_to_int8(q8t, M), q8)
    rows = np.unique(np.concatenate([np.random.RandomState(K).choice(M, min(M, 10), replace=False), [0, M - 1]]))
    xb = host_bits(x[rows])
    eq, es, _ = oracle.rotquant(xb, DT[dt], 256)
    assert np.array_equal(q.cpu().numpy()[rows], eq) and np.array_equal(s.cpu().numpy()[rows], es)
    e8, es8, _ = oracle.rotquant8(xb, DT[dt], 256)
    assert np.array_equal(q8.cpu().numpy()[rows], e8) and np.array_equal(s8r.cpu().numpy()[rows], es8)
    # the padding rows of the last 256-row tile hold zero codes
    full = native.bf6_to_int4(a6, native.bf6_rows(M), K)
    assert not bool(full[M:].any())


@pytest.mark.parametrize("M,N,K,lora", [(600, 1024, 13824, False), (300, 3072, 16384, True),
                                        (2049, 512, 16384, False)])
def test_wide_w4a4_linear_vs_oracle(backend, native, oracle, gpu, M, N, K, lora):
    print(f"wide w4a4 linear M={M} N={N} K={K} lora={lora}", flush=True)
    assert backend.bf6_path_ok(K)
    x = outlier_activations(M, K, seed=M)
    qw, ws = backend.quantize_convrot_w4a4_weight(normal_weight(N, K, seed=N).cuda())
    bias = normal_bias(N, seed=5).cuda()
    w6 = backend.prepare_convrot_w4a4_weight_bf6(qw)
    fused = None
    if lora:
        rng = np.random.RandomState(K)
        d = torch.from_numpy((rng.standard_normal((32, K)) * 0.02).astype(np.float32)).cuda()
        u = torch.from_numpy((rng.standard_normal((N, 32)) * 0.1).astype(np.float32)).cuda()
        fused = backend.fuse_lora_pairs([(d, u, 0.5)])
    y = backend.convrot_w4a4_linear(x.cuda(), qw, ws, bias=bias, lora=fused, qweight_bf6=w6)
    # the int8-MFMA kernels on the packed codes: same accumulators and epilogue
    xg = x.cuda()
    qa, xs = native.convrot_quant_int4(xg, 256)
    if lora:
        t = native.lora_down(xg, fused[0])
        y8 = native.int4_convrot_gemm_lora(qa, qw, xs, ws, bias, t, fused[1], 1.0, native.EPI_BF16)
    else:
        y8 = native.int4_convrot_gemm(qa, qw, xs, ws, bias, torch.bfloat16)
    assert torch.equal(y.view(torch.int16), y8.view(torch.int16))
    if not lora:
        rows = np.unique(np.concatenate([np.random.RandomState(N).choice(M, 6, replace=False), [0, M - 1]]))
        eq, es, _ = oracle.rotquant(host_bits(x[rows]), 1, 256)
        acc = oracle.int_gemm(eq, qw.cpu().numpy())
        want = oracle.epilogue_f32(acc, es, ws.cpu().numpy(), bias.float().cpu().numpy(), out_bf16=True)
        assert np.array_equal(host_bits(y)[rows], want)


def test_wide_w8a8_linear_vs_oracle(backend, oracle, gpu):
    M, N, K = 257, 768, 16384
    print(f"wide w8a8 linear M={M} N={N} K={K}", flush=True)
    import importlib
    e8 = importlib.import_module(backend.__name__ + ".int8_eager")
    x = outlier_activations(M, K, seed=9)
    w = normal_weight(N, K, seed=10)
    qw, ws = e8.quantize_convrot_w8a8_weight(w.cuda(), 256)
    eq, es = oracle.quantize_weight8(host_bits(w), oracle.F16, 256)
    assert np.array_equal(qw.cpu().numpy(), eq) and np.array_equal(ws.cpu().numpy(), es)
    w8t = backend.prepare_convrot_w8a8_weight_i8t(qw)
    assert w8t is not None
    b = normal_bias(N, seed=12).cuda()
    y = backend.convrot_w8a8_linear(x.cuda(), qw, ws, bias=b, qweight_i8t=w8t)
    rows = np.array([0, 5, 100, M - 1])
    want = oracle.linear_w8a8(host_bits(x[rows]), oracle.BF16, eq, es, b.float().cpu().numpy(), 256)
    assert np.array_equal(host_bits(y)[rows], want)
