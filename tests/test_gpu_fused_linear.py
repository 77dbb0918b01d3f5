"""The single-call bf6 linear (cr_convrot_w4a4_linear_bf6, the Linear's forward
path) against the same kernels called one by one: identical bits for every
bias dtype, with and without LoRA, with and without a k split, and against
the oracle's f32 epilogue."""
import numpy as np
import pytest
import torch

from inputs import bf16_bits, normal_bias, normal_weight, outlier_activations

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N,K", [(4608, 3072, 3072), (512, 3072, 12288), (77, 640, 3840), (1, 256, 128)])
@pytest.mark.parametrize("bias_dt", [torch.float16, torch.bfloat16, torch.float32, None])
def test_single_call_equals_steps(backend, native, gpu, M, N, K, bias_dt):
    print(f"fused linear M={M} N={N} K={K} bias={bias_dt}", flush=True)
    G = backend.pick_groupsize(K)
    x = outlier_activations(M, K, seed=M + 3).cuda()
    qw, ws = backend.quantize_convrot_w4a4_weight(normal_weight(N, K, seed=N + 4).cuda(), convrot_groupsize=G)
    w6 = backend.prepare_convrot_w4a4_weight_bf6(qw)
    b = None if bias_dt is None else normal_bias(N, seed=5).to(bias_dt).cuda()
    y = native.convrot_w4a4_linear_bf6(x, w6, ws, b, None, None, 1.0, native.EPI_BF16, G, N)
    a6, xs = native.convrot_quant_bf6(x, G)
    b32 = None if b is None else b.float()
    y1 = native.int4_convrot_gemm_bf6(a6, w6, xs, ws, b32, native.EPI_BF16)
    assert torch.equal(y, y1)
    assert torch.equal(backend.convrot_w4a4_linear(x, qw, ws, bias=b, convrot_groupsize=G, qweight_bf6=w6), y)


@pytest.mark.parametrize("M,N,K,R", [(4608, 3072, 3072, 32), (512, 3072, 12288, 64), (33, 513, 1024, 128),
                                     (1024, 1024, 256, 32), (2000, 640, 1024, 64), (1100, 768, 2048, 32)])
def test_single_call_lora_equals_steps(backend, native, gpu, M, N, K, R):
    x = outlier_activations(M, K, seed=M + 6).cuda()
    qw, ws = backend.quantize_convrot_w4a4_weight(normal_weight(N, K, seed=N + 7).cuda())
    w6 = backend.prepare_convrot_w4a4_weight_bf6(qw)
    b = normal_bias(N, seed=8).cuda()                       # fp16, as the Linear keeps it
    g = torch.Generator(device="cuda").manual_seed(R)
    D = (torch.randn((R, K), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    U = (torch.randn((N, R), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    y = native.convrot_w4a4_linear_bf6(x, w6, ws, b, D, U, 1.0, native.EPI_BF16, 256, N)
    t = native.lora_down(x, D)
    a6, xs = native.convrot_quant_bf6(x, 256)
    y1 = native.int4_convrot_gemm_bf6_lora(a6, w6, xs, ws, b.float(), t, U, 1.0, native.EPI_BF16)
    assert torch.equal(y, y1)


def test_single_call_vs_oracle(backend, native, oracle, gpu):
    M, N, K = 96, 384, 3072
    x = outlier_activations(M, K, seed=9)
    w = normal_weight(N, K, seed=10)
    b = normal_bias(N, seed=11)
    qw, ws = backend.quantize_convrot_w4a4_weight(w.cuda())
    y = backend.convrot_w4a4_linear(x.cuda(), qw, ws, bias=b.cuda())
    eqx, exs, _ = oracle.rotquant(bf16_bits(x), oracle.BF16, 256)
    acc = oracle.int_gemm(eqx, qw.cpu().numpy())
    want = oracle.epilogue_f32(acc, exs, ws.cpu().numpy(), b.float().numpy(), out_bf16=True)
    assert np.array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16), want)


def _lora_pair(N, K, R, seed):
    g = torch.Generator().manual_seed(seed)
    D = (torch.randn(R, K, generator=g) * 0.05).to(torch.bfloat16).cuda()
    U = (torch.randn(N, R, generator=g) * 0.05).to(torch.bfloat16).cuda()
    return D, U


def test_concurrent_host_threads(backend, native, gpu):
    """Six host threads, each on its own stream, call the single-call linear at
    once (the library's launch helpers share per-device caches across threads,
    and the Python layer keeps one workspace per stream): every call returns the
    bits of the same call made alone.  Every other thread adds a rank-32 LoRA,
    whose split down projection and the split GEMM use the workspace."""
    import threading
    cases = [(4608, 3072, 3072), (512, 3072, 12288), (77, 640, 3840), (300, 1024, 9216), (1, 256, 128),
             (640, 768, 2048)]
    prepared = []
    for i, (M, N, K) in enumerate(cases):
        G = backend.pick_groupsize(K)
        x = outlier_activations(M, K, seed=40 + i).cuda()
        qw, ws = backend.quantize_convrot_w4a4_weight(normal_weight(N, K, seed=50 + i).cuda(), convrot_groupsize=G)
        w6 = backend.prepare_convrot_w4a4_weight_bf6(qw)
        b = normal_bias(N, seed=60 + i).cuda()
        D, U = _lora_pair(N, K, 32, 70 + i) if i % 2 == 1 else (None, None)
        want = native.convrot_w4a4_linear_bf6(x, w6, ws, b, D, U, 1.0, native.EPI_BF16, G, N)
        prepared.append((x, w6, ws, b, G, N, D, U, want))
    torch.cuda.synchronize()
    got = [None] * len(cases)
    errors = []
    start = threading.Barrier(len(cases))

    def run(i):
        try:
            x, w6, ws, b, G, N, D, U, _ = prepared[i]
            s = torch.cuda.Stream()
            start.wait(timeout=60)
            with torch.cuda.stream(s):
                outs = [native.convrot_w4a4_linear_bf6(x, w6, ws, b, D, U, 1.0, native.EPI_BF16, G, N)
                        for _ in range(3)]
            s.synchronize()
            got[i] = outs
        except BaseException as e:          # noqa: BLE001 - reported below
            errors.append(e)

    threads = [threading.Thread(target=run, args=(i,)) for i in range(len(cases))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=90)
    assert not errors, errors
    for i, outs in enumerate(got):
        assert outs is not None, f"thread {i} did not finish"
        for y in outs:
            assert torch.equal(y, prepared[i][8]), cases[i]


def test_workspace_reuse_in_stream_order(backend, native, gpu):
    """Linears of different workspace sizes queued back to back on one stream
    (the workspace grows, then is reused by smaller calls) give the bits of the
    same calls made one at a time."""
    cases = [(64, 128, 256, 32), (512, 3072, 12288, 64), (512, 3072, 3072, 32), (4096, 3072, 12288, 32),
             (77, 640, 3840, 96), (512, 3072, 12288, 64)]
    prepared = []
    for i, (M, N, K, R) in enumerate(cases):
        G = backend.pick_groupsize(K)
        x = outlier_activations(M, K, seed=80 + i).cuda()
        qw, ws = backend.quantize_convrot_w4a4_weight(normal_weight(N, K, seed=90 + i).cuda(), convrot_groupsize=G)
        w6 = backend.prepare_convrot_w4a4_weight_bf6(qw)
        b = normal_bias(N, seed=100 + i).cuda()
        D, U = _lora_pair(N, K, R, 110 + i)
        want = native.convrot_w4a4_linear_bf6(x, w6, ws, b, D, U, 1.0, native.EPI_BF16, G, N)
        torch.cuda.synchronize()
        prepared.append((x, w6, ws, b, G, N, D, U, want))
    outs = [native.convrot_w4a4_linear_bf6(x, w6, ws, b, D, U, 1.0, native.EPI_BF16, G, N)
            for (x, w6, ws, b, G, N, D, U, _) in prepared]
    torch.cuda.synchronize()
    for c, y, p in zip(cases, outs, prepared):
        assert torch.equal(y, p[8]), c


@pytest.mark.parametrize("M,N,K,R", [(512, 3072, 3072, 0), (512, 3072, 3072, 32), (512, 3072, 12288, 32),
                                     (4608, 3072, 3072, 64)])
def test_linear_replayed_from_hip_graph(backend, native, gpu, M, N, K, R):
    """The linear captured into a HIP graph (rotate+quant, LoRA down, GEMM with
    its split and epilogue: kernel nodes only, no memset) and replayed with new
    inputs copied into the captured buffer gives the eager call's bits on every
    replay, with eager calls on the same stream between the replays."""
    print(f"graph linear M={M} N={N} K={K} R={R}", flush=True)
    G = backend.pick_groupsize(K)
    qw, ws = backend.quantize_convrot_w4a4_weight(normal_weight(N, K, seed=120).cuda(), convrot_groupsize=G)
    w6 = backend.prepare_convrot_w4a4_weight_bf6(qw)
    b = normal_bias(N, seed=121).cuda()
    lora = _lora_pair(N, K, R, 122) if R else None
    xs = [outlier_activations(M, K, seed=130 + i).cuda() for i in range(4)]

    def call(x):
        return backend.convrot_w4a4_linear(x, qw, ws, b, G, lora=lora, qweight_bf6=w6)

    want = [call(x) for x in xs]
    torch.cuda.synchronize()
    static_x = xs[0].clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call(static_x)                       # warm-up outside the capture (first-use attributes)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = call(static_x)
    for rep in range(2):
        for i, x in enumerate(xs):
            static_x.copy_(x)
            graph.replay()
            eager = call(xs[(i + 1) % len(xs)])   # eager work between replays
            torch.cuda.synchronize()
            assert torch.equal(y, want[i]), (rep, i)
            assert torch.equal(eager, want[(i + 1) % len(xs)]), (rep, i)


@pytest.mark.parametrize("lora", [False, True])
def test_strided_and_batched_inputs_equal_contiguous(backend, native, gpu, lora):
    """A strided view (every other row of a wider buffer, a transposed copy) and
    a [batch, tokens, features] activation give the bits of the same values
    passed contiguous and 2-D, with and without a LoRA."""
    N, K, B, T = 640, 3072, 3, 300
    G = backend.pick_groupsize(K)
    qw, ws = backend.quantize_convrot_w4a4_weight(normal_weight(N, K, seed=31).cuda(), convrot_groupsize=G)
    b = normal_bias(N, seed=32).cuda()
    pair = _lora_pair(N, K, 32, 33) if lora else None
    x3 = outlier_activations(B * T, K, seed=34).reshape(B, T, K).cuda()
    y3 = backend.convrot_w4a4_linear(x3, qw, ws, bias=b, convrot_groupsize=G, lora=pair)
    assert y3.shape == (B, T, N)
    y2 = backend.convrot_w4a4_linear(x3.reshape(B * T, K).contiguous(), qw, ws, bias=b, convrot_groupsize=G, lora=pair)
    assert torch.equal(y3.reshape(B * T, N), y2)
    wide = torch.zeros(2 * B * T, K, dtype=x3.dtype, device="cuda")
    wide[::2] = x3.reshape(B * T, K)
    ys = backend.convrot_w4a4_linear(wide[::2], qw, ws, bias=b, convrot_groupsize=G, lora=pair)
    assert torch.equal(ys, y2)
    xt = x3.reshape(B * T, K).t().contiguous().t()                # column-major storage of the same values
    yt = backend.convrot_w4a4_linear(xt, qw, ws, bias=b, convrot_groupsize=G, lora=pair)
    assert torch.equal(yt, y2)
