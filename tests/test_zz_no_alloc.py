"""The allocation-free linear entry point (cr_convrot_w4a4_linear_bf6_noalloc)
against the workspace entry point it mirrors (cr_convrot_w4a4_linear_bf6),
called through the C-ABI: identical bits on consecutive calls that reuse the
library's scratch (the second with a smaller input, then a k-split shape and
a LoRA shape), and shapes whose workspace exceeds the scratch are refused."""
import ctypes

import pytest
import torch

from inputs import normal_bias, normal_weight, outlier_activations

pytestmark = pytest.mark.gpu

SCRATCH = 64 << 20


def operands(backend, M, N, K, R, seed):
    x = outlier_activations(M, K, seed=seed).cuda()
    qw, ws = backend.quantize_convrot_w4a4_weight(normal_weight(N, K, seed=seed + 1).cuda())
    w6 = backend.prepare_convrot_w4a4_weight_bf6(qw)
    b = normal_bias(N, seed=seed + 2).cuda()                     # fp16, as the Linear keeps it
    D = U = None
    if R:
        g = torch.Generator(device="cuda").manual_seed(seed)
        D = (torch.randn((R, K), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
        U = (torch.randn((N, R), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    return x, w6, ws, b, D, U


def ptr(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def noalloc(lib, x, w6, ws, b, D, U, R, out, M, N, K):
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return lib.cr_convrot_w4a4_linear_bf6_noalloc(ptr(x), 1, ptr(w6), ptr(ws), ptr(b), 2, ptr(D), ptr(U), R,
                                                  ctypes.c_float(1.0), ptr(out), 1, M, N, K, 256, stream)


def workspace_call(lib, x, w6, ws, b, D, U, R, out, M, N, K):
    nbytes = lib.cr_convrot_w4a4_linear_bf6_workspace(M, N, K, R)
    work = torch.zeros((nbytes,), dtype=torch.uint8, device="cuda")     # the split counters start at zero
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return lib.cr_convrot_w4a4_linear_bf6(ptr(x), 1, ptr(w6), ptr(ws), ptr(b), 2, ptr(D), ptr(U), R,
                                          ctypes.c_float(1.0), ptr(out), 1, M, N, K, 256, ptr(work), nbytes, stream)


# consecutive calls on the shared scratch: a large one, a smaller one, a k-split one, LoRA ranks
CALLS = [(4608, 3072, 3072, 32), (300, 3072, 3072, 0), (512, 3072, 12288, 0), (77, 640, 3840, 64)]


def test_noalloc_matches_workspace_entry_point(backend, native, gpu):
    lib = native.load_library()
    outs = []
    for i, (M, N, K, R) in enumerate(CALLS):
        print(f"noalloc call {i}: M={M} N={N} K={K} R={R}", flush=True)
        assert lib.cr_convrot_w4a4_linear_bf6_workspace(M, N, K, R) <= SCRATCH
        args = operands(backend, M, N, K, R, seed=100 + i)
        out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        assert noalloc(lib, *args, R, out, M, N, K) == 0
        ref = torch.empty_like(out)
        assert workspace_call(lib, *args, R, ref, M, N, K) == 0
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), (M, N, K, R)
        outs.append((args, out))
    # the first shape again after the others: the scratch's stale contents do not leak
    (args, first), (M, N, K, R) = outs[0], CALLS[0]
    again = torch.empty_like(first)
    assert noalloc(lib, *args, R, again, M, N, K) == 0
    torch.cuda.synchronize()
    assert torch.equal(again.view(torch.int16), first.view(torch.int16))


def test_noalloc_refuses_shapes_beyond_the_scratch(native, gpu):
    """A shape whose workspace exceeds 64 MiB returns -1 before any device
    work (null pointers are never touched)."""
    lib = native.load_library()
    M, N, K = 16384, 3072, 12288
    assert lib.cr_convrot_w4a4_linear_bf6_workspace(M, N, K, 0) > SCRATCH
    n = ctypes.c_void_p(0)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.cr_convrot_w4a4_linear_bf6_noalloc(n, 1, n, n, n, 0, n, n, 0, ctypes.c_float(1.0), n, 1, M, N, K, 256,
                                                  s) == -1


def test_noalloc_replays_from_a_captured_graph(backend, native, gpu):
    """After one call on the device (which looks up the scratch's address and
    sets the kernels' LDS limits, neither of them a stream operation), the
    entry point records into a HIP graph: every replay, with other calls on the
    same scratch in between, gives the workspace entry point's bits."""
    lib = native.load_library()
    M, N, K, R = 1024, 3072, 3072, 32
    print(f"noalloc graph capture: M={M} N={N} K={K} R={R}", flush=True)
    args = operands(backend, M, N, K, R, seed=200)
    ref = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    assert workspace_call(lib, *args, R, ref, M, N, K) == 0
    out = torch.empty_like(ref)
    assert noalloc(lib, *args, R, out, M, N, K) == 0          # the first call on this device, before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = noalloc(lib, *args, R, out, M, N, K)
    assert rc == 0
    other = operands(backend, 300, 640, 3840, 0, seed=201)
    other_out = torch.empty((300, 640), dtype=torch.bfloat16, device="cuda")
    for i in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), i
        # an eager call of another shape overwrites the scratch before the next replay
        assert noalloc(lib, *other, 0, other_out, 300, 640, 3840) == 0
        torch.cuda.synchronize()
