"""Wide-span convrot groups: the reference's eager rotation, the exact oracle and
the rotate+quantize kernel's fp64 rotation (restated in tests/fp64_rotation.py).

The eager rotation is a bf16 matmul whose float accumulation (torch's CPU BLAS)
drops values far below a group's largest; the oracle rotates exactly; the
kernel's fp64 partial sums are exact while a group's nonzero inputs span at
most 36 binades and round beyond.  Where all three are exact they agree bit for
bit (every other golden).  On the wide-span goldens (tests/golden/inputs.py
WIDE_SPAN_CASES, written from the reference by gen_goldens.py) none of them
reproduces the BLAS's rounding, and these tests pin how the kernel's arithmetic
relates to the reference's there."""
import numpy as np
import pytest
import torch

from fp64_rotation import rotate_fp64_kernel_order
from inputs import WIDE_SPAN_CASES, config1_x, outlier_activations, wide_span_rows, wide_span_rows_typed

F32, BF16, F16 = 0, 1, 2
TORCH_DT = {F32: torch.float32, BF16: torch.bfloat16, F16: torch.float16}


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def host(t, dt):
    return t.contiguous().numpy() if dt == F32 else bits(t)


def same(a, b):
    return np.array_equal(a.view(np.uint32 if a.dtype == np.float32 else np.uint16),
                          b.view(np.uint32 if b.dtype == np.float32 else np.uint16))


@pytest.mark.parametrize("G", [16, 64, 256])
def test_fp64_restatement_equals_exact_rotation_on_narrow_groups(oracle, G):
    xs = [outlier_activations(24, 3072, seed=G), outlier_activations(16, 1024, seed=G + 1, student_t=True),
          config1_x()[:8]]
    for x in xs:
        b = bits(x)
        assert np.array_equal(rotate_fp64_kernel_order(b, G), oracle.rotate(b, BF16, G))
    # genuine f32 values (24-bit significands) and f16
    for dt in (F32, F16):
        x = torch.from_numpy(np.random.RandomState(G).standard_normal((24, 3072)).astype(np.float32)).to(TORCH_DT[dt])
        b = host(x, dt)
        assert same(rotate_fp64_kernel_order(b, G, dt), oracle.rotate(b, dt, G))


@pytest.mark.parametrize("kind", ["mixed", "pairs", "ties"])
@pytest.mark.parametrize("G", [16, 64, 256])
def test_fp64_rotation_exact_for_every_f16_input(oracle, kind, G):
    # f16 values are multiples of 2^-24 below 2^16: every partial sum of a
    # group fits 53 bits, so the kernel's fp64 rotation is the exact one even
    # on rows that span the whole f16 range
    x = wide_span_rows_typed(32, 3072 if G > 16 else 1024, G, G + 1, kind, torch.float16)
    b = host(x, F16)
    assert (((b & 0x7c00) == 0) & ((b & 0x3ff) != 0)).any()     # subnormals
    assert ((b & 0x7fff) >= 0x6000).any()                        # and values of 512 and more
    assert same(rotate_fp64_kernel_order(b, G, F16), oracle.rotate(b, F16, G))


def test_fp64_restatement_rounds_on_wide_span_f32(oracle):
    x = wide_span_rows_typed(32, 3072, 256, 3, "pairs", torch.float32)
    b = host(x, F32)
    differ = (rotate_fp64_kernel_order(b, 256, F32).view(np.uint32) != oracle.rotate(b, F32, 256).view(np.uint32)).mean()
    assert differ > 0.1


def test_fp64_restatement_rounds_on_wide_span_ties(oracle):
    # not vacuous: on tie-heavy wide-span rows the fp64 partial sums lose the
    # values that decide the ties, on a few percent of the rotated values
    x = wide_span_rows(32, 3072, 256, 7, "ties")
    b = bits(x)
    differ = (rotate_fp64_kernel_order(b, 256) != oracle.rotate(b, BF16, 256)).mean()
    assert 0.01 < differ < 0.2


@pytest.mark.parametrize("kind,M,K,G", WIDE_SPAN_CASES)
def test_wide_span_goldens(oracle, goldens, kind, M, K, G):
    """Against the reference's own output on wide-span groups: the kernel's
    rotation is never further from it than the exact one (rotated values, int4
    and int8 codes), and its row scales equal the reference's in every case."""
    key = f"wide_{kind}_g{G}"
    b = bits(wide_span_rows(M, K, G, M + K + G, kind))
    exact = oracle.rotate(b, BF16, G)
    fp64 = rotate_fp64_kernel_order(b, G)
    ref = goldens[key + "_xr"]
    assert (fp64 != ref).sum() <= (exact != ref).sum()
    q_e, s_e, _ = oracle.quant_rows(exact, BF16)
    q_k, s_k, _ = oracle.quant_rows(fp64, BF16)
    assert (q_k != goldens[key + "_q"]).sum() <= (q_e != goldens[key + "_q"]).sum()
    assert np.array_equal(s_k.view(np.uint32), goldens[key + "_s"].view(np.uint32))
    q8_e, _ = oracle.quant_rows8(exact, BF16)
    q8_k, s8_k = oracle.quant_rows8(fp64, BF16)
    assert (q8_k != goldens[key + "_q8"]).sum() <= (q8_e != goldens[key + "_q8"]).sum()
    assert np.array_equal(s8_k.view(np.uint32), goldens[key + "_s8"].view(np.uint32))
