"""CPU check of the B6T layout decoder used by the bf6 GPU tests: an
independent bit-by-bit encoder (integers q -> E3M2 codes of q / 16 -> packed groups ->
swizzled, tile-major chunks) must decode back to the integers."""
import numpy as np

from bf6_format import CHUNK, QOFF, bf6_value, decode_b6t, unpack_int4


_VALUES = bf6_value(np.arange(64))


def enc(q: int) -> int:
    """The E3M2 code whose value is q / 16, found by search over all 64 codes
    (+0 for 0)."""
    return int(np.nonzero(_VALUES == q / 16.0)[0].min())


def f(r: int) -> int:
    return (((r >> 1) ^ (r >> 3)) & 1) | ((r >> 1) & 2)


def encode_b6t(q: np.ndarray) -> np.ndarray:
    rows, K = q.shape
    R = (rows + 255) // 256 * 256
    nkb = K // 128
    out = np.zeros(R * K * 3 // 4, np.uint8)
    for row in range(rows):
        t, r = divmod(row, 256)
        rr, odd = r % 32, (r // 32) % 2 == 1
        for kb in range(nkb):
            base = (t * nkb + kb) * CHUNK
            for g in range(4):
                bits = 0
                for e in range(32):
                    bits |= enc(int(q[row, kb * 128 + 32 * g + e])) << (6 * e)
                dw = np.frombuffer(bits.to_bytes(24, "little"), np.uint8)      # d0..d5
                piece = g ^ f(rr)
                p_at = base + r * 64 + 16 * piece
                q_at = base + QOFF + ((r // 64) * 32 + rr) * 64 + 16 * piece
                if not odd:
                    out[p_at:p_at + 16] = dw[0:16]
                    out[q_at:q_at + 8] = dw[16:24]
                else:
                    out[p_at:p_at + 16] = dw[8:24]
                    out[q_at + 8:q_at + 16] = dw[0:8]
    return out


def test_e3m2_codes_of_int4_values():
    """E3M2's subnormals and first binade are 1/16 apart, so the code of q / 16 is
    |q| with the sign in bit 5 (what the kernels' bf6_code_of_int writes)."""
    vals = np.arange(-8, 8)
    assert np.array_equal(bf6_value(np.array([enc(int(q)) for q in vals])) * 16, vals)
    assert [enc(q) for q in (1, 2, 3, 4, 7, -1, -8)] == [1, 2, 3, 4, 7, 0x21, 0x28]
    assert all(enc(int(q)) == ((0x20 if q < 0 else 0) | abs(int(q))) for q in vals)
    assert bf6_value(np.array([0x20]))[0] == 0.0                     # -0 is a zero code


def test_decoder_inverts_reference_encoder():
    rs = np.random.RandomState(0)
    q = rs.randint(-8, 8, size=(300, 256))          # two row tiles, the second one padded
    assert np.array_equal(decode_b6t(encode_b6t(q), 300), q)


def test_unpack_int4_helper():
    p = np.array([[0x87, 0x0F]], dtype=np.uint8).view(np.int8)
    assert unpack_int4(p).tolist() == [[7, -8, -1, 0]]
