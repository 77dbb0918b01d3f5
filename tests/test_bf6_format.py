"""CPU check of the B6T layout decoder used by the bf6 GPU tests: an
independent bit-by-bit encoder (integers -> E3M2 codes -> packed groups ->
swizzled, tile-major chunks) must decode back to the integers."""
import numpy as np

from bf6_format import CHUNK, QOFF, bf6_value, decode_b6t, unpack_int4


def enc(q: int) -> int:
    if q == 0:
        return 0
    a = abs(q)
    e = a.bit_length() - 1
    m = ((a << 2) >> e) & 3
    return (0x20 if q < 0 else 0) | ((e + 3) << 2) | m


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
    vals = np.arange(-8, 8)
    assert np.array_equal(bf6_value(np.array([enc(int(q)) for q in vals])), vals)
    assert [enc(q) for q in (1, 2, 3, 7, -8)] == [12, 16, 18, 23, 56]


def test_decoder_inverts_reference_encoder():
    rs = np.random.RandomState(0)
    q = rs.randint(-8, 8, size=(300, 256))          # two row tiles, the second one padded
    assert np.array_equal(decode_b6t(encode_b6t(q), 300), q)


def test_unpack_int4_helper():
    p = np.array([[0x87, 0x0F]], dtype=np.uint8).view(np.int8)
    assert unpack_int4(p).tolist() == [[7, -8, -1, 0]]
