"""numpy helpers for the operand layouts of the GEMM paths (test helper): the B6T decoder of the bf6 path and the I8T re-layout of the W8A8 path.

B6T of a [rows, K] matrix (K % 128 == 0): rows padded to R = ceil(rows/256)*256
(zero codes), stored as [R/256][K/128] chunks of 24576 bytes.  An int4 value q
is held as the BF6 (E3M2, bias 3) code of q / 16 (the GEMM scales both operands
by 2^4).  Group g of row r = the 32 codes of k = 128 kb + 32 g .. +31, code e at bits
6e .. 6e+5 of 6 little-endian dwords d0..d5.  In a chunk, with T = r // 32,
rr = r % 32 and f(rr) = ((rr>>1 ^ rr>>3) & 1) | (rr>>1 & 2): the 16-byte piece
g ^ f(rr) at r*64 holds d0..d3 (T even) or d2..d5 (T odd); the 16-byte piece
g ^ f(rr) at 16384 + ((r // 64)*32 + rr)*64 holds d4..d5 of the even-tile row
64p + rr (bytes 0..7) and d0..d1 of the odd-tile row 64p + 32 + rr (bytes 8..15)."""
import numpy as np

CHUNK = 24576
QOFF = 16384


def bf6_value(code: np.ndarray) -> np.ndarray:
    """E3M2 bias-3 codes -> float64 values (normal numbers, subnormals, zero)."""
    code = code.astype(np.int64)
    s = np.where(code & 0x20, -1.0, 1.0)
    e = (code >> 2) & 7
    m = code & 3
    mag = np.where(e == 0, m / 4.0 * 2.0 ** -2, 2.0 ** (e - 3.0) * (1 + m / 4.0))
    return s * mag


def p_row_fn(r: np.ndarray) -> np.ndarray:
    return (((r >> 1) ^ (r >> 3)) & 1) | ((r >> 1) & 2)


def decode_b6t(b6: np.ndarray, rows: int) -> np.ndarray:
    """uint8 B6T buffer -> int64 values [rows, K] (asserts every code is an integer
    and every padding row is zero)."""
    flat = np.ascontiguousarray(b6).reshape(-1)
    R = (rows + 255) // 256 * 256
    K = flat.size // R // 3 * 4
    nkb = K // 128
    ch = flat.reshape(R // 256, nkb, CHUNK)
    r = np.arange(256)
    rr = r % 32
    odd = (r // 32) % 2 == 1
    g = np.arange(4)
    piece = g[None, :] ^ p_row_fn(rr)[:, None]                         # [256, 4]
    P = ch[:, :, :QOFF].reshape(R // 256, nkb, 256, 4, 16)
    Q = ch[:, :, QOFF:].reshape(R // 256, nkb, 128, 4, 16)
    qrow = (r // 64) * 32 + rr                                          # Q row of row r
    Pg = P[:, :, r[:, None], piece]                                     # [T, nkb, 256, 4, 16]
    Qg = Q[:, :, qrow[:, None], piece]                                  # [T, nkb, 256, 4, 16]
    even_bytes = np.concatenate([Pg, Qg[..., :8]], axis=-1)             # d0..d3 | d4..d5
    odd_bytes = np.concatenate([Qg[..., 8:], Pg], axis=-1)              # d0..d1 | d2..d5
    grp = np.where(odd[None, None, :, None, None], odd_bytes, even_bytes)   # [T, nkb, 256, 4, 24]
    bits = np.unpackbits(grp, axis=-1, bitorder="little")
    code = (bits.reshape(*grp.shape[:-1], 32, 6) * (1 << np.arange(6))).sum(-1)   # [T, nkb, 256, 4, 32]
    vals = bf6_value(code) * 16.0                                       # codes hold q / 16
    assert np.all(vals == np.round(vals)), "bf6 code off the 1/16 grid"
    full = vals.transpose(0, 2, 1, 3, 4).reshape(R, K).astype(np.int64)
    assert not full[rows:].any(), "padding rows must hold zero codes"
    return full[:rows]


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """int8 [rows, K/2] -> int64 [rows, K] (low nibble first, two's complement)."""
    p = packed.astype(np.int64) & 0xFF
    lo = ((p & 15) ^ 8) - 8
    hi = ((p >> 4) ^ 8) - 8
    return np.stack([lo, hi], -1).reshape(packed.shape[0], -1)


def i8t_np(q):
    """Host re-layout of int8 codes [rows, K] into I8T, written from the layout's
    definition: [ceil(rows/256)][K/64] chunks of 256 rows x 64 bytes, row r at
    r*64, its 16-byte piece c at (c ^ f(r))*16, padding rows zero."""
    rows, K = q.shape
    tiles, nkb = (rows + 255) // 256, K // 64
    qp = np.zeros((tiles * 256, K), dtype=np.int8)
    qp[:rows] = q
    qt = qp.reshape(tiles, 256, nkb, 4, 16).transpose(0, 2, 1, 3, 4)        # [t, kb, r, c, 16]
    r = np.arange(256)
    f = (((r >> 1) ^ (r >> 3)) & 1) | ((r >> 1) & 2)
    idx = np.arange(4)[None, :] ^ f[:, None]                                  # slot p holds piece p ^ f(r)
    out = np.take_along_axis(qt, idx[None, None, :, :, None], axis=3)
    return out.reshape(tiles * 256, K)
