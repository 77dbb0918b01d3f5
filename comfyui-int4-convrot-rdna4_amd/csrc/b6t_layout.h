// The B6T operand layout of the bf6 GEMM path (shared by the producers in
// rotquant.hip / gemm_bf6.hip and the GEMM consumer).
//
// A matrix [rows, K] with K % 128 == 0 is stored with rows padded to a
// multiple of 256 (zero codes) as [rows/256][K/128] chunks of 24576 bytes;
// the chunk of (row tile, 128-k block) is one operand half of a GEMM LDS
// stage, so the GEMM copies it with contiguous 1 KB DMA instructions.
//
// Group g of row r is the MFMA operand of k = 128 kb + 32 g .. +31: 32 BF6
// (E3M2, exponent bias 3) codes, code e in bits 6e .. 6e+5 of 6 little-endian
// dwords d0..d5 (lane l of v_mfma_*_f8f6f4 supplies row l % 32, k half l / 32).
// Rows come in 32-row tiles T = r / 32 (r within the chunk) and pairs of
// tiles 2p, 2p+1; rr = r % 32, f = the swz() row function (depends on rr only):
//   P part, bytes     0..16383: row r at r*64; 16-byte piece g ^ f holds
//            d0..d3 of group g when T is even, d2..d5 when T is odd
//   Q part, bytes 16384..24575: (p, rr) at 16384 + (p*32 + rr)*64; 16-byte
//            piece g ^ f holds d4..d5 of group g of row 64p + rr (bytes 0..7)
//            and d0..d1 of group g of row 64p + 32 + rr (bytes 8..15)
// So a fragment read is conflict-free (the swizzle spreads each 16-lane phase
// over all 64 banks), one 16-byte Q read serves the fragments of two row
// tiles, and the registers [P even | Q piece | P odd] hold both 6-dword
// operands contiguously.
#pragma once

#include "common.h"

namespace convrot {

constexpr int B6_CHUNK = 24576;          // bytes of one (256-row tile, 128-k block) chunk
constexpr int B6_QOFF = 16384;           // Q part offset inside a chunk

#ifndef CONVROT_SWZ64
#define CONVROT_SWZ64 1
#endif
// chunk swizzle: row r stores its logical chunk c at physical chunk c ^ f(r).
// With 64-byte rows a 16-byte read of chunk c by rows r..r+15 is conflict-free
// when (r & 3, f(r)) takes 16 distinct values (64 banks x 4 B, 16 lanes per
// phase) and when (r & 1, f(r)) takes 8 distinct values over r..r+7 (32 banks,
// 8 lanes per phase); f = (bit1 ^ bit3) | bit2 << 1 satisfies both.
__host__ __device__ __forceinline__ int swz(int row, int chunk) {
    if (CONVROT_SWZ64) return chunk ^ ((((row >> 1) ^ (row >> 3)) & 1) | ((row >> 1) & 2));
    return chunk ^ ((row >> 1) & 3);
}

// byte offsets of group g's P piece and of its 16-byte Q piece for row r (0..255)
__host__ __device__ __forceinline__ int b6_p_off(int r, int g) { return r * 64 + swz(r, g) * 16; }
__host__ __device__ __forceinline__ int b6_q_off(int r, int g) {
    return B6_QOFF + ((r >> 6) * 32 + (r & 31)) * 64 + swz(r, g) * 16;
}
// The I8T operand layout of the W8A8 GEMM: an int8 matrix [rows, K] (K % 64 ==
// 0, rows padded to a multiple of 256 with zero codes) as [rows/256][K/64]
// chunks of 16384 bytes, each the GEMM's LDS stage image of that operand
// block: row r at r*64, its 16-byte piece c (k = 64 kb + 16 c .. +15) at
// swz(r, c)*16.  The GEMM then copies every chunk with contiguous 1 KB DMA
// instructions.
constexpr int I8T_CHUNK = 16384;
__host__ __device__ __forceinline__ int i8t_off(int r, int c) { return r * 64 + swz(r, c) * 16; }

// odd 32-row tiles keep dwords d0..d1 in the Q piece (its bytes 8..15)
__host__ __device__ __forceinline__ bool b6_odd_tile(int r) { return ((r >> 5) & 1) != 0; }

// BF6 code of an int4 value q (-8..7).  The code holds q / 16: E3M2 (bias 3)
// spaces its subnormals (m / 16, m = 0..3) and its first binade ((4 + m) / 16)
// 1/16 apart, and 8 / 16 = 1.0 * 2^-1 is code 0b01000, so the code of q / 16 is
// |q| itself with the sign in bit 5 (-0, 0x20, is a zero as well).  The GEMMs
// scale both operands by 2^4 (E8M0 block scale 131), so every product is q_a q_b.
// On this grid the gfx950 converter (v_cvt_scalef32_pk32_bf6_bf16 with scale
// 16, which divides) rounds a bf16 value z with |z| <= 8.5 to the code of
// rint_even(z), signed zeros included: checked on every such bf16 value.
constexpr uint32_t bf6_code_of_int(int q) { return (q < 0 ? 0x20u : 0u) | (uint32_t)(q < 0 ? -q : q); }
static_assert(bf6_code_of_int(7) == 7 && bf6_code_of_int(-8) == 0x28 && bf6_code_of_int(-1) == 0x21 &&
              bf6_code_of_int(0) == 0, "bf6");
constexpr int B6_OPERAND_E8M0 = 131;   // MFMA block scale of B6T operands: 2^4

}  // namespace convrot
