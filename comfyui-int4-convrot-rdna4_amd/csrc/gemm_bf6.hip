// W4A4 GEMM on the bf6 matrix cores of gfx950, with bit-exact accumulators.
//
// CDNA4 has no int4 matrix instruction, but its v_mfma_scale_f32_32x32x64_f8f6f4
// runs 6-bit float operands at twice the int8 rate, and BF6 (E3M2, exponent
// bias 3) represents every int4 value -8..7 exactly.  Products of two such
// values are integers of magnitude <= 64, and every partial sum of a K-term dot
// product is an integer of magnitude <= 64 K < 2^24 for K < 262144, so the fp32
// accumulation is exact in any order: the accumulators equal the int32 ones of
// the reference int4 GEMM bit for bit, and the epilogues are the int8 kernels'
// (gemm_common.h).  The B6T codes hold q / 16 (b6t_layout.h); block scales of
// 2^4 on both operands (E8M0 131) are exact and make every product q_a q_b.
//
// Operands are in the B6T layout (b6t_layout.h), produced by
// int4_to_bf6t_kernel from the packed int4 layout or directly by the fused
// rotate+quant kernel (rotquant.hip).

#include <type_traits>

#include "gemm_common.h"

namespace convrot {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

// codes of nibbles base .. base+7 (two's complement int4), 6 bits each
constexpr uint64_t bf6_nibble_table(int base) {
    uint64_t t = 0;
    for (int i = 0; i < 8; ++i) {
        const int n = base + i;
        t |= (uint64_t)bf6_code_of_int(n >= 8 ? n - 16 : n) << (6 * i);
    }
    return t;
}

__device__ __forceinline__ uint32_t bf6_of_nibble(uint32_t n) {
    constexpr uint64_t LO = bf6_nibble_table(0), HI = bf6_nibble_table(8);
    const uint64_t t = (n & 8) ? HI : LO;
    return (uint32_t)(t >> ((n & 7) * 6)) & 63u;
}

// 32 packed nibbles (element e = nibble e of the 16 bytes, low nibble first)
// -> one 6-dword bf6 operand
__device__ __forceinline__ void encode_group(uint4 p, uint32_t (&d)[6]) {
    const uint32_t w[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
    for (int i = 0; i < 6; ++i) d[i] = 0;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
        const uint32_t code = bf6_of_nibble((w[e >> 3] >> ((e & 7) * 4)) & 15u);
        const int bit = 6 * e;
        d[bit >> 5] |= code << (bit & 31);
        if ((bit & 31) > 26) d[(bit >> 5) + 1] |= code >> (32 - (bit & 31));
    }
}

// packed int4 [rows, K/2] -> B6T; one thread per (row, 128-k block) of the
// padded matrix, consecutive threads on consecutive rows of one chunk.
__global__ __launch_bounds__(256) void int4_to_bf6t_kernel(const uint8_t* __restrict__ src,
                                                           uint8_t* __restrict__ dst, int rows, int K) {
    const int nkb = K / 128;
    const long long id = (long long)blockIdx.x * 256 + threadIdx.x;
    const int tiles = (rows + 255) / 256;
    if (id >= (long long)tiles * nkb * 256) return;
    const int r = (int)(id & 255);
    const long long tk = id >> 8;                        // tile * nkb + kb
    const int tile = (int)(tk / nkb), kb = (int)(tk % nkb);
    const int row = tile * 256 + r;
    uint4 in[4] = {};
    if (row < rows) {
        const uint4* s = reinterpret_cast<const uint4*>(src + (size_t)row * (K / 2) + (size_t)kb * 64);
#pragma unroll
        for (int g = 0; g < 4; ++g) in[g] = s[g];
    }
    uint8_t* d = dst + (size_t)tk * B6_CHUNK;
    const bool odd = b6_odd_tile(r);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        uint32_t c[6];
        encode_group(in[g], c);
        if (!odd) {
            *reinterpret_cast<uint4*>(d + b6_p_off(r, g)) = make_uint4(c[0], c[1], c[2], c[3]);
            *reinterpret_cast<uint2*>(d + b6_q_off(r, g)) = make_uint2(c[4], c[5]);
        } else {
            *reinterpret_cast<uint4*>(d + b6_p_off(r, g)) = make_uint4(c[2], c[3], c[4], c[5]);
            *reinterpret_cast<uint2*>(d + b6_q_off(r, g) + 8) = make_uint2(c[0], c[1]);
        }
    }
}

// int4 value of a B6T code (bf6_code_of_int: |q| in bits 0..4, sign in bit 5;
// 0 and -0 -> 0)
__device__ __forceinline__ int int_of_bf6(uint32_t c) {
    const int a = (int)(c & 31u);
    return (c & 0x20u) ? -a : a;
}

// B6T -> packed int4 [rows, K/2] (the inverse of int4_to_bf6t_kernel on the
// first `rows` rows): one thread per (row, 32-code group), 16 bytes out.
__global__ __launch_bounds__(256) void bf6t_to_int4_kernel(const uint8_t* __restrict__ src,
                                                           uint8_t* __restrict__ dst, int rows, int K) {
    const int ng = K / 32;
    const long long id = (long long)blockIdx.x * 256 + threadIdx.x;
    if (id >= (long long)rows * ng) return;
    const int row = (int)(id / ng), gi = (int)(id % ng);
    const int kb = gi >> 2, g = gi & 3, r = row & 255;
    const uint8_t* chunk = src + ((size_t)(row >> 8) * (K / 128) + kb) * B6_CHUNK;
    const uint4 p = *reinterpret_cast<const uint4*>(chunk + b6_p_off(r, g));
    const uint4 q = *reinterpret_cast<const uint4*>(chunk + b6_q_off(r, g));
    uint32_t d[6];
    if (!b6_odd_tile(r)) {          // P = d0..d3, Q bytes 0..7 = d4..d5
        d[0] = p.x; d[1] = p.y; d[2] = p.z; d[3] = p.w; d[4] = q.x; d[5] = q.y;
    } else {                        // P = d2..d5, Q bytes 8..15 = d0..d1
        d[0] = q.z; d[1] = q.w; d[2] = p.x; d[3] = p.y; d[4] = p.z; d[5] = p.w;
    }
    uint32_t o[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int e = 0; e < 32; ++e) {
        const int bit = 6 * e;
        uint32_t c = d[bit >> 5] >> (bit & 31);
        if ((bit & 31) > 26) c |= d[(bit >> 5) + 1] << (32 - (bit & 31));
        o[e >> 3] |= ((uint32_t)int_of_bf6(c & 63u) & 15u) << ((e & 7) * 4);
    }
    *reinterpret_cast<uint4*>(dst + (size_t)row * (K / 2) + (size_t)gi * 16) = make_uint4(o[0], o[1], o[2], o[3]);
}

// ---------------------------------------------------------------------------
// GEMM: 256 x 256 tile per workgroup of 8 waves (2 along M x 4 along N, wave
// tile 128 x 64 = 4 x 2 MFMA tiles of 32 x 32).  A stage is the A chunk and
// the B chunk of one 128-k block (48 KB), copied by global_load_lds_dwordx4
// (6 contiguous 1 KB instructions per wave), three stages deep.  Per block
// and wave: 2 k steps x 8 MFMAs over 9 ds_read_b128 fragment reads per k step
// (6 P pieces, 3 Q pieces each shared by two row tiles).  The epilogue goes
// through LDS (epilogue_lds).
// ---------------------------------------------------------------------------

constexpr int B6_BM = 256, B6_BN = 256;
constexpr int B6_THREADS = 512;
constexpr int B6_STAGES = 3;
constexpr int B6_STAGE_BYTES = 2 * B6_CHUNK;              // A chunk + B chunk: 48 KB
constexpr int B6_LOADS = B6_STAGE_BYTES / 16 / B6_THREADS; // 6 DMA instructions per lane
static_assert(B6_LOADS == 6, "the main loop issues a block's copies in slots 2, 4, 6 of two phases");
constexpr int B6_RING_BYTES = B6_STAGES * B6_STAGE_BYTES;  // 144 KB
constexpr int B6_LDS_BYTES = B6_RING_BYTES + EPI_SCALE_FLOATS * 4;
constexpr int BF6_FMT = 3;                                 // f8f6f4 operand format code of BF6 (E3M2)

typedef unsigned v4u __attribute__((ext_vector_type(4)));

// operand of an even row tile: d0..d3 from its P piece, d4..d5 from bytes 0..7 of the Q piece
__device__ __forceinline__ v8i bf6_operand_even(v4u p, v4u q) {
    return (v8i){(int)p.x, (int)p.y, (int)p.z, (int)p.w, (int)q.x, (int)q.y, 0, 0};
}
// operand of an odd row tile: d0..d1 from bytes 8..15 of the Q piece, d2..d5 from its P piece
__device__ __forceinline__ v8i bf6_operand_odd(v4u q, v4u p) {
    return (v8i){(int)q.z, (int)q.w, (int)p.x, (int)p.y, (int)p.z, (int)p.w, 0, 0};
}

// SPLIT: split-K partial kernel.  Workgroup b takes tile b % T and the 128-k
// blocks [s nkb / S, (s + 1) nkb / S) of split s = b / T (T tiles, S splits),
// and stores its raw accumulators (exact integers in fp32) in the workspace in
// register order, 32 KB per wave: part[((s T + tile) 8 + wave) * 8192 +
// (q * 64 + lane) * 4 + e] = acc[q / 8][(q / 4) % 2][4 (q % 4) + e].  The
// scales, the epilogue and the LoRA term run once per output, in the reduce
// kernel below.
template <int EPI, int LR, bool SPLIT>
__global__ __launch_bounds__(B6_THREADS) void w4a4_gemm_bf6_kernel(
        const uint8_t* __restrict__ A6, const uint8_t* __restrict__ W6,
        const float* __restrict__ xs, const float* __restrict__ ws, const void* __restrict__ bias, int bias_dt,
        void* __restrict__ out, int M, int N, int K, LoraArgs lora, int gm, int nsplit,
        float* __restrict__ part) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds6[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3;
    const int tiles_m = (M + B6_BM - 1) / B6_BM, tiles_n = (N + B6_BN - 1) / B6_BN;
    const int nkb_all = K / 128;
    int tm, tn, kb0 = 0, nkb = nkb_all, split = 0, tile = 0;
    if constexpr (SPLIT) {
        const int T = tiles_m * tiles_n;
        split = blockIdx.x / T;
        tile = blockIdx.x - split * T;
        tm = tile % tiles_m;
        tn = tile / tiles_m;
        kb0 = (int)((long long)split * nkb_all / nsplit);
        nkb = (int)((long long)(split + 1) * nkb_all / nsplit) - kb0;
    } else {
        tile_of_block(blockIdx.x, tiles_m, tiles_n, gm, tm, tn);
    }
    const int m0 = tm * B6_BM;
    const int n0 = tn * B6_BN;

    float* sc = reinterpret_cast<float*>(lds6 + B6_RING_BYTES);
    ScaleRegs scr;                                            // staged in LDS after the main loop
    if constexpr (!SPLIT) scr.load(xs, ws, bias, bias_dt, M, N, m0, n0, tid);

    // waves 0..3 copy the A chunk of a block, waves 4..7 the B chunk (6 KB each)
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    const uint8_t* my_chunks = (wave_u < 4 ? A6 + (size_t)tm * nkb_all * B6_CHUNK
                                           : W6 + (size_t)tn * nkb_all * B6_CHUNK) + (size_t)kb0 * B6_CHUNK;
    const uint8_t* my_src = my_chunks + (wave_u & 3) * (B6_LOADS * 1024) + lane * 16;
    const uint32_t my_lds = (uint32_t)(uintptr_t)lds6 + wave_u * (B6_LOADS * 1024);
    v16f acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (v16f){0};

    const int frow = lane & 31;
    const int fhalf = lane >> 5;
    // Per-lane byte offsets of this lane's fragments inside a stage, for the two
    // k steps (group g = 2 s2 + half).  The P-chunk swizzle and the Q-slot
    // permutation depend only on row bits 1..4, so the fragments of row tiles
    // i = 1..3 sit at fixed distances (i * 2048 in P, i * 1024 in Q).
    // Per-lane byte offsets of this lane's P pieces and Q pieces inside a stage,
    // for the two k steps (group g = 2 s2 + half).  The swizzle depends on row
    // bits 1..4 only, so row tile i sits at i * 2048 in P and tile pair p at
    // p * 2048 in Q.  The wave's first A and B row tiles are even.
    uint32_t offPa[2], offQa[2], offPb[2], offQb[2];
    {
        const int ra = wm * 128 + frow, rb = wn * 64 + frow;
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            const int g = 2 * s2 + fhalf;
            offPa[s2] = b6_p_off(ra, g);
            offQa[s2] = b6_q_off(ra, g);
            offPb[s2] = B6_CHUNK + b6_p_off(rb, g);
            offQb[s2] = B6_CHUNK + b6_q_off(rb, g);
        }
    }
    // Fragments of one k step: P pieces of the 4 A and 2 B row tiles, and the 16-byte
    // Q pieces shared by row tiles (0, 1) and (2, 3) of A and (0, 1) of B.
    // (native vector registers: a HIP uint4 assignment from LDS would be an
    // aggregate copy through private memory)
    struct Frags { v4u pa[4], qa[2], pb[2], qb; };
    // read r (0..8) of k step s2 of the block in the stage at byte offset st
    auto read_one = [&](uint32_t st, int s2, int r, Frags& f) __attribute__((always_inline)) {
        const uint8_t* base = lds6 + st;
        if (r < 4) f.pa[r] = *reinterpret_cast<const v4u*>(base + offPa[s2] + r * 2048);
        else if (r < 6) f.qa[r - 4] = *reinterpret_cast<const v4u*>(base + offQa[s2] + (r - 4) * 2048);
        else if (r < 8) f.pb[r - 6] = *reinterpret_cast<const v4u*>(base + offPb[s2] + (r - 6) * 2048);
        else f.qb = *reinterpret_cast<const v4u*>(base + offQb[s2]);
    };
    // MFMA t (0..7) of a k step: A row tile t / 2 against B row tile t % 2
    auto mfma_one = [&](const Frags& f, int t) __attribute__((always_inline)) {
        const int i = t >> 1, j = t & 1;
        const v4u q = f.qa[i >> 1], p = f.pa[i], qb = f.qb, pb = f.pb[j];
        const v8i fa = (i & 1) ? bf6_operand_odd(q, p) : bf6_operand_even(p, q);
        const v8i fb = j ? bf6_operand_odd(qb, pb) : bf6_operand_even(pb, qb);
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(   // transposed tile
                fb, fa, acc[i][j], BF6_FMT, BF6_FMT, 0, B6_OPERAND_E8M0, 0, B6_OPERAND_E8M0);
    };
    // the reads issued after MFMA slot t, in the order the next k step's MFMAs
    // consume them: pb0 qb | pa0 qa0 | pb1 pa1 | pa2 qa1 | pa3 (all in the first
    // five slots, so they have landed when the phase ends)
    auto reads_after = [&](int t, uint32_t st, int s2, Frags& f) __attribute__((always_inline)) {
        if (t == 0) { read_one(st, s2, 6, f); read_one(st, s2, 8, f); }
        if (t == 1) { read_one(st, s2, 0, f); read_one(st, s2, 4, f); }
        if (t == 2) { read_one(st, s2, 7, f); read_one(st, s2, 1, f); }
        if (t == 3) { read_one(st, s2, 2, f); read_one(st, s2, 5, f); }
        if (t == 4) read_one(st, s2, 3, f);
    };
    // DMA instruction j of block kb (past the end: a repeat of the last block)
    // Tile rounds on an XCD (workgroup b runs on XCD b % 8, whose 32 CUs take
    // its workgroups b / 8 = 0..31, 32..63, ... in rounds) alternate the
    // direction of their k walk: a tile of an odd round starts with the k
    // blocks the previous round ended with, whose chunks of the row panels the
    // two rounds share are still in that XCD's L2.  Exact integer products: the
    // sum is the same in any order.  Interleaved A/B on MI355X, M = 4608: qkv
    // 85.6 -> 84.7 us, mlp_up 114.0 -> 111.3 us, one-round shapes unchanged.
    const bool krev = !SPLIT && ((blockIdx.x >> 3) / 32 & 1);
    auto dma_one = [&](int kb, int j) __attribute__((always_inline)) {
        const uint32_t st = my_lds + (kb % B6_STAGES) * B6_STAGE_BYTES;
        const int kc = min(kb, nkb - 1);
        dma16(st + j * 1024, my_src + (size_t)(krev ? nkb - 1 - kc : kc) * B6_CHUNK + j * 1024);
    };
    // Rank-32 LoRA with a bf16 output: the epilogue's t rows m0 .. m0+255 and U
    // rows n0 .. n0+255 (64 bytes each, 32 KB in all, read once per workgroup
    // instead of once per wave) are copied into the ring while the last blocks
    // are multiplied: in phase B of block kb_tu = max(nkb - 2, 0), into that
    // block's stage, in place of the past-the-end copies that would have gone
    // there (the last block's phase A skips its own past-the-end copy into the
    // same stage).  Copy q (0..3) of wave w is 1 KB chunk c = 4 w + q: t rows
    // m0 + 16 c .. for c < 16, U rows n0 + 16 (c - 16) .. above; rows past M / N
    // repeat the last one (they feed only outputs that are never stored).
    constexpr bool LSTAGE = !SPLIT && LR == 1 && (EPI == EPI_BF16 || EPI == EPI_BF16_EAGER);
    const int kb_tu = nkb >= 2 ? nkb - 2 : 0;
    auto dma_tu = [&](uint32_t st, int q) __attribute__((always_inline)) {
        const int c = wave_u * 4 + q;                            // wave-uniform
        const bool is_t = c < 16;
        const int r0 = is_t ? m0 + c * 16 : n0 + (c - 16) * 16;   // may lie past M / N (edge tiles)
        const int last = (is_t ? M : N) - 1;
        // byte offset from the start of t / U: the lane's row, clamped into the
        // matrix (0 <= row <= last, so the copy never leaves it)
        const uint32_t voff = (uint32_t)min(r0 + (lane >> 2), last) * 64 + (lane & 3) * 16;
        dma16_sv((uint32_t)(uintptr_t)lds6 + st + c * 1024, is_t ? lora.t : lora.U, voff);
    };

    // Hand-scheduled pipeline, two phases per 128-k block kb, three stages.  Phase
    // A: the 8 MFMAs of k step 0 (fragments read in the previous phase B), the
    // first five followed by the fragment reads of k step 1, slots 2, 4 and 6 by
    // one DMA instruction each of the second half of block kb+2 (into block kb-1's
    // stage).  Then wait until this wave's copies of block kb+1 have landed and
    // its reads of block kb are done, and pass the barrier: the copies of block
    // kb+1 are visible and no wave reads block kb's stage any more.  Phase B: the
    // 8 MFMAs of k step 1, followed by the fragment reads of k step 0 of block kb+1
    // and, in slots 2, 4 and 6, the first half of block kb+3 (into block kb's
    // stage).  Spreading the copies over both phases, one every other slot, keeps
    // a stalled copy from holding back consecutive MFMAs (2-4% over six copies in
    // a row); sched_barrier(0) pins every slot.
    Frags F0, F1;
#pragma unroll
    for (int j = 0; j < B6_LOADS; ++j) dma_one(0, j);
#pragma unroll
    for (int j = 0; j < B6_LOADS; ++j) dma_one(1, j);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(B6_LOADS));          // block 0 landed, block 1 in flight
    __syncthreads();
#pragma unroll
    for (int j = 0; j < B6_LOADS / 2; ++j) dma_one(2, j);    // first half; the second in phase A of block 0
#pragma unroll
    for (int r = 0; r < 9; ++r) read_one(0, 0, r, F0);
    uint32_t st_cur = 0;                                      // stage of block kb
    // One 128-k block.  MODE 0: the copies described above; MODE 1 (block
    // kb_tu, LSTAGE): phase B copies t / U instead of block kb+3's first half;
    // MODE 2 (the last block, LSTAGE, nkb >= 2): phase A copies nothing.  The
    // LSTAGE blocks run as separate loop bodies, so the common one carries no
    // extra branches or registers.
    auto block = [&](int kb, auto mode_c) __attribute__((always_inline)) {
        constexpr int MODE = decltype(mode_c)::value;
        const uint32_t st_nxt = st_cur == (B6_STAGES - 1) * B6_STAGE_BYTES ? 0u : st_cur + B6_STAGE_BYTES;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            mfma_one(F0, t);
            __builtin_amdgcn_sched_barrier(0);
            if (MODE != 2 && (t == 2 || t == 4 || t == 6)) dma_one(kb + 2, B6_LOADS / 2 + (t - 2) / 2);
            reads_after(t, st_cur, 1, F1);
            __builtin_amdgcn_sched_barrier(0);
        }
        // this wave's copies of block kb+1 landed (the six of block kb+2 may be in
        // flight) and its reads of block kb done: after the barrier block kb's
        // stage is free
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(B6_LOADS) & 0xc07f);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            mfma_one(F1, t);
            __builtin_amdgcn_sched_barrier(0);
            if (t == 2 || t == 4 || t == 6) {
                if (MODE == 1) {
                    dma_tu(st_cur, t == 2 ? 0 : t == 4 ? 1 : 2);
                    if (t == 6) dma_tu(st_cur, 3);
                } else {
                    dma_one(kb + 3, (t - 2) / 2);
                }
            }
            reads_after(t, st_nxt, 0, F0);
            __builtin_amdgcn_sched_barrier(0);
        }
        st_cur = st_nxt;
    };
    if constexpr (LSTAGE) {
        for (int kb = 0; kb < kb_tu; ++kb) block(kb, std::integral_constant<int, 0>{});
        block(kb_tu, std::integral_constant<int, 1>{});
        if (nkb >= 2) block(nkb - 1, std::integral_constant<int, 2>{});
    } else {
        for (int kb = 0; kb < nkb; ++kb) block(kb, std::integral_constant<int, 0>{});
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));                 // the copies past the end have landed

    if constexpr (SPLIT) {
        float4* dst = reinterpret_cast<float4*>(part) +
                      ((size_t)(split * tiles_m * tiles_n + tile) * 8 + wave) * 2048 + lane;
#pragma unroll
        for (int q = 0; q < 32; ++q) {
            const v16f& a = acc[q >> 3][(q >> 2) & 1];
            const int r = 4 * (q & 3);
            dst[q * 64] = make_float4(a[r], a[r + 1], a[r + 2], a[r + 3]);
        }
        return;
    }
    scr.store(sc, bias, bias_dt, M, N, m0, n0, tid);
    __syncthreads();                                     // every wave is done with the stages; scales staged
    // keep the epilogue's index arithmetic out of the main loop's registers
    int em0 = m0, en0 = n0, elane = lane;
    asm volatile("" : "+s"(M), "+s"(N), "+v"(em0), "+v"(en0), "+v"(elane));
    if constexpr (LSTAGE) {
        // t / U sit in the first 32 KB of stage kb_tu % 3; the waves' output
        // scratch (12 KB each) fills the other two stages
        const int tu = kb_tu % B6_STAGES;
        constexpr int SCR = 2 * B6_STAGE_BYTES / (B6_THREADS / 64);
        uint8_t* scr = lds6 + ((tu + 1 + (wave >> 2)) % B6_STAGES) * B6_STAGE_BYTES + (wave & 3) * SCR;
        epilogue_lds<EPI, 4, 2, LR, SCR>(acc, sc, out, M, N, em0, en0, em0 + wm * 128, en0 + wn * 64, elane, lora,
                                         scr, lds6 + tu * B6_STAGE_BYTES);
    } else {
        constexpr int SCR = B6_RING_BYTES / (B6_THREADS / 64);
        epilogue_lds<EPI, 4, 2, LR, SCR>(acc, sc, out, M, N, em0, en0, em0 + wm * 128,
                                         en0 + wn * 64, elane, lora, lds6 + wave * SCR);
    }
}

// ---------------------------------------------------------------------------
// Small grids: tiles of UA x UB units of 64 rows (BM = 64 UA rows of A, BN =
// 64 UB rows of B), one wave per 64 x 64 piece (2 x 2 MFMA 32 x 32 tiles, 8
// MFMAs per 128-k block and wave).  With 256 x 256 tiles a grid of few row
// tiles (M <= 2048 or so) leaves most CUs idle.  Two shapes are built: 128 x
// 128 (the quarter tile, 4 waves, three stages) and 128 x 192 (6 waves, four
// stages), the latter for grids whose 128 x 128 tiles would put two
// workgroups on some CUs while its own cover the CUs once
// (gemm_bf6_small_shape below).
// A 64-row unit of a B6T chunk (rows 64h .. 64h+63) is its P bytes h*4096 ..
// +4095 and its Q rows 32h .. 32h+31 (bytes 16384 + h*2048 .. +2047), copied
// into LDS as [P 4 KB][Q 2 KB]: a stage is the tile's A units, then its B
// units, of one 128-k block (6 KB, 6 DMA instructions per unit), in a ring
// of NST stages.  A wave's 64 rows of A are one unit, and so are its 64 rows of
// B: the fragment offsets of a local row rl < 64 are those of the full chunk
// with the unit's Q part at 4096 (the swizzle depends on row bits 1..4 only).
// Units of an edge tile past the operand's padded rows re-read the last unit
// (they feed only outputs that are never stored).  Same two-phase schedule as
// the big kernel: per phase 4 MFMAs, the first three each followed by the
// next k step's fragment reads in consumption order and by a third of the
// phase's DMA instructions (phase A: the second part of block kb+NST-1,
// phase B: the first part of block kb+NST).  Same accumulators, same epilogue: the
// outputs equal the 256 x 256 kernel's bit for bit.
//
// SPLIT (S = nsplit > 1): workgroup b takes tile b % T and the 128-k blocks
// [s nkb / S, (s + 1) nkb / S) of split s = b / T.
// Every workgroup stores its raw accumulators (exact integers in fp32) in the
// workspace with device-scope stores, waits until they are done and takes a
// ticket from the tile's counter; the one that draws the last ticket adds the
// other S - 1 partials to its own (exact in any order: integers below 2^24),
// sets the counter back to zero and runs the epilogue.
// No workgroup waits for another, so no launch order or residency can stall
// the grid.  The counters (one per tile, at most 512) must be zero when a
// workspace is first used; every call leaves them zero.
// ---------------------------------------------------------------------------
constexpr int B6S_UNIT = 6144;                                  // 64 rows of a chunk: P 4 KB + Q 2 KB
constexpr int B6S_UNIT_Q = 4096;                                // Q part inside a unit
constexpr int B6S_STAGES = 3;                                   // 128 x 128: 4 and 6 measured no faster
constexpr int B6S_MAX_SPLIT_TILES = 512;                        // split counters per workspace
constexpr int B6S_BM = 128, B6S_BN = 128;                       // the quarter tile

template <int UA, int UB, int NST_ = B6S_STAGES>
struct B6Small {
    static constexpr int NST = NST_;                            // ring stages
    static constexpr int BM = 64 * UA, BN = 64 * UB;
    static constexpr int WAVES = UA * UB;
    static constexpr int THREADS = 64 * WAVES;
    static constexpr int UNITS = UA + UB;
    static constexpr int STAGE_BYTES = UNITS * B6S_UNIT;
    static constexpr int LOADS = 6 * UNITS / WAVES;             // DMA instructions per wave and block
    static constexpr int LOADS_B = LOADS / 2;                    // first part: NST blocks ahead, phase B
    static constexpr int LOADS_A = LOADS - LOADS_B;              // second part: NST-1 blocks ahead, phase A
    static constexpr int RING_BYTES = NST * STAGE_BYTES;
    static constexpr int LDS_BYTES = RING_BYTES + EPI_SCALE_FLOATS * 4 + 16;   // + the split ticket
    static_assert(6 * UNITS % WAVES == 0, "whole DMA instructions per wave");
    static_assert((NST - 2) * LOADS + LOADS_B <= 63 && NST >= 3, "vmcnt range");
    static_assert(BM <= 256 && BN <= 256 && THREADS >= BM && THREADS >= BN, "staged scales");
};
static_assert(B6Small<2, 2>::BM == B6S_BM && B6Small<2, 2>::BN == B6S_BN, "quarter tile");

// tile shapes of the small kernel (gemm_bf6_small_shape)
enum : int { SMALL_128x128 = 0, SMALL_128x192 = 1 };
constexpr int B6S_STAGES_192 = 4;                              // ring stages of the 128 x 192 shape

template <int EPI, int LR, bool SPLIT, int UA, int UB, int NSTAGES>
__global__ __launch_bounds__(64 * UA * UB) void w4a4_gemm_bf6_small_kernel(
        const uint8_t* __restrict__ A6, const uint8_t* __restrict__ W6,
        const float* __restrict__ xs, const float* __restrict__ ws, const void* __restrict__ bias, int bias_dt,
        void* __restrict__ out, int M, int N, int K, LoraArgs lora, int gm, int nsplit,
        float* __restrict__ part, unsigned* __restrict__ cnt) {
    using S = B6Small<UA, UB, NSTAGES>;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds6[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / UB, wn = wave % UB;
    const int tiles_m = (M + S::BM - 1) / S::BM, tiles_n = (N + S::BN - 1) / S::BN;
    const int nkb_all = K / 128;
    int tm, tn, kb0 = 0, nkb = nkb_all, split = 0, tix = blockIdx.x;
    if constexpr (SPLIT) {
        const int T = tiles_m * tiles_n;
        split = blockIdx.x / T;
        tix = blockIdx.x - split * T;
        kb0 = (int)((long long)split * nkb_all / nsplit);
        nkb = (int)((long long)(split + 1) * nkb_all / nsplit) - kb0;
    }
    tile_of_block(tix, tiles_m, tiles_n, gm, tm, tn);
    const int m0 = tm * S::BM;
    const int n0 = tn * S::BN;

    float* sc = reinterpret_cast<float*>(lds6 + S::RING_BYTES);
    ScaleRegs scr;                                              // staged in LDS after the main loop
    scr.load(xs, ws, bias, bias_dt, M, N, m0, n0, tid);

    // Copy j (0 .. LOADS-1) of this wave is instruction i = wave * LOADS + j of the
    // stage's 6 * UNITS: KB i % 6 (P 0..3, Q 4..5) of unit i / 6 (A units, then B
    // units).  Per copy: this lane's source at the split's first block, and the
    // copy's LDS offset inside a stage (wave-uniform).
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    const int last_a = ((M + 255) >> 8) * 4 - 1, last_b = ((N + 255) >> 8) * 4 - 1;   // last 64-row units
    const uint8_t* csrc[S::LOADS];
    uint32_t cdst[S::LOADS];
#pragma unroll
    for (int j = 0; j < S::LOADS; ++j) {
        const int ins = wave_u * S::LOADS + j;
        const int u = ins / 6, o = ins - 6 * u;
        const bool is_a = u < UA;
        const int gr = is_a ? min((m0 >> 6) + u, last_a) : min((n0 >> 6) + u - UA, last_b);   // 64-row unit
        const int h = gr & 3;
        const int off = o < 4 ? h * 4096 + o * 1024 : B6_QOFF + h * 2048 + (o - 4) * 1024;
        csrc[j] = (is_a ? A6 : W6) + ((size_t)(gr >> 2) * nkb_all + kb0) * B6_CHUNK + off + lane * 16;
        cdst[j] = (uint32_t)(uintptr_t)lds6 + u * B6S_UNIT + o * 1024;
    }
    auto dma_one = [&](int kb, int j) __attribute__((always_inline)) {
        dma16(cdst[j] + (kb % S::NST) * S::STAGE_BYTES, csrc[j] + (size_t)min(kb, nkb - 1) * B6_CHUNK);
    };
    // the copies of one part issued after MFMA slot t (1..3) of a phase: a third each
    auto dma_part = [&](int kb, int t, int first, int n) __attribute__((always_inline)) {
#pragma unroll
        for (int j = n * (t - 1) / 3; j < n * t / 3; ++j) dma_one(kb, first + j);
    };

    v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (v16f){0};

    const int frow = lane & 31;
    const int fhalf = lane >> 5;
    // per-lane byte offsets (inside a stage) of this lane's P and Q pieces for the
    // two k steps; the wave's A rows are unit wm, its B rows unit UA + wn, and its
    // second row tile of either sits 2048 bytes further in P
    uint32_t offPa[2], offQa[2], offPb[2], offQb[2];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
        const int g = 2 * s2 + fhalf;
        offPa[s2] = wm * B6S_UNIT + b6_p_off(frow, g);
        offQa[s2] = wm * B6S_UNIT + B6S_UNIT_Q + b6_q_off(frow, g) - B6_QOFF;
        offPb[s2] = (UA + wn) * B6S_UNIT + b6_p_off(frow, g);
        offQb[s2] = (UA + wn) * B6S_UNIT + B6S_UNIT_Q + b6_q_off(frow, g) - B6_QOFF;
    }
    struct Frags { v4u pa[2], qa, pb[2], qb; };
    auto read_one = [&](uint32_t st, int s2, int r, Frags& f) __attribute__((always_inline)) {
        const uint8_t* base = lds6 + st;
        if (r < 2) f.pa[r] = *reinterpret_cast<const v4u*>(base + offPa[s2] + r * 2048);
        else if (r == 2) f.qa = *reinterpret_cast<const v4u*>(base + offQa[s2]);
        else if (r < 5) f.pb[r - 3] = *reinterpret_cast<const v4u*>(base + offPb[s2] + (r - 3) * 2048);
        else f.qb = *reinterpret_cast<const v4u*>(base + offQb[s2]);
    };
    // MFMA t (0..3): A row tile t / 2 against B row tile t % 2
    auto mfma_one = [&](const Frags& f, int t) __attribute__((always_inline)) {
        const int i = t >> 1, j = t & 1;
        const v8i fa = i ? bf6_operand_odd(f.qa, f.pa[1]) : bf6_operand_even(f.pa[0], f.qa);
        const v8i fb = j ? bf6_operand_odd(f.qb, f.pb[1]) : bf6_operand_even(f.pb[0], f.qb);
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(   // transposed tile
                fb, fa, acc[i][j], BF6_FMT, BF6_FMT, 0, B6_OPERAND_E8M0, 0, B6_OPERAND_E8M0);
    };
    // reads issued after MFMA slot t, in the order the next k step consumes them:
    // pa0 qa | pb0 qb | pb1 pa1
    auto reads_after = [&](int t, uint32_t st, int s2, Frags& f) __attribute__((always_inline)) {
        if (t == 0) { read_one(st, s2, 0, f); read_one(st, s2, 2, f); }
        if (t == 1) { read_one(st, s2, 3, f); read_one(st, s2, 5, f); }
        if (t == 2) { read_one(st, s2, 4, f); read_one(st, s2, 1, f); }
    };

    // Ring of NST stages, block b in stage b % NST: blocks 0 .. NST-2 and the
    // first part of NST-1 in the prologue; at block kb, phase A copies the second
    // part of block kb+NST-1 (into block kb-1's stage) and phase B the first
    // part of block kb+NST (into block kb's stage, free after the barrier).
    constexpr int NST = S::NST;
    Frags F0, F1;
#pragma unroll
    for (int b = 0; b < NST - 1; ++b)
#pragma unroll
        for (int j = 0; j < S::LOADS; ++j) dma_one(b, j);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm((NST - 2) * S::LOADS));   // block 0 landed, blocks 1 .. NST-2 in flight
    __syncthreads();
#pragma unroll
    for (int j = 0; j < S::LOADS_B; ++j) dma_one(NST - 1, j);   // first part; the second in phase A of block 0
#pragma unroll
    for (int r = 0; r < 6; ++r) read_one(0, 0, r, F0);
    uint32_t st_cur = 0;
    for (int kb = 0; kb < nkb; ++kb) {
        const uint32_t st_nxt = st_cur == (NST - 1) * S::STAGE_BYTES ? 0u : st_cur + S::STAGE_BYTES;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            mfma_one(F0, t);
            __builtin_amdgcn_sched_barrier(0);
            if (t >= 1) dma_part(kb + NST - 1, t, S::LOADS_B, S::LOADS_A);
            reads_after(t, st_cur, 1, F1);
            __builtin_amdgcn_sched_barrier(0);
        }
        // this wave's copies of block kb+1 landed (those of blocks kb+2 .. kb+NST-1
        // may be in flight) and its reads of block kb done: after the barrier block
        // kb's stage is free
        __builtin_amdgcn_s_waitcnt(vmcnt_imm((NST - 2) * S::LOADS) & 0xc07f);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            mfma_one(F1, t);
            __builtin_amdgcn_sched_barrier(0);
            if (t >= 1) dma_part(kb + NST, t, 0, S::LOADS_B);
            reads_after(t, st_nxt, 0, F0);
            __builtin_amdgcn_sched_barrier(0);
        }
        st_cur = st_nxt;
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));                 // the copies past the end have landed
    __syncthreads();                                          // every wave is done with the stages
    if constexpr (SPLIT) {
        // Partial of split s: value q (0..63) of a lane is acc[q / 32][(q / 16) % 2][q % 16], at
        // part[((s T + tile) WAVES + wave) 4096 + q 64 + lane].  Written and read with device-scope
        // relaxed atomic accesses (coherent across the XCDs' L2 caches without writing an L2 back);
        // each wave's vmcnt(0) before the barrier orders its stores before the ticket.
        const int T = tiles_m * tiles_n;
        auto slot = [&](int s) { return part + ((size_t)(s * T + tix) * S::WAVES + wave) * 4096 + lane; };
        float* dst = slot(split);
#pragma unroll
        for (int q = 0; q < 64; ++q)
            __hip_atomic_store(dst + q * 64, acc[q >> 5][(q >> 4) & 1][q & 15], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));             // this wave's partial is stored
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __syncthreads();                                      // ... and every other wave's
        unsigned* ticket = reinterpret_cast<unsigned*>(lds6 + S::RING_BYTES + EPI_SCALE_FLOATS * 4);
        if (tid == 0) *ticket = __hip_atomic_fetch_add(cnt + tix, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (*ticket != (unsigned)nsplit - 1) return;          // another split finishes this tile
        if (tid == 0) __hip_atomic_store(cnt + tix, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int s = 0; s < nsplit; ++s) {
            if (s == split) continue;
            const float* src = slot(s);
            float p[64];
#pragma unroll
            for (int q = 0; q < 64; ++q) p[q] = __hip_atomic_load(src + q * 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int q = 0; q < 64; ++q) acc[q >> 5][(q >> 4) & 1][q & 15] += p[q];
        }
    }
    scr.store(sc, bias, bias_dt, M, N, m0, n0, tid);
    __syncthreads();
    int em0 = m0, en0 = n0, elane = lane;
    asm volatile("" : "+s"(M), "+s"(N), "+v"(em0), "+v"(en0), "+v"(elane));
    constexpr int SCR = S::RING_BYTES / S::WAVES;
    epilogue_lds<EPI, 2, 2, LR, SCR, 8, true>(acc, sc, out, M, N, em0, en0, em0 + wm * 64, en0 + wn * 64, elane,
                                              lora, lds6 + wave * SCR);
}

// Split-K reduce: one 256-lane workgroup per (tile, wave slot) of the main
// kernel; its wave v takes the slot's 32-row tile v.  A wave sums the S
// partials of its 32 x 64 piece in split order (exact: integers below 2^24)
// into the main kernel's accumulator layout and runs the same epilogue code on
// it, so every output equals the unsplit kernel's bit for bit.
constexpr int B6R_WAVES = 4;
constexpr int B6R_SCR = 32 * (2 * 32 * 4 + 16);        // one 32-row f32 pass of the epilogue scratch

template <int EPI, int LR>
__global__ __launch_bounds__(64 * B6R_WAVES) void w4a4_bf6_splitk_reduce_kernel(
        const float* __restrict__ part, int nsplit, const float* __restrict__ xs, const float* __restrict__ ws,
        const void* __restrict__ bias, int bias_dt, void* __restrict__ out, int M, int N, LoraArgs lora) {
    __shared__ __attribute__((aligned(16))) float sc[EPI_SCALE_FLOATS];
    __shared__ __attribute__((aligned(16))) uint8_t scr[B6R_WAVES][B6R_SCR];
    const int lane = threadIdx.x & 63;
    const int v = threadIdx.x >> 6;                      // row tile of the slot
    const int tiles_m = (M + B6_BM - 1) / B6_BM, tiles_n = (N + B6_BN - 1) / B6_BN;
    const int T = tiles_m * tiles_n;
    const int tile = blockIdx.x >> 3, w = blockIdx.x & 7;
    const int tm = tile % tiles_m, tn = tile / tiles_m;
    const int m0 = tm * B6_BM, n0 = tn * B6_BN;
    const int wm = w >> 2, wn = w & 3;
    stage_scales(sc, xs, ws, bias, bias_dt, M, N, m0, n0, threadIdx.x, 64 * B6R_WAVES);
    v16f acc[1][2];
    acc[0][0] = (v16f){0};
    acc[0][1] = (v16f){0};
    for (int s = 0; s < nsplit; ++s) {
        const float4* src = reinterpret_cast<const float4*>(part) + ((size_t)(s * T + tile) * 8 + w) * 2048 +
                            (size_t)v * 8 * 64 + lane;
        float4 q4[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) q4[q] = src[q * 64];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            v16f& a = acc[0][q >> 2];
            const int r = 4 * (q & 3);
            a[r] += q4[q].x; a[r + 1] += q4[q].y; a[r + 2] += q4[q].z; a[r + 3] += q4[q].w;
        }
    }
    __syncthreads();                                     // staged scales visible
    epilogue_lds<EPI, 1, 2, LR, B6R_SCR>(acc, sc, out, M, N, m0, n0, m0 + wm * 128 + v * 32, n0 + wn * 64,
                                         lane, lora, scr[v]);
}

bool gemm_bf6_small_tiles(int M, int N, int K);
int gemm_bf6_small_shape(int M, int N, int K, int nsplit);

// One launch of the small kernel of shape (UA, UB) with NST stages, split nsplit ways.
template <int EPI, int LR, int UA, int UB, int NST = B6S_STAGES>
static hipError_t launch_small(const uint8_t* A6, const uint8_t* W6, const float* xs, const float* ws,
                               const void* bias, int bias_dt, void* out, int M, int N, int K, const LoraArgs& la,
                               int nsplit, float* part, unsigned* cnt, int dev, hipStream_t st) {
    using S = B6Small<UA, UB, NST>;
    const int sm = (M + S::BM - 1) / S::BM;
    const int sn = (N + S::BN - 1) / S::BN;
    if (nsplit <= 1) {
        static std::atomic<bool> attr[kMaxDev];
        const hipError_t e = lds_limit_once(
                attr, dev, reinterpret_cast<const void*>(&w4a4_gemm_bf6_small_kernel<EPI, LR, false, UA, UB, NST>),
                S::LDS_BYTES);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL((w4a4_gemm_bf6_small_kernel<EPI, LR, false, UA, UB, NST>), dim3(sm * sn), dim3(S::THREADS),
                           S::LDS_BYTES, st, A6, W6, xs, ws, bias, bias_dt, out, M, N, K, la, tile_group_rows(sm), 1,
                           nullptr, nullptr);
        return hipGetLastError();
    }
    {
        static std::atomic<bool> attr[kMaxDev];
        const hipError_t e = lds_limit_once(
                attr, dev, reinterpret_cast<const void*>(&w4a4_gemm_bf6_small_kernel<EPI, LR, true, UA, UB, NST>),
                S::LDS_BYTES);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL((w4a4_gemm_bf6_small_kernel<EPI, LR, true, UA, UB, NST>), dim3(sm * sn * nsplit),
                           dim3(S::THREADS), S::LDS_BYTES, st, A6, W6, xs, ws, bias, bias_dt, out, M, N, K, la,
                           tile_group_rows(sm), nsplit, part, cnt);
        return hipGetLastError();
    }
}

// Every split workspace starts with the counters of the small-tile kernel's
// split (B6S_MAX_SPLIT_TILES of them, kSplitCounterBytes); the partials follow.
static_assert(B6S_MAX_SPLIT_TILES * 4 == kSplitCounterBytes, "counter region of the documented workspace layout");

template <int EPI, int LR>
static hipError_t launch_bf6(const uint8_t* A6, const uint8_t* W6, const float* xs, const float* ws,
                             const void* bias, int bias_dt, void* out, int M, int N, int K, const LoraArgs& la,
                             int nsplit, float* part, hipStream_t st) {
    static std::atomic<bool> attr_set[kMaxDev];
    static std::atomic<bool> attr_split[kMaxDev];
    int dev = 0;
    hipError_t e = current_device(&dev);
    if (e != hipSuccess) return e;
    // workspace (nsplit > 1): the split counters, then the partials
    unsigned* cnt = nullptr;
    if (nsplit > 1) {
        cnt = reinterpret_cast<unsigned*>(part);
        part = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(part) + kSplitCounterBytes);
    }
    if (gemm_bf6_small_tiles(M, N, K)) {
        if (gemm_bf6_small_shape(M, N, K, nsplit) == SMALL_128x192)
            return launch_small<EPI, LR, 2, 3, B6S_STAGES_192>(A6, W6, xs, ws, bias, bias_dt, out, M, N, K, la, nsplit,
                                                               part, cnt, dev, st);
        return launch_small<EPI, LR, 2, 2>(A6, W6, xs, ws, bias, bias_dt, out, M, N, K, la, nsplit, part, cnt, dev,
                                           st);
    }
    const int tiles_m = (M + B6_BM - 1) / B6_BM;
    const int ntiles = tiles_m * ((N + B6_BN - 1) / B6_BN);
    if (nsplit <= 1) {
        e = lds_limit_once(attr_set, dev, reinterpret_cast<const void*>(&w4a4_gemm_bf6_kernel<EPI, LR, false>),
                           B6_LDS_BYTES);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL((w4a4_gemm_bf6_kernel<EPI, LR, false>), dim3(ntiles), dim3(B6_THREADS), B6_LDS_BYTES,
                           st, A6, W6, xs, ws, bias, bias_dt, out, M, N, K, la, tile_group_rows(tiles_m), 1, nullptr);
        return hipGetLastError();
    }
    // the partial kernel is the same for every epilogue and LoRA rank
    e = lds_limit_once(attr_split, dev, reinterpret_cast<const void*>(&w4a4_gemm_bf6_kernel<EPI_ACC, 0, true>),
                       B6_LDS_BYTES);
    if (e != hipSuccess) return e;
    const LoraArgs none{nullptr, nullptr, 0, 0.0f};
    hipLaunchKernelGGL((w4a4_gemm_bf6_kernel<EPI_ACC, 0, true>), dim3(ntiles * nsplit), dim3(B6_THREADS),
                       B6_LDS_BYTES, st, A6, W6, nullptr, nullptr, nullptr, 0, nullptr, M, N, K, none, 1, nsplit, part);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((w4a4_bf6_splitk_reduce_kernel<EPI, LR>), dim3(ntiles * 8), dim3(64 * B6R_WAVES), 0, st,
                       part, nsplit, xs, ws, bias, bias_dt, out, M, N, la);
    return hipGetLastError();
}

hipError_t int4_to_bf6_launch(const void* src, void* dst, int rows, int K, hipStream_t st) {
    if (rows == 0) return hipSuccess;
    const long long n = (long long)((rows + 255) / 256) * (K / 128) * 256;
    hipLaunchKernelGGL(int4_to_bf6t_kernel, dim3((unsigned)(n / 256)), dim3(256), 0, st,
                       reinterpret_cast<const uint8_t*>(src), reinterpret_cast<uint8_t*>(dst), rows, K);
    return hipGetLastError();
}

hipError_t bf6_to_int4_launch(const void* src, void* dst, int rows, int K, hipStream_t st) {
    if (rows == 0) return hipSuccess;
    const long long n = (long long)rows * (K / 32);
    hipLaunchKernelGGL(bf6t_to_int4_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       reinterpret_cast<const uint8_t*>(src), reinterpret_cast<uint8_t*>(dst), rows, K);
    return hipGetLastError();
}

hipError_t gemm_bf6_launch(const void* A6, const void* W6, const float* xs, const float* ws, const void* bias,
                           int bias_dt, const void* t, const void* U, int R, float scale, void* out, int M, int N,
                           int K, int epi, int nsplit, void* workspace, hipStream_t st) {
    float* part = reinterpret_cast<float*>(workspace);
    if (M == 0 || N == 0) return hipSuccess;
    const uint8_t* a = reinterpret_cast<const uint8_t*>(A6);
    const uint8_t* w = reinterpret_cast<const uint8_t*>(W6);
    if (t == nullptr) {
        const LoraArgs none{nullptr, nullptr, 0, 0.0f};
        switch (epi) {
            case EPI_F32: return launch_bf6<EPI_F32, 0>(a, w, xs, ws, bias, bias_dt, out, M, N, K, none, nsplit, part, st);
            case EPI_BF16: return launch_bf6<EPI_BF16, 0>(a, w, xs, ws, bias, bias_dt, out, M, N, K, none, nsplit, part, st);
            case EPI_BF16_EAGER: return launch_bf6<EPI_BF16_EAGER, 0>(a, w, xs, ws, bias, bias_dt, out, M, N, K, none, nsplit, part, st);
            case EPI_ACC: return launch_bf6<EPI_ACC, 0>(a, w, xs, ws, bias, bias_dt, out, M, N, K, none, nsplit, part, st);
            default: return hipErrorInvalidValue;
        }
    }
    const LoraArgs la{reinterpret_cast<const __bf16*>(t), reinterpret_cast<const __bf16*>(U), R, scale};
    if (R % 32 != 0 || R < 32 || R > 128) return hipErrorInvalidValue;
#define BF6_LORA_CASE(LRV)                                                                                      \
    case LRV:                                                                                                   \
        switch (epi) {                                                                                          \
            case EPI_F32: return launch_bf6<EPI_F32, LRV>(a, w, xs, ws, bias, bias_dt, out, M, N, K, la, nsplit, part, st);            \
            case EPI_BF16: return launch_bf6<EPI_BF16, LRV>(a, w, xs, ws, bias, bias_dt, out, M, N, K, la, nsplit, part, st);          \
            case EPI_BF16_EAGER: return launch_bf6<EPI_BF16_EAGER, LRV>(a, w, xs, ws, bias, bias_dt, out, M, N, K, la, nsplit, part, st); \
            default: return hipErrorInvalidValue;                                                               \
        }
    switch (R / 32) {
        BF6_LORA_CASE(1) BF6_LORA_CASE(2) BF6_LORA_CASE(3) BF6_LORA_CASE(4)
        default: return hipErrorInvalidValue;
    }
#undef BF6_LORA_CASE
}

// Number of k splits for an M x N x K product (1: no split).  Cost model,
// fitted to kernel traces of M = 512 .. 2048 and K = 3072 .. 12288: a launch
// runs in waves of 256 workgroups (one per CU); a workgroup costs 0.82 us per
// 128-k block plus 2.5 us; a split adds the reduce kernel, 3.1 us plus 0.09 us
// per (tile, split) partial (256 KB written and read back).  A split must win
// by 8% to be taken.
// The 128 x 128 kernel when its grid stays within about two workgroups per CU
// and rows are short, or the grid is small enough for the kernel's own split
// (long rows on at most 192 quarter tiles); other long rows go through the
// k-split 256 x 256 kernel.  Measured against the 256 x 256 kernel with its
// chosen split (HIP events, bf16 out): 512 x 3072 -> 3072 16.8 / 25.4 us,
// 1024 x 3072 -> 3072 17.5 / 23.8, 2048 x 3072 -> 3072 23.5 / 26.3, 512 x
// 3072 -> 12288 22.0 / 24.5, 512 x 3840 -> 15360 26.9 / 28.6; but 1024 x
// 3072 -> 9216 34.5 / 26.3 and, unsplit, 512 x 12288 -> 3072 41.1 / 32.2.
// Burst-timed on MI355X with the quarter-tile split (below): 512 x 12288 ->
// 3072 27.6 us (S = 2) against 30.0 for the 256 x 256 split and reduce, 1024 x
// 12288 -> 3072 39.3 against 40.0; 2048 x 12288 -> 3072 63.8 unsplit against
// 60.4, so 384 quarter tiles with long rows stay on the 256 x 256 kernel.
bool gemm_bf6_small_tiles(int M, int N, int K) {
    const long long tiles = (long long)((M + B6S_BM - 1) / B6S_BM) * ((N + B6S_BN - 1) / B6S_BN);
    return tiles <= B6S_MAX_SPLIT_TILES && (K <= 4096 || tiles <= 192);
}

// Tile shape of a small-kernel launch: 128 x 192 when its grid covers the CUs
// once (split workgroups included) and the 128 x 128 one does not (more than
// 256 workgroups put two on some CUs); otherwise 128 x 128.  Measured on
// MI355X (bursts of launches, bf16 out, us, 128 x 128 / 128 x 192 with 4
// stages), K = 3072: 512 -> 9216 17.9 / 16.2, 512 -> 12288 19.5 / 17.4, 768 ->
// 6144 17.6 / 16.0, 1024 -> 6144 19.1 / 17.2, 1536 -> 3072 17.5 / 15.8, 2048
// -> 3072 18.7 / 17.0; where 128 x 128 fits the CUs (512 -> 3072 12.9 / 15.0,
// 512 -> 6144 13.5 / 15.6) or 128 x 192 does not (512 x 3840 -> 15360 25.9 /
// 35.5, 768 -> 9216 20.1 / 29.5) the 128 x 128 tile wins.  Split in two, K =
// 12288: 1024 -> 3072 37.9 / 35.9, 768 -> 3072 35.1 / 32.1, 512 -> 6144 38.1 /
// 35.6.  A 64 x 128 tile (2 waves) costs as much per 128-k block as 128 x 128
// with 2 to 4 stages and never won.
int gemm_bf6_small_shape(int M, int N, int K, int nsplit) {
    (void)K;
    const long long tm = (M + 127) / 128;
    const long long t128 = tm * ((N + 127) / 128) * nsplit, t192 = tm * ((N + 191) / 192) * nsplit;
    return t128 > 256 && t192 <= 256 ? SMALL_128x192 : SMALL_128x128;
}

// The workgroup tile (rows of A x rows of B) of a bf6 GEMM launch.
void gemm_bf6_tile(int M, int N, int K, int nsplit, int* bm, int* bn) {
    if (!gemm_bf6_small_tiles(M, N, K)) { *bm = B6_BM; *bn = B6_BN; return; }
    *bm = 128;
    *bn = gemm_bf6_small_shape(M, N, K, nsplit) == SMALL_128x192 ? 192 : 128;
}

// Splits of the quarter-tile kernel.  Its launch costs about 5.5 us however
// short the rows (6.1 us at K = 256, M x N = 512 x 3072: the first copies'
// latency, the epilogue and the store drain), a 128-k block 0.35 us with one
// workgroup per CU, and two workgroups on a CU run each at about half speed;
// the split's partial exchange (device-scope stores, the ticket, the last
// split's loads) adds 4-5 us.  So a split pays only for long rows on a grid
// that leaves CUs free: measured at 512 x K -> 3072 (96 tiles), K = 3072
// 13.7 us unsplit / 13.9 split in two, K = 6144 22.0 / 18.5, K = 12288 38.9 /
// 27.4 (S = 4: 27.5); 1024 x 12288 -> 3072 (192 tiles) 44.0 / 39.3; at
// K = 3072 no split won on any of 15 shapes.  Grids of 129 to 192 quarter
// tiles split in two run on 128 x 192 tiles (at most 256 workgroups, see
// gemm_bf6_small_shape), and only for rows of 64 blocks or more: 1024 x 6144
// -> 3072 runs 22.2 us unsplit against 23.6 split on 128 x 192 (24.3 on 128 x
// 128).
static int small_nsplit(int M, int N, int K) {
    const int T = ((M + B6S_BM - 1) / B6S_BM) * ((N + B6S_BN - 1) / B6S_BN);
    const int nkb = K / 128;
    if (nkb < 48) return 1;
    if (T <= 64 && nkb >= 96) return 4;
    if (T <= 128) return 2;
    return T <= 192 && nkb >= 64 ? 2 : 1;     // split in two on 128 x 192 tiles
}

int gemm_bf6_choose_nsplit(int M, int N, int K) {
    if (gemm_bf6_small_tiles(M, N, K)) return small_nsplit(M, N, K);
    const int tiles = ((M + B6_BM - 1) / B6_BM) * ((N + B6_BN - 1) / B6_BN);
    const int nkb = K / 128;
    auto cost = [&](int s) {
        const double waves = (double)((tiles * s + 255) / 256);
        double c = waves * ((double)nkb / s * 0.82 + 2.5);
        if (s > 1) c += 3.1 + 0.09 * s * tiles;
        return c;
    };
    int best = 1;
    const double c1 = cost(1);
    double bc = c1;
    for (int s = 2; s <= 16 && s <= nkb / 2; ++s) {
        const double c = cost(s);
        if (c < bc) { bc = c; best = s; }
    }
    return bc < 0.92 * c1 ? best : 1;
}

// The counters, then the largest of the three tile shapes' partials (one f32
// per output of every tile and split).
size_t gemm_bf6_splitk_workspace(int M, int N, int nsplit) {
    auto part_bytes = [&](int bm, int bn) {
        return (size_t)nsplit * ((M + bm - 1) / bm) * ((N + bn - 1) / bn) * (size_t)bm * bn * sizeof(float);
    };
    const size_t full = part_bytes(B6_BM, B6_BN), q = part_bytes(128, 128), w = part_bytes(128, 192);
    const size_t most = full > q ? (full > w ? full : w) : (q > w ? q : w);
    return nsplit <= 1 ? 0 : kSplitCounterBytes + most;
}

}  // namespace convrot
