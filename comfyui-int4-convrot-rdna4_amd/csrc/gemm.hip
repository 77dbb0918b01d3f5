// W4A4 GEMM with int32 accumulation and a fused dequant epilogue (gfx950).
//
//   acc[m, n] = sum_k qx[m, k] * qw[n, k]          (signed nibbles, exact int32)
//   out[m, n] = epilogue(acc, xs[m], ws[n], bias[n])
//
// Inputs are the reference's packed layout (_int4/_codec.py:19-25): row-major
// int8 [rows, K/2], element 2j in the low nibble of byte j, element 2j+1 in
// the high nibble.  Semantics follow _int4/eager.py:154-169 (int4_linear).
//
// CDNA4 has no int4 matrix instruction, so nibbles become int8 operands of
// v_mfma_i32_32x32x32_i8.  The unpack needs no sign extension: for a packed
// dword w, (w & 0xF0F0F0F0) holds 16 * q(odd k) in every byte and
// ((w << 4) & 0xF0F0F0F0) holds 16 * q(even k), both exact signed int8
// (16 * -8 = -128).  The MFMA therefore accumulates 256 * acc, which stays
// below 2^31 for K < 131072, and an arithmetic shift by 8 recovers acc.  The
// k order inside one MFMA does not matter as long as A and B use the same
// permutation, which they do (same loads, same unpack).
//
// W8A8 (the reference's int8 tier, _int4/int8_eager.py): with I8 the operands
// are plain int8 [rows, K] (_int4/int8_eager.py:31-47 storage) and feed the
// same MFMA unchanged, 64 k per 64-byte LDS row block, accumulating acc itself
// (|acc| <= 127^2 K < 2^31 for K < 133000).
//
// Tiling: a 512-lane workgroup computes a 256 x 256 tile; its 8 waves form a
// 2 (M) x 4 (N) grid of 128 x 64 wave tiles (4 x 2 MFMA 32x32 tiles).  Packed
// nibbles are staged through LDS in 128-k blocks (64 bytes per row, rows
// padded to 80 bytes so every 8-lane phase of a ds_read_b128 hits distinct
// banks), double-buffered, one barrier per block.

#include "gemm_common.h"

namespace convrot {

constexpr int TBM = 256, TBN = 256;  // workgroup tile
constexpr int TBK = 128;             // k values per LDS block
constexpr int ROWB = TBK / 2;        // packed bytes per row per block (64)
constexpr int LDS_STRIDE = 80;       // padded row stride in bytes
constexpr int NTHR = 512;
constexpr int WTM = 128, WTN = 64;   // wave tile
constexpr int FM = WTM / 32, FN = WTN / 32;

__device__ __forceinline__ void unpack16(uint4 p, v4i& lo_step, v4i& hi_step) {
    // 32 nibbles -> two MFMA operands of 16 int8 each (16 * q)
    lo_step = (v4i){(int)((p.x << 4) & 0xF0F0F0F0u), (int)(p.x & 0xF0F0F0F0u),
                    (int)((p.y << 4) & 0xF0F0F0F0u), (int)(p.y & 0xF0F0F0F0u)};
    hi_step = (v4i){(int)((p.z << 4) & 0xF0F0F0F0u), (int)(p.z & 0xF0F0F0F0u),
                    (int)((p.w << 4) & 0xF0F0F0F0u), (int)(p.w & 0xF0F0F0F0u)};
}

template <int EPI, bool LORA, bool I8>
__global__ __launch_bounds__(NTHR) void w4a4_gemm_kernel(
        const int8_t* __restrict__ Xp, const int8_t* __restrict__ Wp,
        const float* __restrict__ xs, const float* __restrict__ ws, const float* __restrict__ bias,
        void* __restrict__ out, int M, int N, int K, LoraArgs lora) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[2][(TBM + TBN) * LDS_STRIDE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 2;            // 0..1
    const int wn = wave & 3;             // 0..3
    const int m0 = blockIdx.y * TBM;
    const int n0 = blockIdx.x * TBN;
    const int Kb = I8 ? K : K / 2;       // operand bytes per row
    // k range of this workgroup: split blockIdx.z of gridDim.z (1 unless split-K)
    const int nkb_all = (Kb + ROWB - 1) / ROWB;
    const int kb_begin = (int)((long long)blockIdx.z * nkb_all / gridDim.z);
    const int kb_end = (int)((long long)(blockIdx.z + 1) * nkb_all / gridDim.z);

    // global -> LDS staging: (TBM + TBN) rows x 4 chunks of 16 B = 2048 chunks, 4 per lane
    uint4 stage[4];
    auto gload = [&](int kb) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int id = tid + j * NTHR;          // 0..2047
            const int r = id >> 2;                  // 0..511 (A rows then B rows)
            const int c16 = id & 3;
            const int kbyte = kb * ROWB + c16 * 16;
            uint4 v = make_uint4(0u, 0u, 0u, 0u);
            if (r < TBM) {
                const int gm = m0 + r;
                if (gm < M && kbyte < Kb)
                    v = *reinterpret_cast<const uint4*>(Xp + (size_t)gm * Kb + kbyte);
            } else {
                const int gn = n0 + (r - TBM);
                if (gn < N && kbyte < Kb)
                    v = *reinterpret_cast<const uint4*>(Wp + (size_t)gn * Kb + kbyte);
            }
            stage[j] = v;
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int id = tid + j * NTHR;
            const int r = id >> 2;
            const int c16 = id & 3;
            *reinterpret_cast<uint4*>(&lds[buf][r * LDS_STRIDE + c16 * 16]) = stage[j];
        }
    };

    v16i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = (v16i){0};

    gload(kb_begin);
    lstore(0);
    __syncthreads();

    const int frow = lane & 31;          // fragment row within a 32-row tile
    const int fhalf = lane >> 5;         // which 16-byte half of a 32-byte k slice

    for (int kb = kb_begin; kb < kb_end; ++kb) {
        const int buf = (kb - kb_begin) & 1;
        if (kb + 1 < kb_end) gload(kb + 1);
        const uint8_t* la = &lds[buf][0];
        const uint8_t* lb = &lds[buf][TBM * LDS_STRIDE];
#pragma unroll
        for (int s2 = 0; s2 < 2 && I8; ++s2) {      // W8A8: two 32-k slices per block, bytes used as they are
            const int koff = s2 * 32 + fhalf * 16;
            v4i a[FM], b[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i)
                a[i] = *reinterpret_cast<const v4i*>(la + (wm * WTM + i * 32 + frow) * LDS_STRIDE + koff);
#pragma unroll
            for (int j = 0; j < FN; ++j)
                b[j] = *reinterpret_cast<const v4i*>(lb + (wn * WTN + j * 32 + frow) * LDS_STRIDE + koff);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
        }
#pragma unroll
        for (int s2 = 0; s2 < 2 && !I8; ++s2) {     // two 64-k slices per block
            const int koff = s2 * 32 + fhalf * 16;
            v4i a_lo[FM], a_hi[FM], b_lo[FN], b_hi[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const uint4 p = *reinterpret_cast<const uint4*>(la + (wm * WTM + i * 32 + frow) * LDS_STRIDE + koff);
                unpack16(p, a_lo[i], a_hi[i]);
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const uint4 p = *reinterpret_cast<const uint4*>(lb + (wn * WTN + j * 32 + frow) * LDS_STRIDE + koff);
                unpack16(p, b_lo[j], b_hi[j]);
            }
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_lo[i], b_lo[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_hi[i], b_hi[j], acc[i][j], 0, 0, 0);
                }
        }
        if (kb + 1 < kb_end) lstore(buf ^ 1);
        __syncthreads();
    }

    epilogue_tiles<EPI, FM, FN, LORA, I8 ? 0 : 8>(acc, xs, ws, bias, out, M, N, m0 + wm * WTM, n0 + wn * WTN, lane, lora);
}

// ---------------------------------------------------------------------------
// Pipelined kernel (K % 128 == 0; W8A8: K % 64 == 0).
//
// 256 x 256 tile per workgroup of 2 x WN waves (default 8 waves of 128 x 64:
// 4 x 2 MFMA 32x32 tiles each, two waves per SIMD so one wave's unpack and
// LDS waits overlap the other's MFMAs).  Operands stream through a
// P_STAGES-deep LDS ring filled by global_load_lds_dwordx4 (no register
// staging): blocks kb+1 .. kb+P_STAGES-1 are in flight while block kb is
// multiplied, one barrier per 128-k block.  LDS rows are 64 bytes with the
// 16-byte chunk index XOR-swizzled (see swz) so fragment reads are
// bank-conflict-free; the swizzle is applied on the global side so each DMA
// instruction still fills 1 KB of LDS linearly.  Rows past M / N load a valid
// row (their outputs are never stored); K needs no tail.  Workgroups are
// renumbered so that each XCD (workgroup id mod 8) gets a contiguous range of
// tiles.
// ---------------------------------------------------------------------------

constexpr int P_BM = 256, P_BN = 256, P_BK = 128;
constexpr int P_ROWB = P_BK / 2;                       // 64 packed bytes per row per block
#ifndef CONVROT_PIPE_WN
#define CONVROT_PIPE_WN 4            // waves along N: 4 -> 8 waves of 128 x 64
#endif
#ifndef CONVROT_PIPE_STAGES
#define CONVROT_PIPE_STAGES 4        // LDS ring depth (blocks of 128 k)
#endif
constexpr int P_STAGES = CONVROT_PIPE_STAGES;
constexpr int P_STAGE_BYTES = (P_BM + P_BN) * P_ROWB;  // 32 KB
constexpr int P_LDS_BYTES = P_STAGES * P_STAGE_BYTES + EPI_SCALE_FLOATS * 4;

// TM (W8A8 only): operands in the I8T layout (b6t_layout.h) instead of
// row-major: each stage half is one contiguous 16 KB chunk.
template <int EPI, int WN, bool LORA, bool I8, bool TM = false>
__global__ __launch_bounds__(128 * WN) void w4a4_gemm_pipe_kernel(
        const int8_t* __restrict__ Xp, const int8_t* __restrict__ Wp,
        const float* __restrict__ xs, const float* __restrict__ ws, const float* __restrict__ bias,
        void* __restrict__ out, int M, int N, int K, LoraArgs lora, int gm) {
    extern __shared__ __attribute__((aligned(16))) uint8_t plds[];

    constexpr int P_THREADS = 128 * WN;                 // 2 x WN waves
    constexpr int P_LOADS = P_STAGE_BYTES / 16 / P_THREADS;
    constexpr int WTN_P = P_BN / WN;                    // wave tile: 128 x WTN_P
    constexpr int PFN = WTN_P / 32;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    int tm, tn;
    tile_of_block(blockIdx.x, (M + P_BM - 1) / P_BM, (N + P_BN - 1) / P_BN, gm, tm, tn);
    const int m0 = tm * P_BM;
    const int n0 = tn * P_BN;
    const int Kb = I8 ? K : K / 2;                      // operand bytes per row
    const int nkb_all = Kb / P_ROWB;
    // k range of this workgroup: split blockIdx.y of gridDim.y (1 unless split-K);
    // every split holds at least one block (the launch keeps gridDim.y <= nkb_all)
    const int kb_begin = (int)((long long)blockIdx.y * nkb_all / gridDim.y);
    const int nkb = (int)((long long)(blockIdx.y + 1) * nkb_all / gridDim.y) - kb_begin;
    float* sc = reinterpret_cast<float*>(plds + P_STAGES * P_STAGE_BYTES);
    stage_scales(sc, xs, ws, bias, M, N, m0, n0, tid, 128 * WN);   // visible after the loop's first barrier

    static_assert(!TM || (I8 && WN == 4), "I8T operands: W8A8, 8 waves");
    // DMA source rows / chunks for this lane's P_LOADS instructions (fixed per tile)
    const int8_t* src[P_LOADS];
    if constexpr (TM) {   // waves 0..3 copy the A chunk, waves 4..7 the B chunk, 1 KB per instruction
        const int8_t* base = (wave < 4 ? Xp + (size_t)tm * nkb_all * I8T_CHUNK : Wp + (size_t)tn * nkb_all * I8T_CHUNK)
                             + (size_t)kb_begin * I8T_CHUNK;
#pragma unroll
        for (int j = 0; j < P_LOADS; ++j) src[j] = base + ((wave & 3) * P_LOADS + j) * 1024 + lane * 16;
    } else
#pragma unroll
    for (int j = 0; j < P_LOADS; ++j) {
        const int slot = (wave * P_LOADS + j) * 64 + lane;   // 16-byte slot of the stage
        const int r = slot >> 2;                             // 0..511: A rows then B rows
        const int c = swz(r, slot & 3);                      // logical chunk stored at this slot
        if (r < P_BM) {
            const int gm = min(m0 + r, M - 1);
            src[j] = Xp + (size_t)gm * Kb + (size_t)kb_begin * P_ROWB + c * 16;
        } else {
            const int gn = min(n0 + (r - P_BM), N - 1);
            src[j] = Wp + (size_t)gn * Kb + (size_t)kb_begin * P_ROWB + c * 16;
        }
    }
    const uint32_t lds_base = (uint32_t)(uintptr_t)plds;

    v16i acc[4][PFN];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < PFN; ++j) acc[i][j] = (v16i){0};

    const int frow = lane & 31;
    const int fhalf = lane >> 5;

    if constexpr (I8) {
        // W8A8: hand-scheduled loop, two phases per 64-k block kb (k steps of 32).
        // Phase A: the 8 MFMAs of k step 0 (fragments read in the previous phase
        // B), the first five followed by the fragment reads of k step 1, slots 2
        // and 5 by one DMA instruction each of the second half of block
        // kb+P_STAGES-2 (into the stage of block kb-2).  Then wait until this
        // wave's copies of block kb+1 have landed and pass the barrier.  Phase B:
        // the 8 MFMAs of k step 1, followed by the fragment reads of k step 0 of
        // block kb+1 and, in slots 2 and 5, the first half of block kb+P_STAGES-1
        // (into the stage of block kb-1, whose reads were all consumed before this
        // barrier).  Copies spread over both phases hold back fewer consecutive
        // MFMAs than four in a row (3.5-9% on the Flux block shapes).  Reads go in
        // the order the MFMAs consume them; copies past the end repeat the last
        // block into a free stage, so the loop has no branch.  sched_barrier(0)
        // pins every slot.
        static_assert(P_LOADS == 4 && PFN == 2, "W8A8 schedule");
        typedef unsigned v4u __attribute__((ext_vector_type(4)));
        struct Frags { v4u fa[4], fb[2]; };
        auto read_one = [&](int kb, int s2, int r, Frags& f) __attribute__((always_inline)) {
            const uint8_t* la = plds + (kb % P_STAGES) * P_STAGE_BYTES;
            const int c = 2 * s2 + fhalf;
            if (r < 4) {
                const int row = wm * 128 + r * 32 + frow;
                f.fa[r] = *reinterpret_cast<const v4u*>(la + row * P_ROWB + swz(row, c) * 16);
            } else {
                const int row = wn * WTN_P + (r - 4) * 32 + frow;
                f.fb[r - 4] = *reinterpret_cast<const v4u*>(la + P_BM * P_ROWB + row * P_ROWB + swz(row, c) * 16);
            }
        };
        auto mfma_one = [&](const Frags& f, int t) __attribute__((always_inline)) {
            const int i = t >> 1, j = t & 1;
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(v4i, f.fb[j]),
                                                             __builtin_bit_cast(v4i, f.fa[i]), acc[i][j], 0, 0, 0);
        };
        // reads after MFMA slot t: fb0 fa0 | fb1 | fa1 | fa2 | fa3
        auto reads_after = [&](int t, int kb, int s2, Frags& f) __attribute__((always_inline)) {
            if (t == 0) { read_one(kb, s2, 4, f); read_one(kb, s2, 0, f); }
            if (t == 1) read_one(kb, s2, 5, f);
            if (t == 2) read_one(kb, s2, 1, f);
            if (t == 3) read_one(kb, s2, 2, f);
            if (t == 4) read_one(kb, s2, 3, f);
        };
        auto dma_one = [&](int kb, int j) __attribute__((always_inline)) {
            const uint32_t st = lds_base + (kb % P_STAGES) * P_STAGE_BYTES + wave * P_LOADS * 1024;
            dma16(st + j * 1024, src[j] + (size_t)min(kb, nkb - 1) * (TM ? I8T_CHUNK : P_ROWB));
        };
        Frags F0, F1;
#pragma unroll
        for (int p = 0; p < P_STAGES - 2; ++p)
#pragma unroll
            for (int j = 0; j < P_LOADS; ++j) dma_one(p, j);
#pragma unroll
        for (int j = 0; j < P_LOADS / 2; ++j) dma_one(P_STAGES - 2, j);   // the rest in phase A of block 0
        __builtin_amdgcn_s_waitcnt(vmcnt_imm((P_STAGES - 3) * P_LOADS + P_LOADS / 2));   // block 0 landed
        __syncthreads();
#pragma unroll
        for (int r = 0; r < 6; ++r) read_one(0, 0, r, F0);
        for (int kb = 0; kb < nkb; ++kb) {
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                mfma_one(F0, t);
                __builtin_amdgcn_sched_barrier(0);
                if (t == 2 || t == 5) dma_one(kb + P_STAGES - 2, P_LOADS / 2 + (t == 2 ? 0 : 1));
                reads_after(t, kb, 1, F1);
                __builtin_amdgcn_sched_barrier(0);
            }
            __builtin_amdgcn_s_waitcnt(vmcnt_imm((P_STAGES - 3) * P_LOADS));   // block kb+1 landed
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                mfma_one(F1, t);
                __builtin_amdgcn_sched_barrier(0);
                if (t == 2 || t == 5) dma_one(kb + P_STAGES - 1, t == 2 ? 0 : 1);
                reads_after(t, kb + 1, 0, F0);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));            // the copies past the end have landed
    } else {
        // Packed int4: the W8A8 loop with the nibble unpack.  A 16-byte fragment (32
        // nibbles of one row and k step) becomes two MFMA operands of 16 int8 values
        // 16 q: its first 8 bytes the "lo" operand, its last 8 the "hi" one (both sides
        // unpack alike, so the k order inside a step is immaterial; the epilogue drops
        // the factor 256).  Two phases per 128-k block kb, one per k step of 64: the 8
        // lo MFMAs, then the 8 hi ones.  In the 16 slots of a phase: the hi operands of
        // this step are unpacked (slots 0..5, consumed from slot 8), the fragments of
        // the next step are read (3..8), one DMA instruction goes out in slots 6 and 9
        // (phase A: the second half of block kb+P_STAGES-2; phase B: the first half of
        // block kb+P_STAGES-1), and the lo operands of the next step are unpacked
        // (10..15, after this step's lo MFMAs).  Fragments are read and unpacked in
        // the order the MFMAs consume them: B0, B1, A0..A3.
        static_assert(P_LOADS == 4 && PFN == 2, "int4 schedule");
        typedef unsigned v4u __attribute__((ext_vector_type(4)));
        struct Frags { v4u fa[4], fb[2]; };
        struct Ops { v4i alo[4], ahi[4], blo[2], bhi[2]; };
        constexpr int kOrder[6] = {4, 5, 0, 1, 2, 3};    // fragment r: A row tile r < 4, else B tile r - 4
        auto read_one = [&](int kb, int s2, int r, Frags& f) __attribute__((always_inline)) {
            const uint8_t* la = plds + (kb % P_STAGES) * P_STAGE_BYTES;
            const int c = 2 * s2 + fhalf;
            if (r < 4) {
                const int row = wm * 128 + r * 32 + frow;
                f.fa[r] = *reinterpret_cast<const v4u*>(la + row * P_ROWB + swz(row, c) * 16);
            } else {
                const int row = wn * WTN_P + (r - 4) * 32 + frow;
                f.fb[r - 4] = *reinterpret_cast<const v4u*>(la + P_BM * P_ROWB + row * P_ROWB + swz(row, c) * 16);
            }
        };
        // 8 packed bytes (16 nibbles) -> 16 int8 values 16 q (as unpack16)
        auto unpack8 = [](unsigned x, unsigned y) __attribute__((always_inline)) {
            return (v4i){(int)((x << 4) & 0xF0F0F0F0u), (int)(x & 0xF0F0F0F0u),
                         (int)((y << 4) & 0xF0F0F0F0u), (int)(y & 0xF0F0F0F0u)};
        };
        auto unpack_lo = [&](const Frags& f, int r, Ops& o) __attribute__((always_inline)) {
            if (r < 4) o.alo[r] = unpack8(f.fa[r].x, f.fa[r].y);
            else o.blo[r - 4] = unpack8(f.fb[r - 4].x, f.fb[r - 4].y);
        };
        auto unpack_hi = [&](const Frags& f, int r, Ops& o) __attribute__((always_inline)) {
            if (r < 4) o.ahi[r] = unpack8(f.fa[r].z, f.fa[r].w);
            else o.bhi[r - 4] = unpack8(f.fb[r - 4].z, f.fb[r - 4].w);
        };
        // MFMA t (0..15) of a k step: lo operands for t < 8, hi for t >= 8; A tile (t & 7) / 2, B tile t % 2
        auto mfma_one = [&](const Ops& o, int t) __attribute__((always_inline)) {
            const int i = (t & 7) >> 1, j = t & 1;
            if (t < 8) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.blo[j], o.alo[i], acc[i][j], 0, 0, 0);
            else acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.bhi[j], o.ahi[i], acc[i][j], 0, 0, 0);
        };
        auto dma_one = [&](int kb, int j) __attribute__((always_inline)) {
            const uint32_t st = lds_base + (kb % P_STAGES) * P_STAGE_BYTES + wave * P_LOADS * 1024;
            dma16(st + j * 1024, src[j] + (size_t)min(kb, nkb - 1) * P_ROWB);
        };
        Frags F0, F1;
        Ops O;
#pragma unroll
        for (int p = 0; p < P_STAGES - 2; ++p)
#pragma unroll
            for (int j = 0; j < P_LOADS; ++j) dma_one(p, j);
#pragma unroll
        for (int j = 0; j < P_LOADS / 2; ++j) dma_one(P_STAGES - 2, j);   // the rest in phase A of block 0
        __builtin_amdgcn_s_waitcnt(vmcnt_imm((P_STAGES - 3) * P_LOADS + P_LOADS / 2));   // block 0 landed
        __syncthreads();
#pragma unroll
        for (int r = 0; r < 6; ++r) read_one(0, 0, kOrder[r], F0);
#pragma unroll
        for (int r = 0; r < 6; ++r) unpack_lo(F0, kOrder[r], O);
        for (int kb = 0; kb < nkb; ++kb) {
#pragma unroll
            for (int t = 0; t < 16; ++t) {            // phase A: k step 0 of block kb
                mfma_one(O, t);
                __builtin_amdgcn_sched_barrier(0);
                if (t < 6) unpack_hi(F0, kOrder[t], O);
                if (t >= 3 && t < 9) read_one(kb, 1, kOrder[t - 3], F1);
                if (t == 6 || t == 9) dma_one(kb + P_STAGES - 2, P_LOADS / 2 + (t == 6 ? 0 : 1));
                if (t >= 10) unpack_lo(F1, kOrder[t - 10], O);
                __builtin_amdgcn_sched_barrier(0);
            }
            __builtin_amdgcn_s_waitcnt(vmcnt_imm((P_STAGES - 3) * P_LOADS));   // block kb+1 landed
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < 16; ++t) {            // phase B: k step 1 of block kb
                mfma_one(O, t);
                __builtin_amdgcn_sched_barrier(0);
                if (t < 6) unpack_hi(F1, kOrder[t], O);
                if (t >= 3 && t < 9) read_one(kb + 1, 0, kOrder[t - 3], F0);
                if (t == 6 || t == 9) dma_one(kb + P_STAGES - 1, t == 6 ? 0 : 1);
                if (t >= 10) unpack_lo(F0, kOrder[t - 10], O);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));            // the copies past the end have landed
    }

    __syncthreads();                                     // every wave is done with the stages
    constexpr int SCR = P_STAGES * P_STAGE_BYTES / (2 * WN);
    epilogue_lds<EPI, 4, PFN, (LORA ? -1 : 0), SCR, I8 ? 0 : 8>(acc, sc, out, M, N, m0, n0, m0 + wm * 128,
                                         n0 + wn * WTN_P, lane, lora, plds + wave * SCR);
}

// nsplit > 1 (EPI_ATOMIC_ACC only): the k blocks are split over nsplit
// workgroups per tile, at most one split per k block.
template <int EPI, bool LORA, bool I8 = false, bool TM = false>
static hipError_t launch_epi(const int8_t* Xp, const int8_t* Wp, const float* xs, const float* ws,
                             const float* bias, void* out, int M, int N, int K, const LoraArgs& la,
                             hipStream_t st, int nsplit = 1) {
    const int Kb = I8 ? K : K / 2;
    if (TM || Kb % P_ROWB == 0) {
        constexpr int WN = CONVROT_PIPE_WN;
        const int ntiles = ((M + P_BM - 1) / P_BM) * ((N + P_BN - 1) / P_BN);
        static std::atomic<bool> attr_set[kMaxDev];
        int dev = 0;
        hipError_t e = current_device(&dev);
        if (e != hipSuccess) return e;
        e = lds_limit_once(attr_set, dev,
                           reinterpret_cast<const void*>(&w4a4_gemm_pipe_kernel<EPI, WN, LORA, I8, TM>), P_LDS_BYTES);
        if (e != hipSuccess) return e;
        const int splits = min(nsplit, Kb / P_ROWB);
        hipLaunchKernelGGL((w4a4_gemm_pipe_kernel<EPI, WN, LORA, I8, TM>), dim3(ntiles, splits), dim3(128 * WN),
                           P_LDS_BYTES, st, Xp, Wp, xs, ws, bias, out, M, N, K, la,
                           tile_group_rows((M + P_BM - 1) / P_BM));
    } else if constexpr (!TM) {
        const int splits = min(nsplit, (Kb + ROWB - 1) / ROWB);
        dim3 grid((N + TBN - 1) / TBN, (M + TBM - 1) / TBM, splits), block(NTHR);
        hipLaunchKernelGGL((w4a4_gemm_kernel<EPI, LORA, I8>), grid, block, 0, st, Xp, Wp, xs, ws, bias, out, M, N, K, la);
    }
    return hipGetLastError();
}

hipError_t gemm_launch(const int8_t* Xp, const int8_t* Wp, const float* xs, const float* ws,
                       const float* bias, void* out, int M, int N, int K, int epi, hipStream_t st) {
    if (M == 0 || N == 0) return hipSuccess;
    const LoraArgs none{nullptr, nullptr, 0, 0.0f};
    switch (epi) {
        case EPI_F32: return launch_epi<EPI_F32, false>(Xp, Wp, xs, ws, bias, out, M, N, K, none, st);
        case EPI_BF16: return launch_epi<EPI_BF16, false>(Xp, Wp, xs, ws, bias, out, M, N, K, none, st);
        case EPI_BF16_EAGER: return launch_epi<EPI_BF16_EAGER, false>(Xp, Wp, xs, ws, bias, out, M, N, K, none, st);
        case EPI_ACC: return launch_epi<EPI_ACC, false>(Xp, Wp, xs, ws, bias, out, M, N, K, none, st);
        default: return hipErrorInvalidValue;
    }
}

// W8A8: plain int8 operands X [M, K], W [N, K] (K % 16 == 0) on the same
// kernels (64 operand bytes per row and LDS block: 64 k), exact int32 acc.
hipError_t gemm_i8_launch(const int8_t* X, const int8_t* W, const float* xs, const float* ws,
                          const float* bias, void* out, int M, int N, int K, int epi, hipStream_t st) {
    if (M == 0 || N == 0) return hipSuccess;
    const LoraArgs none{nullptr, nullptr, 0, 0.0f};
    switch (epi) {
        case EPI_F32: return launch_epi<EPI_F32, false, true>(X, W, xs, ws, bias, out, M, N, K, none, st);
        case EPI_BF16: return launch_epi<EPI_BF16, false, true>(X, W, xs, ws, bias, out, M, N, K, none, st);
        case EPI_ACC: return launch_epi<EPI_ACC, false, true>(X, W, xs, ws, bias, out, M, N, K, none, st);
        default: return hipErrorInvalidValue;
    }
}

// W8A8 GEMM on I8T operands (K % 64 == 0; rows of A and W padded to 256)
hipError_t gemm_i8t_launch(const int8_t* X, const int8_t* W, const float* xs, const float* ws,
                           const float* bias, void* out, int M, int N, int K, int epi, hipStream_t st) {
    if (M == 0 || N == 0) return hipSuccess;
    if (K % 64 != 0) return hipErrorInvalidValue;
    const LoraArgs none{nullptr, nullptr, 0, 0.0f};
    switch (epi) {
        case EPI_F32: return launch_epi<EPI_F32, false, true, true>(X, W, xs, ws, bias, out, M, N, K, none, st);
        case EPI_BF16: return launch_epi<EPI_BF16, false, true, true>(X, W, xs, ws, bias, out, M, N, K, none, st);
        case EPI_ACC: return launch_epi<EPI_ACC, false, true, true>(X, W, xs, ws, bias, out, M, N, K, none, st);
        default: return hipErrorInvalidValue;
    }
}

// row-major int8 [rows, K] -> I8T (K % 64 == 0); one thread per 16-byte piece
// of the padded matrix, consecutive threads on the pieces of consecutive rows
__global__ __launch_bounds__(256) void int8_to_i8t_kernel(const int8_t* __restrict__ src, int8_t* __restrict__ dst,
                                                          int rows, int K) {
    const int nkb = K / 64;
    const long long id = (long long)blockIdx.x * 256 + threadIdx.x;
    const int tiles = (rows + 255) / 256;
    if (id >= (long long)tiles * nkb * 1024) return;
    const int c = (int)(id & 3), r = (int)((id >> 2) & 255);
    const long long tk = id >> 10;                       // tile * nkb + kb
    const int tile = (int)(tk / nkb), kb = (int)(tk % nkb);
    const int row = tile * 256 + r;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (row < rows) v = *reinterpret_cast<const uint4*>(src + (size_t)row * K + kb * 64 + c * 16);
    *reinterpret_cast<uint4*>(dst + (size_t)tk * I8T_CHUNK + i8t_off(r, c)) = v;
}

hipError_t int8_to_i8t_launch(const void* src, void* dst, int rows, int K, hipStream_t st) {
    if (rows < 0 || K <= 0 || K % 64 != 0) return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    const long long threads = (long long)((rows + 255) / 256) * (K / 64) * 1024;
    hipLaunchKernelGGL(int8_to_i8t_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                       reinterpret_cast<const int8_t*>(src), reinterpret_cast<int8_t*>(dst), rows, K);
    return hipGetLastError();
}

// I8T -> row-major int8 [rows, K] (the inverse of int8_to_i8t_kernel on the
// first `rows` rows): one thread per (row, 16-byte piece).
__global__ __launch_bounds__(256) void i8t_to_int8_kernel(const int8_t* __restrict__ src, int8_t* __restrict__ dst,
                                                          int rows, int K) {
    const int np = K / 16;
    const long long id = (long long)blockIdx.x * 256 + threadIdx.x;
    if (id >= (long long)rows * np) return;
    const int row = (int)(id / np), pc = (int)(id % np);
    const int kb = pc >> 2, c = pc & 3;
    const int8_t* chunk = src + ((size_t)(row >> 8) * (K / 64) + kb) * I8T_CHUNK;
    *reinterpret_cast<uint4*>(dst + (size_t)row * K + (size_t)pc * 16) =
        *reinterpret_cast<const uint4*>(chunk + i8t_off(row & 255, c));
}

hipError_t i8t_to_int8_launch(const void* src, void* dst, int rows, int K, hipStream_t st) {
    if (rows < 0 || K <= 0 || K % 64 != 0) return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    const long long n = (long long)rows * (K / 16);
    hipLaunchKernelGGL(i8t_to_int8_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       reinterpret_cast<const int8_t*>(src), reinterpret_cast<int8_t*>(dst), rows, K);
    return hipGetLastError();
}

// Split-K finalize: accum holds the exact int32 accumulators (the sum of every
// split's partial); each becomes fl32(fl32(float(acc) * xs[m]) * ws[n]) in
// place, the unsplit f32 epilogue without its bias term.
__global__ __launch_bounds__(256) void splitk_finalize_kernel(float* __restrict__ accum, const float* __restrict__ xs,
                                                              const float* __restrict__ ws, int M, int N) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long long)M * N) return;
    const int m = (int)(i / N), n = (int)(i - (long long)m * N);
    const int acc = __float_as_int(accum[i]);
    accum[i] = __fmul_rn(__fmul_rn((float)acc, xs[m]), ws[n]);
}

// The reference's split-K contract (_int4/int4_gemm.hip:259-330, 634-645):
// accum f32 [M, N] arrives zeroed; afterwards it holds the scaled product
// without bias.  Here each split adds its exact integer partial (the int32
// view of the zeroed buffer starts at 0), and the finalize scales the total
// once, so the result is the unsplit f32 epilogue bit for bit for every
// nsplit (the reference adds separately rounded float partials).
hipError_t gemm_splitk_launch(const int8_t* Xp, const int8_t* Wp, const float* xs, const float* ws, float* accum,
                              int M, int N, int K, int nsplit, hipStream_t st) {
    if (M == 0 || N == 0) return hipSuccess;
    const LoraArgs none{nullptr, nullptr, 0, 0.0f};
    hipError_t e = launch_epi<EPI_ATOMIC_ACC, false>(Xp, Wp, nullptr, nullptr, nullptr, accum, M, N, K, none, st,
                                                     nsplit);
    if (e != hipSuccess) return e;
    const long long n = (long long)M * N;
    hipLaunchKernelGGL(splitk_finalize_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, accum, xs, ws, M,
                       N);
    return hipGetLastError();
}

hipError_t gemm_lora_launch(const int8_t* Xp, const int8_t* Wp, const float* xs, const float* ws,
                            const float* bias, const void* t, const void* U, int R, float scale, void* out,
                            int M, int N, int K, int epi, hipStream_t st) {
    if (M == 0 || N == 0) return hipSuccess;
    const LoraArgs la{reinterpret_cast<const __bf16*>(t), reinterpret_cast<const __bf16*>(U), R, scale};
    switch (epi) {
        case EPI_F32: return launch_epi<EPI_F32, true>(Xp, Wp, xs, ws, bias, out, M, N, K, la, st);
        case EPI_BF16: return launch_epi<EPI_BF16, true>(Xp, Wp, xs, ws, bias, out, M, N, K, la, st);
        case EPI_BF16_EAGER: return launch_epi<EPI_BF16_EAGER, true>(Xp, Wp, xs, ws, bias, out, M, N, K, la, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace convrot
