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
// Tiling: a 512-lane workgroup computes a 256 x 256 tile; its 8 waves form a
// 2 (M) x 4 (N) grid of 128 x 64 wave tiles (4 x 2 MFMA 32x32 tiles).  Packed
// nibbles are staged through LDS in 128-k blocks (64 bytes per row, rows
// padded to 80 bytes so every 8-lane phase of a ds_read_b128 hits distinct
// banks), double-buffered, one barrier per block.

#include "common.h"

namespace convrot {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

enum : int { EPI_F32 = 0, EPI_BF16 = 1, EPI_BF16_EAGER = 2, EPI_ACC = 3 };

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

__device__ __forceinline__ float bf16r(float f) { return round_to_dt<DT_BF16>(f); }

// Optional fused dynamic-LoRA term: out += scale * t[m, :] . U[n, :] (rank R).
struct LoraArgs {
    const __bf16* t;      // [M, R] bf16 (x @ D^T, from lora_down)
    const __bf16* U;      // [N, R] bf16
    int R;                // multiple of 16 (0: no LoRA)
    float scale;
};

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// Epilogue of a wave's FMT x FNT grid of 32x32 accumulator tiles at (row0, col0).
// 32x32 layout: lane l, register r -> col = l % 32, row = 8 (r / 4) + 4 (l / 32) + r % 4.
// The LoRA product uses the same layout (bf16 MFMA over R), issued by the
// whole wave before any per-lane bounds check.
template <int EPI, int FMT, int FNT, bool LORA>
__device__ __forceinline__ void epilogue_tiles(const v16i (&acc)[FMT][FNT], const float* __restrict__ xs,
                                               const float* __restrict__ ws, const float* __restrict__ bias,
                                               void* __restrict__ out, int M, int N, int row0, int col0,
                                               int lane, const LoraArgs& la) {
    const int h = lane >> 5;
#pragma unroll
    for (int i = 0; i < FMT; ++i) {
        const int rbase = row0 + i * 32 + 4 * h;
        float xsv[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = rbase + 8 * (r >> 2) + (r & 3);
            xsv[r] = (EPI != EPI_ACC && row < M) ? xs[row] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < FNT; ++j) {
            const int col = col0 + j * 32 + (lane & 31);
            f32x16_t lacc = (f32x16_t){0};
            if constexpr (LORA) {
                const int trow = row0 + i * 32 + (lane & 31);          // MFMA A row of this lane
                for (int rk = 0; rk < la.R; rk += 16) {
                    const int k = rk + 8 * h;
                    const bf16x8_t a = trow < M ? *reinterpret_cast<const bf16x8_t*>(la.t + (size_t)trow * la.R + k)
                                                : (bf16x8_t){0};
                    const bf16x8_t b = col < N ? *reinterpret_cast<const bf16x8_t*>(la.U + (size_t)col * la.R + k)
                                               : (bf16x8_t){0};
                    lacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, lacc, 0, 0, 0);
                }
            }
            if (col >= N) continue;
            float wsc = 0.0f, bv = 0.0f;
            if constexpr (EPI != EPI_ACC) {
                wsc = ws[col];
                if (bias) bv = bias[col];
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = rbase + 8 * (r >> 2) + (r & 3);
                if (row >= M) continue;
                const int a = acc[i][j][r] >> 8;
                const size_t o = (size_t)row * N + col;
                if constexpr (EPI == EPI_ACC) {
                    reinterpret_cast<int32_t*>(out)[o] = a;
                } else if constexpr (EPI == EPI_BF16_EAGER) {
                    float v = bf16r(bf16r((float)a) * bf16r(xsv[r]));
                    v = bf16r(v * bf16r(wsc));
                    if (bias) v = bf16r(v + bf16r(bv));
                    if constexpr (LORA) v = bf16r(v + bf16r(__fmul_rn(la.scale, lacc[r])));
                    reinterpret_cast<uint16_t*>(out)[o] = (uint16_t)f32_to_bf16_bits(v);
                } else {
                    float v = __fmul_rn(__fmul_rn((float)a, xsv[r]), wsc);
                    if (bias) v = __fadd_rn(v, bv);
                    if constexpr (LORA) v = __fadd_rn(v, __fmul_rn(la.scale, lacc[r]));
                    if constexpr (EPI == EPI_F32) reinterpret_cast<float*>(out)[o] = v;
                    else reinterpret_cast<uint16_t*>(out)[o] = (uint16_t)f32_to_bf16_bits(v);
                }
            }
        }
    }
}

template <int EPI, bool LORA>
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
    const int Kb = K / 2;                // packed bytes per row
    const int nkb = (K + TBK - 1) / TBK;

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

    gload(0);
    lstore(0);
    __syncthreads();

    const int frow = lane & 31;          // fragment row within a 32-row tile
    const int fhalf = lane >> 5;         // which 16-byte half of a 32-byte k slice

    for (int kb = 0; kb < nkb; ++kb) {
        const int buf = kb & 1;
        if (kb + 1 < nkb) gload(kb + 1);
        const uint8_t* la = &lds[buf][0];
        const uint8_t* lb = &lds[buf][TBM * LDS_STRIDE];
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {            // two 64-k slices per block
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
        if (kb + 1 < nkb) lstore(buf ^ 1);
        __syncthreads();
    }

    epilogue_tiles<EPI, FM, FN, LORA>(acc, xs, ws, bias, out, M, N, m0 + wm * WTM, n0 + wn * WTN, lane, lora);
}

// ---------------------------------------------------------------------------
// Pipelined kernel (K % 128 == 0).
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

#ifndef CONVROT_SWZ64
#define CONVROT_SWZ64 1
#endif
// chunk swizzle: row r stores its logical chunk c at physical chunk c ^ f(r).
// With 64-byte rows a 16-byte read of chunk c by rows r..r+15 is conflict-free
// when (r & 3, f(r)) takes 16 distinct values (64 banks x 4 B, 16 lanes per
// phase) and when (r & 1, f(r)) takes 8 distinct values over r..r+7 (32 banks,
// 8 lanes per phase); f = (bit1 ^ bit3) | bit2 << 1 satisfies both.
__device__ __forceinline__ int swz(int row, int chunk) {
    if (CONVROT_SWZ64) return chunk ^ ((((row >> 1) ^ (row >> 3)) & 1) | ((row >> 1) & 2));
    return chunk ^ ((row >> 1) & 3);
}

// s_waitcnt immediate that waits until at most n vector-memory operations are
// outstanding (vmcnt split over bits 3:0 and 15:14; expcnt / lgkmcnt not waited)
constexpr int vmcnt_imm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }

template <int EPI, int WN, bool LORA>
__global__ __launch_bounds__(128 * WN) void w4a4_gemm_pipe_kernel(
        const int8_t* __restrict__ Xp, const int8_t* __restrict__ Wp,
        const float* __restrict__ xs, const float* __restrict__ ws, const float* __restrict__ bias,
        void* __restrict__ out, int M, int N, int K, LoraArgs lora) {
    extern __shared__ __attribute__((aligned(16))) uint8_t plds[];

    constexpr int P_THREADS = 128 * WN;                 // 2 x WN waves
    constexpr int P_LOADS = P_STAGE_BYTES / 16 / P_THREADS;
    constexpr int WTN_P = P_BN / WN;                    // wave tile: 128 x WTN_P
    constexpr int PFN = WTN_P / 32;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int tiles_m = (M + P_BM - 1) / P_BM;
    const int ntiles = tiles_m * ((N + P_BN - 1) / P_BN);
    // XCD-aware renumbering: workgroup b runs on XCD b % 8
    int b = blockIdx.x;
    {
        const int per = ntiles / 8, rem = ntiles % 8, x = b % 8, l = b / 8;
        b = x * per + min(x, rem) + l;
    }
    const int m0 = (b % tiles_m) * P_BM;
    const int n0 = (b / tiles_m) * P_BN;
    const int Kb = K / 2;
    const int nkb = K / P_BK;

    // DMA source rows / chunks for this lane's P_LOADS instructions (fixed per tile)
    const int8_t* src[P_LOADS];
#pragma unroll
    for (int j = 0; j < P_LOADS; ++j) {
        const int slot = (wave * P_LOADS + j) * 64 + lane;   // 16-byte slot of the stage
        const int r = slot >> 2;                             // 0..511: A rows then B rows
        const int c = swz(r, slot & 3);                      // logical chunk stored at this slot
        if (r < P_BM) {
            const int gm = min(m0 + r, M - 1);
            src[j] = Xp + (size_t)gm * Kb + c * 16;
        } else {
            const int gn = min(n0 + (r - P_BM), N - 1);
            src[j] = Wp + (size_t)gn * Kb + c * 16;
        }
    }
    // The DMA is issued from inline asm so the compiler does not add its own
    // conservative vmcnt(0) before every LDS read; the explicit waits below
    // (each lane waits for its own loads before the barrier that publishes a
    // stage) are the only synchronisation.  LDS address of lane i = m0 + 16 i.
    const uint32_t lds_base = (uint32_t)(uintptr_t)plds;
    auto issue = [&](int kb) {
        const uint32_t st = lds_base + (kb % P_STAGES) * P_STAGE_BYTES + wave * P_LOADS * 1024;
#pragma unroll
        for (int j = 0; j < P_LOADS; ++j) {
            const uint32_t m0v = __builtin_amdgcn_readfirstlane(st + j * 1024);
            asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
                         :
                         : "s"(m0v), "v"(src[j] + kb * P_ROWB)
                         : "memory", "m0");
        }
    };

    v16i acc[4][PFN];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < PFN; ++j) acc[i][j] = (v16i){0};

    const int frow = lane & 31;
    const int fhalf = lane >> 5;

#pragma unroll
    for (int p = 0; p < P_STAGES - 1; ++p)
        if (p < nkb) issue(p);
    for (int kb = 0; kb < nkb; ++kb) {
        // block kb landed: only the newer blocks' P_LOADS-per-block may stay in flight
        if (kb + 1 < nkb) __builtin_amdgcn_s_waitcnt(vmcnt_imm((P_STAGES - 2) * P_LOADS));
        else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        __syncthreads();
        if (kb + P_STAGES - 1 < nkb) issue(kb + P_STAGES - 1);
        const uint8_t* la = plds + (kb % P_STAGES) * P_STAGE_BYTES;
        const uint8_t* lb = la + P_BM * P_ROWB;
        uint4 fa[2][4], fb[2][PFN];
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            const int c = 2 * s2 + fhalf;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = wm * 128 + i * 32 + frow;
                fa[s2][i] = *reinterpret_cast<const uint4*>(la + r * P_ROWB + swz(r, c) * 16);
            }
#pragma unroll
            for (int j = 0; j < PFN; ++j) {
                const int r = wn * WTN_P + j * 32 + frow;
                fb[s2][j] = *reinterpret_cast<const uint4*>(lb + r * P_ROWB + swz(r, c) * 16);
            }
        }
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            v4i a_lo[4], a_hi[4], b_lo[PFN], b_hi[PFN];
#pragma unroll
            for (int i = 0; i < 4; ++i) unpack16(fa[s2][i], a_lo[i], a_hi[i]);
#pragma unroll
            for (int j = 0; j < PFN; ++j) unpack16(fb[s2][j], b_lo[j], b_hi[j]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < PFN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_lo[i], b_lo[j], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < PFN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_hi[i], b_hi[j], acc[i][j], 0, 0, 0);
        }
    }

    epilogue_tiles<EPI, 4, PFN, LORA>(acc, xs, ws, bias, out, M, N, m0 + wm * 128, n0 + wn * WTN_P, lane, lora);
}

template <int EPI, bool LORA>
static hipError_t launch_epi(const int8_t* Xp, const int8_t* Wp, const float* xs, const float* ws,
                             const float* bias, void* out, int M, int N, int K, const LoraArgs& la,
                             hipStream_t st) {
    if (K % P_BK == 0) {
        constexpr int WN = CONVROT_PIPE_WN;
        const int ntiles = ((M + P_BM - 1) / P_BM) * ((N + P_BN - 1) / P_BN);
        static bool attr_set = false;
        if (!attr_set) {
            hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&w4a4_gemm_pipe_kernel<EPI, WN, LORA>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               P_STAGES * P_STAGE_BYTES);
            if (e != hipSuccess) return e;
            attr_set = true;
        }
        hipLaunchKernelGGL((w4a4_gemm_pipe_kernel<EPI, WN, LORA>), dim3(ntiles), dim3(128 * WN),
                           P_STAGES * P_STAGE_BYTES, st, Xp, Wp, xs, ws, bias, out, M, N, K, la);
    } else {
        dim3 grid((N + TBN - 1) / TBN, (M + TBM - 1) / TBM), block(NTHR);
        hipLaunchKernelGGL((w4a4_gemm_kernel<EPI, LORA>), grid, block, 0, st, Xp, Wp, xs, ws, bias, out, M, N, K, la);
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
