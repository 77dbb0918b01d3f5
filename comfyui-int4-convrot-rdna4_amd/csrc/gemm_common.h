// Pieces shared by the W4A4 GEMM kernels (int8 MFMA on packed nibbles in
// gemm.hip, bf6 MFMA on pre-encoded operands in gemm_bf6.hip): the output
// epilogues (with the optional fused LoRA term), the LDS chunk swizzle, the
// global->LDS DMA issue and the pipeline waits.
#pragma once

#include "b6t_layout.h"
#include "common.h"

namespace convrot {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// EPI_ATOMIC_ACC: the k-split partial of the packed split-K entry point; the
// exact integer accumulator of the workgroup's k range is added atomically
// into an int32 [M, N] buffer (integer sums are exact in any order).
enum : int { EPI_F32 = 0, EPI_BF16 = 1, EPI_BF16_EAGER = 2, EPI_ACC = 3, EPI_ATOMIC_ACC = 4 };

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

// Accumulator of one output: the int4-on-int8-MFMA kernels accumulate 256 * acc
// in int32 (operands are 16 * q: ASH = 8), the W8A8 kernels acc itself (ASH =
// 0; the float conversion of |acc| >= 2^24 rounds to nearest even, as the
// reference's (float)acc does), the bf6 kernels acc exactly in fp32 (integer
// products, |partial sums| < 2^24).
template <int ASH> __device__ __forceinline__ int acc_int(int v) { return v >> ASH; }
template <int ASH> __device__ __forceinline__ int acc_int(float v) { return (int)v; }
template <int ASH> __device__ __forceinline__ float acc_float(int v) { return (float)(v >> ASH); }
template <int ASH> __device__ __forceinline__ float acc_float(float v) { return v; }   // an exact integer already

// Per-tile epilogue scales staged in LDS by the workgroup at kernel start:
// xs of the tile's 256 rows, ws and bias of its 256 columns (0 outside M / N).
// A missing bias is staged as -0.0, which makes the epilogue's bias add an
// exact identity (x + -0 == x for every float, -0 included), so the epilogue
// needs no per-element select.
constexpr int EPI_SCALE_FLOATS = 3 * 256;

// bias_dt: element type of the bias vector (DT_F32, DT_BF16 or DT_F16; the
// Linear keeps its bias in fp16, so the fused path reads it as stored).
__device__ __forceinline__ float load_bias(const void* __restrict__ bias, int bias_dt, int i) {
    if (bias_dt == DT_F16) return f16bits_to_f32(reinterpret_cast<const uint16_t*>(bias)[i]);
    if (bias_dt == DT_BF16) return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(bias)[i] << 16);
    return reinterpret_cast<const float*>(bias)[i];
}

__device__ __forceinline__ void stage_scales(float* sc, const float* __restrict__ xs, const float* __restrict__ ws,
                                             const void* __restrict__ bias, int bias_dt, int M, int N, int m0,
                                             int n0, int tid, int nthreads) {
    for (int i = tid; i < EPI_SCALE_FLOATS; i += nthreads) {
        const int part = i >> 8, k = i & 255;
        float v = 0.0f;
        if (part == 0) { if (xs && m0 + k < M) v = xs[m0 + k]; }
        else if (part == 1) { if (ws && n0 + k < N) v = ws[n0 + k]; }
        else { v = (bias && n0 + k < N) ? load_bias(bias, bias_dt, n0 + k) : -0.0f; }   // x + (-0) == x, -0 included
        sc[i] = v;
    }
}

__device__ __forceinline__ void stage_scales(float* sc, const float* __restrict__ xs, const float* __restrict__ ws,
                                             const float* __restrict__ bias, int M, int N, int m0, int n0,
                                             int tid, int nthreads) {
    stage_scales(sc, xs, ws, static_cast<const void*>(bias), DT_F32, M, N, m0, n0, tid, nthreads);
}

// The same staging in two steps: load() issues the global loads into
// registers at kernel start, ahead of the main loop's first copies, so their
// latency overlaps the copies' instead of preceding them (stage_scales waits
// for each load before its LDS store); store() writes them to LDS after the
// main loop, whose final vmcnt(0) has retired them.  Threads 0..255 (whole
// waves) each load the xs, ws and bias entries of tile row / column k = tid,
// with clamped indices, so that no load is conditional on a lane and none
// waits for another.
struct ScaleRegs {
    float x, w;
    uint32_t b;   // the bias element's bits in its own type
    __device__ __forceinline__ void load(const float* __restrict__ xs, const float* __restrict__ ws,
                                         const void* __restrict__ bias, int bias_dt, int M, int N, int m0, int n0,
                                         int tid) {
        x = 0.0f; w = 0.0f; b = 0u;
        if (tid >= 256) return;
        const int kx = min(m0 + tid, M - 1), kw = min(n0 + tid, N - 1);
        if (xs) x = xs[kx];
        if (ws) w = ws[kw];
        if (bias) b = bias_dt == DT_F32 ? __float_as_uint(reinterpret_cast<const float*>(bias)[kw])
                                        : (uint32_t)reinterpret_cast<const uint16_t*>(bias)[kw];
    }
    // the values stage_scales writes (0 outside M / N, -0 for an absent bias)
    __device__ __forceinline__ void store(float* sc, const void* __restrict__ bias, int bias_dt, int M, int N,
                                          int m0, int n0, int tid) const {
        if (tid >= 256) return;
        sc[tid] = m0 + tid < M ? x : 0.0f;
        sc[256 + tid] = n0 + tid < N ? w : 0.0f;
        float v = -0.0f;
        if (bias && n0 + tid < N)
            v = bias_dt == DT_F16 ? f16bits_to_f32(b) : bias_dt == DT_BF16 ? __uint_as_float(b << 16) : __uint_as_float(b);
        sc[512 + tid] = v;
    }
};

// Epilogue of a wave's FMT x FNT grid of 32x32 accumulator tiles at (row0, col0).
// 32x32 layout: lane l, register r -> col = l % 32, row = 8 (r / 4) + 4 (l / 32) + r % 4.
// The LoRA product uses the same layout (bf16 MFMA over R), issued by the
// whole wave before any per-lane bounds check.
template <int EPI, int FMT, int FNT, bool LORA, int ASH = 8, typename AccV>
__device__ __forceinline__ void epilogue_tiles(const AccV (&acc)[FMT][FNT], const float* __restrict__ xs,
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
            xsv[r] = (EPI != EPI_ACC && EPI != EPI_ATOMIC_ACC && row < M) ? xs[row] : 0.0f;
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
            if constexpr (EPI != EPI_ACC && EPI != EPI_ATOMIC_ACC) {
                wsc = ws[col];
                if (bias) bv = bias[col];
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = rbase + 8 * (r >> 2) + (r & 3);
                if (row >= M) continue;
                const int a = acc_int<ASH>(acc[i][j][r]);
                const size_t o = (size_t)row * N + col;
                if constexpr (EPI == EPI_ACC) {
                    reinterpret_cast<int32_t*>(out)[o] = a;
                } else if constexpr (EPI == EPI_ATOMIC_ACC) {
                    atomicAdd(reinterpret_cast<int32_t*>(out) + o, a);
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

// Epilogue through LDS for kernels that accumulate the TRANSPOSED tile
// (MFMA with the B fragment as first operand): in a 32x32 accumulator lane l,
// register r holds output row l % 32 and column 8 (r / 4) + 4 (l / 32) + r % 4,
// so each lane owns 4 consecutive columns of one row per register quad.  The
// values are computed as in epilogue_tiles, written to the wave's LDS scratch
// in row-major order (one 8- or 16-byte write per quad; rows padded by 16
// bytes), then copied out with one 16-byte store per lane and chunk so each
// store instruction writes whole row segments.  Rows are processed in passes
// of PT row tiles that fit SCR_BYTES.  `scr` must be 16-byte aligned and owned
// by this wave; `sc` holds the workgroup tile's staged scales (stage_scales).
//
// LR selects the LoRA term: 0 none; -1 rank la.R read at run time (one
// dependent t / U load pair per 16 ranks and tile); 1..4 rank 32 * LR known at
// compile time, loaded in batches of 32 ranks (two t and two U fragments) per
// tile.  For rank 32 with a bf16 output the t fragments of all the wave's row
// tiles and the U fragments of its columns are loaded together up front, so
// the wave waits for them once (a row tile's work is too short to hide the
// next tile's load: fetching t one row tile ahead cost ~3 us per 256 x 256
// tile).  The MFMA sequence (16-rank steps in ascending order) is the same in
// every mode, so are the results.
//
// tu_lds (rank 32, bf16 output only): the workgroup tile's t rows tile_m0 ..
// +255 and U rows tile_n0 .. +255 staged in LDS (64 bytes per row, U at
// +16384), read there instead of from global memory.
template <int EPI, int FMT, int FNT, int LR, int SCR_BYTES, int ASH = 8, bool HOIST = false, typename AccV>
__device__ __forceinline__ void epilogue_lds(const AccV (&acc)[FMT][FNT], const float* sc,
                                             void* __restrict__ out, int M, int N, int tile_m0, int tile_n0,
                                             int row0, int col0, int lane, const LoraArgs& la, uint8_t* scr,
                                             const uint8_t* tu_lds = nullptr) {
    constexpr bool LORA = LR != 0;
    constexpr bool PRE = LR == 1 && (EPI == EPI_BF16 || EPI == EPI_BF16_EAGER);
    constexpr int ES = (EPI == EPI_BF16 || EPI == EPI_BF16_EAGER) ? 2 : 4;
    constexpr int RB = FNT * 32 * ES;                // bytes of one wave-tile row
    constexpr int RS = RB + 16;                      // padded LDS row stride
    // One 32-row tile per staging pass: the stores of a pass drain while the next
    // pass computes.  Staging all of a wave's rows at once (one pass of compute,
    // then one of stores) measured 2.3% slower over the four Flux linears at M =
    // 4608 and 4.8% at 4096 x 3072 -> 3072 (interleaved A/B, same bits); equal
    // for the 128 x 128 kernel.
    constexpr int PT = 1;
    static_assert(SCR_BYTES >= 32 * RS, "scratch too small for one row tile");
    constexpr int CW = RB / 16;                      // 16-byte chunks per row
    // the store pass maps the 64 lanes onto whole rows of 16-byte chunks
    static_assert(64 % CW == 0, "a wave's lanes cover whole rows of the staged tile (FNT 1, 2 or 4)");
    constexpr int EPC = 16 / ES;                     // elements per chunk
    const int h = lane >> 5;
    const int l32 = lane & 31;
    const bool vec = ((size_t)N * ES) % 16 == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
    // compile-time rank: fragments of 16-rank steps s0, s0 + 1 of row tile i (t) / column tile j (U)
    constexpr int RK = LR > 0 ? 32 * LR : 32;
    auto load_t2 = [&](int i, int s0, bf16x8_t (&dst)[2]) {
        const int trow = row0 + i * 32 + l32;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int k = 16 * (s0 + s) + 8 * h;
            if (PRE && tu_lds != nullptr)
                dst[s] = trow < M ? *reinterpret_cast<const bf16x8_t*>(tu_lds + (trow - tile_m0) * 64 + 2 * k)
                                  : (bf16x8_t){0};
            else
                dst[s] = trow < M ? *reinterpret_cast<const bf16x8_t*>(la.t + (size_t)trow * RK + k) : (bf16x8_t){0};
        }
    };
    auto load_u2 = [&](int j, int s0, bf16x8_t (&dst)[2]) {
        const int ucol = col0 + j * 32 + l32;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int k = 16 * (s0 + s) + 8 * h;
            if (PRE && tu_lds != nullptr)
                dst[s] = ucol < N ? *reinterpret_cast<const bf16x8_t*>(tu_lds + 16384 + (ucol - tile_n0) * 64 + 2 * k)
                                  : (bf16x8_t){0};
            else
                dst[s] = ucol < N ? *reinterpret_cast<const bf16x8_t*>(la.U + (size_t)ucol * RK + k) : (bf16x8_t){0};
        }
    };
    bf16x8_t uf[PRE ? FNT : 1][2], tall[PRE ? FMT : 1][2];
    if constexpr (PRE) {
#pragma unroll
        for (int i = 0; i < FMT; ++i) load_t2(i, 0, tall[i]);
#pragma unroll
        for (int j = 0; j < FNT; ++j) load_u2(j, 0, uf[j]);
    }
    // HOIST: the lane's row scales and its columns' scales and biases (FNT column
    // tiles x 4 quads, 8 FNT + FMT registers) are read from the staged copy up
    // front.  The compiler keeps an LDS read behind any earlier LDS write it may
    // alias, so reads between the scratch writes each wait out their latency,
    // which a wave alone on its SIMD (small grids) cannot hide; kernels with two
    // waves per SIMD and no registers to spare read them where they are used.
    constexpr bool SCALED = EPI != EPI_ACC && EPI != EPI_ATOMIC_ACC;
    constexpr bool HS = HOIST && SCALED;
    float xrow[HS ? FMT : 1];
    float4 wcol[HS ? FNT : 1][4], bcol[HS ? FNT : 1][4];
    if constexpr (HS) {
#pragma unroll
        for (int i = 0; i < FMT; ++i) xrow[i] = sc[row0 - tile_m0 + i * 32 + l32];
#pragma unroll
        for (int j = 0; j < FNT; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int c = col0 - tile_n0 + j * 32 + 4 * h + 8 * q;
                wcol[j][q] = *reinterpret_cast<const float4*>(sc + 256 + c);
                bcol[j][q] = *reinterpret_cast<const float4*>(sc + 512 + c);
            }
    }
#pragma unroll
    for (int i0 = 0; i0 < FMT; i0 += PT) {
#pragma unroll
        for (int ii = 0; ii < PT; ++ii) {
            const int i = i0 + ii;
            float xsv;
            if constexpr (HS) xsv = xrow[i];
            else xsv = sc[row0 - tile_m0 + i * 32 + l32];
#pragma unroll
            for (int j = 0; j < FNT; ++j) {
                f32x16_t lacc = (f32x16_t){0};
                if constexpr (PRE) {
#pragma unroll
                    for (int s = 0; s < 2; ++s)
                        lacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(uf[j][s], tall[i][s], lacc, 0, 0, 0);   // transposed
                } else if constexpr (LR > 0) {
#pragma unroll
                    for (int c = 0; c < LR; ++c) {                     // 32 ranks per batch of loads
                        bf16x8_t ta[2], ub[2];
                        load_t2(i, 2 * c, ta);
                        load_u2(j, 2 * c, ub);
#pragma unroll
                        for (int s = 0; s < 2; ++s)
                            lacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ub[s], ta[s], lacc, 0, 0, 0);   // transposed
                    }
                } else if constexpr (LR < 0) {
                    const int trow = row0 + i * 32 + l32;
                    const int ucol = col0 + j * 32 + l32;
                    for (int rk = 0; rk < la.R; rk += 16) {
                        const int k = rk + 8 * h;
                        const bf16x8_t a = trow < M ? *reinterpret_cast<const bf16x8_t*>(la.t + (size_t)trow * la.R + k)
                                                    : (bf16x8_t){0};
                        const bf16x8_t b = ucol < N ? *reinterpret_cast<const bf16x8_t*>(la.U + (size_t)ucol * la.R + k)
                                                    : (bf16x8_t){0};
                        lacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, a, lacc, 0, 0, 0);   // transposed
                    }
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    uint8_t* dst = scr + (ii * 32 + l32) * RS + (j * 32 + 8 * q + 4 * h) * ES;
                    float wq[4] = {0.f, 0.f, 0.f, 0.f}, bq[4] = {0.f, 0.f, 0.f, 0.f};
                    if constexpr (SCALED) {
                        float4 w4, b4;
                        if constexpr (HS) {
                            w4 = wcol[j][q];
                            b4 = bcol[j][q];
                        } else {   // this quad's column scales and biases, read from the staged copy
                            const int c = col0 - tile_n0 + j * 32 + 4 * h + 8 * q;
                            w4 = *reinterpret_cast<const float4*>(sc + 256 + c);
                            b4 = *reinterpret_cast<const float4*>(sc + 512 + c);
                        }
                        wq[0] = w4.x; wq[1] = w4.y; wq[2] = w4.z; wq[3] = w4.w;
                        bq[0] = b4.x; bq[1] = b4.y; bq[2] = b4.z; bq[3] = b4.w;
                    }
                    if constexpr (EPI == EPI_ACC || EPI == EPI_ATOMIC_ACC) {
                        *reinterpret_cast<int4*>(dst) = make_int4(acc_int<ASH>(acc[i][j][4 * q]), acc_int<ASH>(acc[i][j][4 * q + 1]),
                                                                  acc_int<ASH>(acc[i][j][4 * q + 2]), acc_int<ASH>(acc[i][j][4 * q + 3]));
                    } else {
                        float v[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float a = acc_float<ASH>(acc[i][j][4 * q + e]);
                            if constexpr (EPI == EPI_BF16_EAGER) {
                                float t = bf16r(bf16r(a) * bf16r(xsv));
                                t = bf16r(t * bf16r(wq[e]));
                                t = bf16r(t + bf16r(bq[e]));                        // -0 when there is no bias
                                if constexpr (LORA) t = bf16r(t + bf16r(__fmul_rn(la.scale, lacc[4 * q + e])));
                                v[e] = t;
                            } else {
                                float t = __fmul_rn(__fmul_rn(a, xsv), wq[e]);
                                t = __fadd_rn(t, bq[e]);                            // -0 when there is no bias
                                if constexpr (LORA) t = __fadd_rn(t, __fmul_rn(la.scale, lacc[4 * q + e]));
                                v[e] = t;
                            }
                        }
                        if constexpr (ES == 4) {
                            *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
                        } else {
                            *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
                        }
                    }
                }
            }
        }
        wave_sync();
        constexpr int NCH = PT * 32 * CW;
        constexpr int RSTEP = 64 / CW;                               // rows advanced per 64 chunks
        const int cc = lane % CW;
        const int col = col0 + cc * EPC;
        const int rl0 = lane / CW;
        uint8_t* orow = reinterpret_cast<uint8_t*>(out) + ((size_t)(row0 + i0 * 32 + rl0) * N + col) * ES;
        // A pass whose 32 rows and whose wave-tile columns all lie inside the
        // output (16-byte aligned rows): every lane stores every chunk, so its
        // LDS reads go out together and one wait covers them, instead of one
        // read, wait and bounds-checked store after another.  Wave-uniform.
        if (EPI != EPI_ATOMIC_ACC && vec && row0 + i0 * 32 + PT * 32 <= M && col0 + FNT * 32 <= N) {
            uint4 d[NCH / 64];
#pragma unroll
            for (int q = 0; q < NCH / 64; ++q)
                d[q] = *reinterpret_cast<const uint4*>(scr + (rl0 + q * RSTEP) * RS + cc * 16);
            typedef unsigned v4u_st __attribute__((ext_vector_type(4)));
#pragma unroll
            for (int q = 0; q < NCH / 64; ++q)
                __builtin_nontemporal_store((v4u_st){d[q].x, d[q].y, d[q].z, d[q].w},
                                            reinterpret_cast<v4u_st*>(orow + (size_t)q * RSTEP * N * ES));
            wave_sync();
            continue;
        }
#pragma unroll
        for (int q0 = 0; q0 < NCH; q0 += 64) {
            const int rl = rl0 + (q0 / 64) * RSTEP;
            const int row = row0 + i0 * 32 + rl;
            uint8_t* o = orow + (size_t)(q0 / 64) * RSTEP * N * ES;
            if (row < M && col < N) {
                const uint4 d = *reinterpret_cast<const uint4*>(scr + rl * RS + cc * 16);
                if constexpr (EPI == EPI_ATOMIC_ACC) {     // one atomic add per int32 accumulator
                    const uint32_t w[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (col + e < N) atomicAdd(reinterpret_cast<int32_t*>(o) + e, (int32_t)w[e]);
                } else if (vec && col + EPC <= N) {
                    // non-temporal: the output is not read again by this kernel, and
                    // streaming it past the L2 measured 3% faster over the four Flux
                    // linears at M = 4608 (proj 6%) in an interleaved A/B
                    typedef unsigned v4u_st __attribute__((ext_vector_type(4)));
                    __builtin_nontemporal_store((v4u_st){d.x, d.y, d.z, d.w}, reinterpret_cast<v4u_st*>(o));
                } else {
                    const uint32_t w[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
                    for (int e = 0; e < EPC; ++e) {
                        if (col + e < N) {
                            if constexpr (ES == 2) reinterpret_cast<uint16_t*>(o)[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
                            else reinterpret_cast<uint32_t*>(o)[e] = w[e];
                        }
                    }
                }
            }
        }
        wave_sync();
    }
}

// s_waitcnt immediate that waits until at most n vector-memory operations are
// outstanding (vmcnt split over bits 3:0 and 15:14; expcnt / lgkmcnt not waited)
constexpr int vmcnt_imm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }


// Tile of workgroup `bid` in a tiles_m x tiles_n grid: workgroups are
// renumbered so that each XCD (bid % 8 on MI355X's round-robin dispatch) gets a
// contiguous range of tiles, and tiles are ordered m-fastest within groups of
// `gm` tile rows, so the tiles an XCD runs at one time form a compact block
// that shares A and B chunks in its L2.
__device__ __forceinline__ void tile_of_block(int bid, int tiles_m, int tiles_n, int gm, int& tm, int& tn) {
    const int ntiles = tiles_m * tiles_n;
    const int per = ntiles / 8, rem = ntiles % 8, x = bid % 8, l = bid / 8;
    const int b = x * per + min(x, rem) + l;
    const int grp = b / (gm * tiles_n), inb = b % (gm * tiles_n);
    const int rows_in = min(gm, tiles_m - grp * gm);
    tm = grp * gm + inb % rows_in;
    tn = inb / rows_in;
}

// Row-group size for tile_of_block: about 8 tile rows, a divisor of tiles_m
// when one is close (18 row tiles -> 9).
inline int tile_group_rows(int tiles_m) {
    if (tiles_m <= 8) return tiles_m > 0 ? tiles_m : 1;
    const int cand[] = {8, 9, 7, 6, 10, 12};
    for (int c : cand)
        if (tiles_m % c == 0) return c;
    return 8;
}

// One 16-byte-per-lane global->LDS DMA (global_load_lds_dwordx4): lane i of
// the wave writes lds_addr + 16 i.  Issued from inline asm so the compiler
// adds no conservative vmcnt(0) of its own before later LDS reads; callers
// synchronise with wait_block_landed + a barrier.
__device__ __forceinline__ void dma16(uint32_t lds_addr, const void* src) {
    const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_addr);
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(m0v), "v"(src)
                 : "memory", "m0");
}

// The same copy with a wave-uniform base address and a per-lane byte offset
// (the SADDR form: one VGPR per lane instead of a 64-bit address).
__device__ __forceinline__ void dma16_sv(uint32_t lds_addr, const void* base, uint32_t voff) {
    const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_addr);
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(m0v), "v"(voff), "s"(base)
                 : "memory", "m0");
}

// Wait until this lane's DMA of the oldest in-flight block has landed, given
// that `newer` younger blocks (LOADS instructions each) were issued after it.
// vmcnt counts vector-memory operations completing in issue order, so waiting
// for <= newer * LOADS outstanding is exactly "the oldest block is done".
template <int MAXNEWER, int LOADS>
__device__ __forceinline__ void wait_block_landed(int newer) {
    static_assert(MAXNEWER <= 3 && MAXNEWER * LOADS <= 63, "vmcnt range");
    if (MAXNEWER >= 3 && newer >= 3) __builtin_amdgcn_s_waitcnt(vmcnt_imm(3 * LOADS));
    else if (MAXNEWER >= 2 && newer == 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * LOADS));
    else if (MAXNEWER >= 1 && newer == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(LOADS));
    else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
}

}  // namespace convrot
