// Fused ConvRot rotation + rowwise int4 quantization + nibble packing (gfx950).
//
// Computes, for every row of x [M, K] (dtype DT) and convrot block size G:
//   xr  = RNE_DT( x_g @ H_G )          exactly rounded block-Hadamard rotation
//   a   = max(max_k |xr|, DT(1e-10))
//   s   = RNE_DT( fl32(a / 7) )        -> scale[m] (float)
//   q   = rint_even( RNE_DT( fl32(xr / s) ) )   (or the stochastic variant)
//   out = nibble pack, even k in the low nibble
// which is the arithmetic of the reference eager path
// (_int4/eager.py:65-79 rotation, :104-120 quantizer, _int4/_codec.py:19-25
// pack).  Nothing here follows the reference RDNA4 kernel
// (_int4/int4_gemm.hip:348-408), whose fp32-reciprocal arithmetic differs.
// The int8 tier (W8A8) uses the same kernels with 127 in place of 7, codes
// clamped to [-127, 127] and stored as plain int8 (_int4/int8_eager.py:22-28;
// again the eager arithmetic, not _int4/int4_gemm.hip:572-626, which keeps an
// unrounded fp32 scale).
//
// Work layout
//   * A lane owns a "chunk" of 16 consecutive elements (32 B of bf16, two
//     16-byte loads).  Chunks of one row are spread over `tpr` lanes; when a
//     row has more than 256 chunks a lane takes NPASS chunks (passes).
//   * The 16 elements cover two base-4 digits (d0, d1) of the Hadamard index,
//     so the first two radix-4 stages run in registers.  For G = 64 / 256 the
//     remaining digit(s) live across 4 / 16 lanes; one LDS transpose of the
//     fp64 partial sums brings them into registers for the last stage(s).
//   * Every butterfly runs in fp64.  A group's partial sums are integer
//     multiples of its smallest input ulp bounded by G * max|x|, so they are
//     exact whenever the group's nonzero inputs span at most 53 - 8 - 2*log4(G)
//     - 1 binades (bf16; 36 for G = 256), which real activations satisfy by a
//     wide margin; f16 inputs always (multiples of 2^-24 below 2^16, so every
//     partial sum is a multiple of 2^-24 below 2^48).  The exact value is then
//     rounded once to DT.  Wider groups
//     get fp64-rounded partial sums in the stage order below (restated on the
//     CPU by tests/fp64_rotation.py); the reference's own float matmul rounds
//     those groups too, and more.
//   * The row absmax is reduced through an LDS atomic max; codes go through
//     an LDS byte buffer so each lane stores 8 contiguous packed bytes.
//
// Quantizer exactness.  xr and s are values of DT (p = 8 significant bits for
// bf16, 11 for f16).  Their quotient mx/ms * 2^d is never a DT rounding
// midpoint (that needs an odd (p+1)-bit numerator, while odd(mx)/odd(ms) has
// at most p bits) and lies at least 2^-(2p+1) (relative) from every midpoint.
// So any approximation P of xr/s with relative error below that distance has
// RNE_DT(P) == RNE_DT(xr/s) == RNE_DT(fl32(xr/s)):
//   bf16: P = fl32(xr * fl32(1/s)), error <= 2^-23 < 2^-17;
//   f16:  P = fl32(fl64(xr * fl64(1/s))), error <= 2^-24 + 2^-52 < 2^-23.
// f32 uses the IEEE fp32 division directly.

#include "b6t_layout.h"
#include "common.h"

namespace convrot {

constexpr int kChunk = 16;       // elements per lane per pass
constexpr int kMaxThreads = 256; // lanes per workgroup
constexpr int kPad = 17;         // fp64 words per lane slot in the transpose buffer

// radix-4 stage of the regular Hadamard H4 on four values:
// H4 v = (sum v) 1 - 2 reverse(v)   (H4 as in _int4/eager.py:32-36)
// (every value is exact: sums of inputs times powers of two; fma keeps one op)
__device__ __forceinline__ void h4_stage(double& a, double& b, double& c, double& d, double scale) {
    const double S = (scale == 1.0) ? ((a + b) + (c + d)) : ((a + b) + (c + d)) * scale;
    double t = -2.0 * scale;
    // -2 is an inline constant of the 3-operand fma; any other factor would be
    // a literal, which only the 2-operand fmac takes (plus a copy of S per
    // output): hold it in an SGPR pair instead
    if (scale != 1.0) asm("" : "+s"(t));
    const double na = __builtin_fma(t, d, S), nb = __builtin_fma(t, c, S);
    const double nc = __builtin_fma(t, b, S), nd = __builtin_fma(t, a, S);
    a = na; b = nb; c = nc; d = nd;
}

// stage over one base-4 digit of the 16-entry register array (stride 1 or 4)
template <int STRIDE>
__device__ __forceinline__ void stage16(double (&v)[16], double scale) {
#pragma unroll
    for (int base = 0; base < 16; ++base) {
        if ((base / STRIDE) % 4 != 0) continue;
        h4_stage(v[base], v[base + STRIDE], v[base + 2 * STRIDE], v[base + 3 * STRIDE], scale);
    }
}

template <int DT>
__device__ __forceinline__ void load_chunk(const void* __restrict__ x, size_t elem, double (&v)[16]) {
    if constexpr (DT == DT_F32) {
        const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(x) + elem);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint4 w = p[q];
            v[4 * q + 0] = (double)__uint_as_float(w.x);
            v[4 * q + 1] = (double)__uint_as_float(w.y);
            v[4 * q + 2] = (double)__uint_as_float(w.z);
            v[4 * q + 3] = (double)__uint_as_float(w.w);
        }
    } else {
        const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(x) + elem);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            uint4 w4 = p[q];
            uint32_t w[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (DT == DT_BF16) {
                    v[8 * q + 2 * j] = (double)bf16lo_to_f32(w[j]);
                    v[8 * q + 2 * j + 1] = (double)bf16hi_to_f32(w[j]);
                } else {
                    v[8 * q + 2 * j] = (double)f16bits_to_f32(w[j]);
                    v[8 * q + 2 * j + 1] = (double)f16bits_to_f32(w[j] >> 16);
                }
            }
        }
    }
}

template <int DT>
__device__ __forceinline__ float load_scalar(const void* __restrict__ p, size_t i) {
    if constexpr (DT == DT_F32) return reinterpret_cast<const float*>(p)[i];
    else if constexpr (DT == DT_BF16) return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(p)[i] << 16);
    else return f16bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

// the python scalar 1e-10 of the eager clamp, converted to the tensor dtype
template <int DT>
__device__ __forceinline__ float clamp_floor() {
    if constexpr (DT == DT_F32) return 1e-10f;
    else if constexpr (DT == DT_BF16) return __uint_as_float(0x2edc0000u);  // bf16(1e-10)
    else return 0.0f;                                                        // f16(1e-10) underflows
}

// group-local element index held in register slot i after the last stage,
// for lane position gl within the group (see the transpose below)
template <int G>
__device__ __forceinline__ int final_elem(int gl, int i) {
    if constexpr (G == 256) return gl + 16 * i;
    else if constexpr (G == 64) return 16 * (i >> 2) + 4 * gl + (i & 3);
    else return i;
}

template <int DT, int G, int NPASS, bool STOCH, bool I8>
__global__ __launch_bounds__(kMaxThreads) void rotquant_kernel(
        const void* __restrict__ x, const void* __restrict__ noise,
        int8_t* __restrict__ qout, float* __restrict__ sout,
        int M, int K, int tpr, int rows_per_wg) {
    constexpr int LPG = G / kChunk;             // lanes per convrot group
    __shared__ double tbuf[kMaxThreads * kPad];
    __shared__ uint32_t cbuf[kMaxThreads * 4];  // 16 code bytes per lane slot
    __shared__ uint32_t rowmax[kMaxThreads];

    const int tid = threadIdx.x;
    const int rloc = tid / tpr;
    const int t = tid - rloc * tpr;
    const int row = blockIdx.x * rows_per_wg + rloc;
    const bool row_ok = (rloc < rows_per_wg) && (row < M);
    const int nchunks = K / kChunk;
    const int gl = t % LPG;                     // lane position inside its group
    const int gfirst = tid - gl;                // workgroup slot of the group's first lane

    if (tid < rows_per_wg) rowmax[tid] = 0u;

    float xr[NPASS][kChunk];
    float lmax = 0.0f;

#pragma unroll
    for (int p = 0; p < NPASS; ++p) {
        const int c = p * tpr + t;
        const bool ok = row_ok && (c < nchunks);
        double v[16];
        if (ok) {
            load_chunk<DT>(x, (size_t)row * K + (size_t)c * kChunk, v);
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = 0.0;
        }
        // digits d0 (stride 1) and d1 (stride 4) in registers
        if constexpr (G == 16) {
            stage16<1>(v, 1.0);
            stage16<4>(v, 0.25);                // 1/sqrt(16), exact
        } else {
            stage16<1>(v, 1.0);
            stage16<4>(v, 1.0);
            // transpose across the LPG lanes of the group through LDS
            __syncthreads();                    // previous pass finished reading
#pragma unroll
            for (int i = 0; i < 16; ++i) tbuf[tid * kPad + i] = v[i];
            __syncthreads();
            if constexpr (G == 256) {
                // lane gl takes position gl of every lane's 16: w[m] = (d0d1 = gl, d2d3 = m)
#pragma unroll
                for (int m = 0; m < 16; ++m) v[m] = tbuf[(gfirst + m) * kPad + gl];
                stage16<1>(v, 1.0);
                stage16<4>(v, 1.0 / 16.0);      // 1/sqrt(256), exact
            } else {                            // G == 64, LPG == 4
                // w[a + 4 b] = (d0d1 = 4 gl + a, d2 = b)
#pragma unroll
                for (int b = 0; b < 4; ++b)
#pragma unroll
                    for (int a = 0; a < 4; ++a) v[a + 4 * b] = tbuf[(gfirst + b) * kPad + 4 * gl + a];
                stage16<4>(v, 1.0 / 8.0);       // 1/sqrt(64), exact
            }
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float r = round_f64_to_dt<DT>(v[i]);
            xr[p][i] = r;
            if (ok) lmax = fmaxf(lmax, fabsf(r));
        }
    }

    // row absmax (non-negative floats order like their bit patterns)
    __syncthreads();
    if (row_ok) atomicMax(&rowmax[rloc], __float_as_uint(lmax));
    __syncthreads();

    float a = __uint_as_float(row_ok ? rowmax[rloc] : 0u);
    a = fmaxf(a, clamp_floor<DT>());
    constexpr float QMAX = I8 ? 127.0f : 7.0f;
    const float s = round_to_dt<DT>(a / QMAX);  // IEEE division (no fast-math)
    if (row_ok && t == 0) sout[row] = s;
    const double rinv = 1.0 / (double)s;
    const float rinv32 = 1.0f / s;
    const float kMagic = 12582912.0f;           // 1.5 * 2^23: float add rounds to integer, ties to even

#pragma unroll
    for (int p = 0; p < NPASS; ++p) {
        const int c = p * tpr + t;
        const bool ok = row_ok && (c < nchunks);
        const int gbase = (c - gl) * kChunk;    // group's first element within the row
        uint8_t codes[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float z;
            if constexpr (DT == DT_F32) z = xr[p][i] / s;
            else if constexpr (DT == DT_BF16) z = round_to_dt<DT>(xr[p][i] * rinv32);
            else z = round_to_dt<DT>((float)((double)xr[p][i] * rinv));
            int q;
            if constexpr (STOCH) {
                const int e = final_elem<G>(gl, i);
                float u = ok ? load_scalar<DT>(noise, (size_t)row * K + gbase + e) : 0.0f;
                float f = floorf(round_to_dt<DT>(z + u));
                f = fminf(fmaxf(f, -7.0f), 7.0f);
                q = (f == f) ? (int)f : 0;      // NaN (0/0 when s == 0) -> 0
            } else {
                // f16 rows of zeros have s == 0 and give 0/0: the code is 0
                if constexpr (DT == DT_F16) z = (z == z) ? z : 0.0f;
                z = fminf(fmaxf(z, -QMAX), QMAX);       // |z| <= QMAX (1 + 2^-9) already; guards non-finite input
                q = (int)__float_as_uint(z + kMagic);   // low byte = rint_even(z)
            }
            codes[i] = I8 ? (uint8_t)q : (uint8_t)(q & 0xF);
        }
        // scatter codes to their element positions, then read back own chunk
        __syncthreads();
        uint8_t* cb = reinterpret_cast<uint8_t*>(cbuf);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int e = final_elem<G>(gl, i);
            cb[(gfirst + e / kChunk) * 16 + (e % kChunk)] = codes[i];
        }
        __syncthreads();
        if (I8 && ok) {
            *reinterpret_cast<uint4*>(qout + (size_t)row * K + (size_t)c * kChunk) =
                reinterpret_cast<const uint4*>(cbuf)[tid];
        } else if (ok) {
            const uint4 w = reinterpret_cast<const uint4*>(cbuf)[tid];
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
            uint32_t o[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                uint32_t t0 = ws[2 * h] | (ws[2 * h] >> 4);
                uint32_t t1 = ws[2 * h + 1] | (ws[2 * h + 1] >> 4);
                o[h] = (t0 & 0xffu) | ((t0 >> 8) & 0xff00u) | ((t1 & 0xffu) << 16) | ((t1 << 8) & 0xff000000u);
            }
            uint2* dst = reinterpret_cast<uint2*>(qout + (size_t)row * (K / 2) + (size_t)c * (kChunk / 2));
            *dst = make_uint2(o[0], o[1]);
        }
    }
}

// ---------------------------------------------------------------------------
// Row-split kernel (K <= 32768).
//
// A workgroup of W waves quantizes row blockIdx.x (the grid is M).  A row of K
// elements is K/16 chunks; wave w of the workgroup rotates chunks
// (p * W + w) * 64 + lane for the passes p < P, so W * P passes of 64 lanes
// cover the row.  While a pass is rotated, the wave loads its next pass.
// The fp64 transpose and the code gather use a private LDS region per wave;
// the row absmax is a shuffle reduction within each wave and then a max over
// the W waves through LDS, the workgroup's one barrier per row.  Rounded
// rotated values stay in registers as packed 16-bit pairs until the row scale
// is known.  Splitting rows over the waves of a workgroup keeps every wave's
// share of the work small, so the last rows of the launch do not leave a few
// waves running a whole row each while the rest of the chip idles.
// ---------------------------------------------------------------------------

constexpr int kRowMaxWaves = 4;                        // waves per workgroup, rows of up to 12288
constexpr int kRowWideWaves = 16;                      // waves per workgroup, rows of up to 32768
constexpr int kRowMaxPass = 6;                         // passes per wave
constexpr int kRowWaveLds = 64 * kPad * 8;             // LDS bytes per wave

typedef unsigned v16u __attribute__((ext_vector_type(16)));
typedef unsigned v6u __attribute__((ext_vector_type(6)));
typedef __bf16 v32bf __attribute__((ext_vector_type(32)));

template <int DT>
struct ChunkRegs { uint4 r[DT == DT_F32 ? 4 : 2]; };

template <int DT>
__device__ __forceinline__ void load_regs(const void* __restrict__ x, size_t elem, ChunkRegs<DT>& c) {
    constexpr int esz = DT == DT_F32 ? 4 : 2;
    const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(x) + elem * esz);
#pragma unroll
    for (int q = 0; q < (DT == DT_F32 ? 4 : 2); ++q) c.r[q] = p[q];
}

template <int DT>
__device__ __forceinline__ void regs_to_f64(const ChunkRegs<DT>& c, double (&v)[16]) {
    if constexpr (DT == DT_F32) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            v[4 * q + 0] = (double)__uint_as_float(c.r[q].x);
            v[4 * q + 1] = (double)__uint_as_float(c.r[q].y);
            v[4 * q + 2] = (double)__uint_as_float(c.r[q].z);
            v[4 * q + 3] = (double)__uint_as_float(c.r[q].w);
        }
    } else {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const uint32_t w[4] = {c.r[q].x, c.r[q].y, c.r[q].z, c.r[q].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (DT == DT_BF16) {
                    v[8 * q + 2 * j] = (double)bf16lo_to_f32(w[j]);
                    v[8 * q + 2 * j + 1] = (double)bf16hi_to_f32(w[j]);
                } else {
                    v[8 * q + 2 * j] = (double)f16bits_to_f32(w[j]);
                    v[8 * q + 2 * j + 1] = (double)f16bits_to_f32(w[j] >> 16);
                }
            }
        }
    }
}

// storage of 16 rounded values: packed 16-bit pairs for bf16/f16, floats for f32
template <int DT> struct Held { uint32_t w[8]; };
template <> struct Held<DT_F32> { float f[16]; };

template <int DT>
__device__ __forceinline__ void hold(Held<DT>& h, int i, float a, float b) {   // values i, i+1
    if constexpr (DT == DT_F32) {
        h.f[i] = a; h.f[i + 1] = b;
    } else if constexpr (DT == DT_BF16) {
        h.w[i >> 1] = (__float_as_uint(a) >> 16) | (__float_as_uint(b) & 0xffff0000u);
    } else {
        h.w[i >> 1] = (uint32_t)__half_as_ushort(__float2half_rn(a)) |
                      ((uint32_t)__half_as_ushort(__float2half_rn(b)) << 16);
    }
}

template <int DT>
__device__ __forceinline__ float held(const Held<DT>& h, int i) {
    if constexpr (DT == DT_F32) return h.f[i];
    else if constexpr (DT == DT_BF16) return (i & 1) ? bf16hi_to_f32(h.w[i >> 1]) : bf16lo_to_f32(h.w[i >> 1]);
    else return f16bits_to_f32((i & 1) ? (h.w[i >> 1] >> 16) : h.w[i >> 1]);
}

// fp64 -> float with the bits below float precision folded into a sticky bit
// (see round_f64_to_dt): rounding the result once to bf16/f16 equals rounding
// the fp64 value once.  Monotone, so the max of jammed values rounds to the
// max of the rounded values.
// The whole low dword is below the bf16 / f16 guard bit, so only whether it
// is nonzero matters.  It is replaced by the float bits of its value as an
// unsigned integer: 0 for 0, else a pattern in [0x3F800000, 0x4F800000] whose
// bits 31..29 (the last three a float keeps) are not all clear and stay so
// after the rounding to float, which cannot carry past bit 31.  Below those
// bits the replacement is less than one unit of bit 32, so it changes no
// rounding decision of the conversion either (subnormal results included).
// One conversion instead of a compare and a select.
__device__ __forceinline__ float jam_to_f32(double d) {
    const uint64_t u = (uint64_t)__double_as_longlong(d);
    const uint32_t lo = __float_as_uint((float)(uint32_t)u);
    return (float)__longlong_as_double((long long)((u & 0xffffffff00000000ull) | lo));
}


// Store the 32 codes of group k0 .. k0+31 of `row` (6 packed dwords, k0 % 32 ==
// 0) at their place in a B6T buffer (placement: b6t_layout.h).
__device__ __forceinline__ void b6_store_group(int8_t* out, int row, int K, int k0, const uint32_t (&d)[6]) {
    const int kb = k0 >> 7, g = (k0 >> 5) & 3, r = row & 255;
    uint8_t* chunk = reinterpret_cast<uint8_t*>(out) + ((size_t)(row >> 8) * (K >> 7) + kb) * B6_CHUNK;
    uint32_t* p = reinterpret_cast<uint32_t*>(chunk + b6_p_off(r, g));
    uint32_t* q = reinterpret_cast<uint32_t*>(chunk + b6_q_off(r, g));
    if (!b6_odd_tile(r)) {          // P = d0..d3, Q bytes 0..7 = d4..d5
        *reinterpret_cast<uint4*>(p) = make_uint4(d[0], d[1], d[2], d[3]);
        *reinterpret_cast<uint2*>(q) = make_uint2(d[4], d[5]);
    } else {                        // P = d2..d5, Q bytes 8..15 = d0..d1
        *reinterpret_cast<uint4*>(p) = make_uint4(d[2], d[3], d[4], d[5]);
        *reinterpret_cast<uint2*>(q + 2) = make_uint2(d[0], d[1]);
    }
}

// OUT selects the code format: OUT_PACK4 packed nibbles; OUT_B6T the B6T
// layout of the bf6 GEMM (b6t_layout.h; K % 128 == 0; rows M .. ceil(M/256)*256
// get zero codes); OUT_I8 the int8 tier's plain int8 codes (scale a / 127,
// codes clamped to [-127, 127], _int4/int8_eager.py:22-28).
// OUT_I8T the same int8 codes in the I8T layout of the W8A8 GEMM (b6t_layout.h;
// K % 64 == 0; padding rows get zero codes).
enum : int { OUT_PACK4 = 0, OUT_B6T = 1, OUT_I8 = 2, OUT_I8T = 3 };

// all butterfly stages of one chunk (16 values of the lane in v); tbuf is the
// wave's transpose buffer
template <int G>
__device__ __forceinline__ void rotate_chunk(double (&v)[16], double* tbuf, int lane, int gl, int gfirst) {
    if constexpr (G == 16) {
        stage16<1>(v, 1.0);
        stage16<4>(v, 0.25);
    } else {
        stage16<1>(v, 1.0);
        stage16<4>(v, 1.0);
#pragma unroll
        for (int i = 0; i < 16; ++i) tbuf[lane * kPad + i] = v[i];
        wave_sync();
        if constexpr (G == 256) {
#pragma unroll
            for (int m = 0; m < 16; ++m) v[m] = tbuf[(gfirst + m) * kPad + gl];
            stage16<1>(v, 1.0);
            stage16<4>(v, 1.0 / 16.0);
        } else {
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int a = 0; a < 4; ++a) v[a + 4 * b] = tbuf[(gfirst + b) * kPad + 4 * gl + a];
            stage16<4>(v, 1.0 / 8.0);
        }
        wave_sync();
    }
}

// max(m, |a|, |b|) in one instruction
__device__ __forceinline__ float absmax3(float m, float a, float b) {
    float r;
    asm("v_max3_f32 %0, %1, |%2|, |%3|" : "=v"(r) : "v"(m), "v"(a), "v"(b));
    return r;
}

// round the 16 rotated values to DT, keep them in h and fold them into lmax
template <int DT>
__device__ __forceinline__ void hold_chunk(const double (&v)[16], Held<DT>& h, float& lmax) {
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
        if constexpr (DT == DT_BF16) {
            // lmax gathers jammed values: its RNE is the max of the rounded values
            const float f0 = jam_to_f32(v[i]), f1 = jam_to_f32(v[i + 1]);
            h.w[i >> 1] = pack_bf16x2(f0, f1);
            lmax = absmax3(lmax, f0, f1);
        } else {
            const float r0 = round_f64_to_dt<DT>(v[i]);
            const float r1 = round_f64_to_dt<DT>(v[i + 1]);
            hold<DT>(h, i, r0, r1);
            lmax = absmax3(lmax, r0, r1);
        }
    }
}

// max(v, v of another lane) on the bit patterns of non-negative floats (the
// integer order of such patterns is their float order), the other lane chosen
// by the DPP control CTRL on the rows in ROW_MASK (other rows take 0: keep v)
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t umax_dpp(uint32_t v) {
    const uint32_t t = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xf, false);
    return v > t ? v : t;
}

// max over the 64 lanes of a non-negative, non-NaN float, as a wave-uniform value
__device__ __forceinline__ float wave_max_nonneg(float f) {
    uint32_t v = __float_as_uint(f);
    v = umax_dpp<0xb1, 0xf>(v);     // quad_perm [1,0,3,2]
    v = umax_dpp<0x4e, 0xf>(v);     // quad_perm [2,3,0,1]
    v = umax_dpp<0x124, 0xf>(v);    // row_ror:4
    v = umax_dpp<0x128, 0xf>(v);    // row_ror:8: every lane holds its row's max
    v = umax_dpp<0x142, 0xa>(v);    // row_bcast:15 into rows 1 and 3
    v = umax_dpp<0x143, 0xc>(v);    // row_bcast:31 into rows 2 and 3: lane 63 holds the max
    return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)v, 63));
}

// max(a, b, c) in one instruction (no NaN operands here)
__device__ __forceinline__ float fmax3(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// LR: also finish the linear's LoRA down projection for every row (LoraSum):
// wave 0 loads the row's partials at the start of the row and stores their sum
// after the row's codes, so the loads' latency hides behind the rotation.
// MAXW: the largest workgroup (in waves) the instance serves; RS = 8 or 16
// row-absmax slots per row parity.
// The kernel needs about 64 VGPRs, so the compiler would schedule for 8 waves
// per SIMD; its 8.7 KB of LDS per wave admits at most 18 waves per CU (4 to 5
// per SIMD), and scheduling for that occupancy leaves the loads more room
// (interleaved A/B on MI355X, B6T out: 16384 x 3072 42.0 -> 37.4 us, 4608 x
// 3072 13.8 -> 13.7 us).
template <int DT, int G, int P, int OUT, bool LR, int MAXW = kRowMaxWaves>
__global__ __launch_bounds__(64 * MAXW) __attribute__((amdgpu_waves_per_eu(4, 5))) void rotquant_row_kernel(
        const void* __restrict__ x, int8_t* __restrict__ qout, float* __restrict__ sout, int M, int K,
        LoraSum ls) {
    constexpr int LPG = G / kChunk;
    constexpr bool B6 = OUT == OUT_B6T;
    constexpr bool INT8 = OUT == OUT_I8 || OUT == OUT_I8T;
    constexpr float QMAX = INT8 ? 127.0f : 7.0f;
    // Per-wave LDS: the fp64 transpose buffer of the rotation, reused as the
    // code reorder buffer of the quantize loop (which runs after every pass of
    // the row; a wave's LDS operations complete in order).  Codes: bytes (64
    // chunks x 16) for the integer outputs; for B6T the rounded codes as bf16,
    // chunk ch at (ch / 16) * 544 + (ch % 16) * 32 bytes (the pad spreads the
    // four 16-lane groups over the banks), one region per pass parity so that
    // two passes are converted together.  After the W wave buffers: the
    // per-wave row absmax, RS slots per row parity (slots W..RS-1 hold zeros).
    constexpr int RS = MAXW <= 8 ? 8 : 16;
    static_assert(MAXW <= 16, "row absmax slots");
    constexpr int kB6Group = 544;
    constexpr int kB6Region = 4 * kB6Group;
    static_assert(kRowWaveLds >= (B6 ? 2 * kB6Region : 64 * 16), "code buffer");
    extern __shared__ __attribute__((aligned(16))) double rq_lds[];

    const int W = __builtin_amdgcn_readfirstlane(blockDim.x >> 6);
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    double* tbuf = rq_lds + wv * (64 * kPad);
    uint8_t* cb = reinterpret_cast<uint8_t*>(tbuf);
    float* red = reinterpret_cast<float*>(rq_lds + W * (64 * kPad));
    auto b6_slot = [&](int ch, int pos, int region) {
        return reinterpret_cast<uint16_t*>(cb + region * kB6Region + (ch >> 4) * kB6Group + (ch & 15) * 32) + pos;
    };
    const int nchunks = K / kChunk;
    const int gl = lane % LPG;
    const int gfirst = lane - gl;
    const float kMagic = 12582912.0f;
    if (wv == 0 && lane < 2 * RS && (lane & (RS - 1)) >= W) red[lane] = 0.0f;   // before the first barrier

    // One row per workgroup (the grid is M).  Two chunk buffers in turn: while
    // pass p is rotated from bufs[p & 1], the wave loads its next pass into the
    // other one, so no register copies carry a prefetch across passes.  Every
    // load is unconditional (a lane past the row end reads the pass's first
    // chunk, a next pass past the row end re-reads this one): with no branch
    // around it, each pass waits for its own loads only.  Lanes past the row
    // end (whole convrot groups, since K % G == 0) rotate those copies; they
    // are left out of the row absmax and store no codes.
    ChunkRegs<DT> bufs[2];
    const int row = blockIdx.x;
    {
        const int c0 = wv * 64;   // < nchunks: W <= number of passes of a row
        load_regs<DT>(x, (size_t)row * K + (size_t)(c0 + lane < nchunks ? c0 + lane : c0) * kChunk, bufs[0]);
    }

    {
        Held<DT> hv[P];
        float lmax = 0.0f;
        float lp[8];                 // LoRA partials of rank column `lane` (LR, wave 0)
        if constexpr (LR) {
            if (wv == 0) {
#pragma unroll
                for (int s = 0; s < 8; ++s)
                    lp[s] = (s < ls.S && lane < ls.R) ? ls.part[((size_t)s * M + row) * ls.R + lane] : 0.0f;
            }
        }
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int c0 = (p * W + wv) * 64;     // wave-uniform
            if (c0 < nchunks) {
                const int c = c0 + lane;
                const bool ok = c < nchunks;
                double v[16];
                regs_to_f64<DT>(bufs[p & 1], v);
                if (p + 1 < P) {
                    const int n0 = ((p + 1) * W + wv) * 64;
                    const int l0 = n0 < nchunks ? n0 : c0;
                    load_regs<DT>(x, (size_t)row * K + (size_t)(l0 + lane < nchunks ? l0 + lane : l0) * kChunk,
                                  bufs[(p + 1) & 1]);
                }
                rotate_chunk<G>(v, tbuf, lane, gl, gfirst);
                float pmax = 0.0f;
                hold_chunk<DT>(v, hv[p], pmax);
                lmax = ok ? fmaxf(lmax, pmax) : lmax;
            }
        }
        // row absmax: across the wave (lmax is never NaN: it starts at 0 and
        // v_max3 drops NaN operands), then across the W waves
        lmax = wave_max_nonneg(lmax);
        if (W > 1) {
            float* rb = red;
            if (lane == 0) rb[wv] = lmax;
            __syncthreads();
            const float4 r0 = reinterpret_cast<const float4*>(rb)[0];
            const float4 r1 = reinterpret_cast<const float4*>(rb)[1];
            lmax = fmax3(fmax3(r0.x, r0.y, r0.z), fmax3(r0.w, r1.x, r1.y), fmax3(r1.z, r1.w, 0.0f));
            if constexpr (RS == 16) {
                const float4 r2 = reinterpret_cast<const float4*>(rb)[2];
                const float4 r3 = reinterpret_cast<const float4*>(rb)[3];
                lmax = fmax3(lmax, fmax3(r2.x, r2.y, r2.z), fmax3(r2.w, r3.x, r3.y));
                lmax = fmax3(lmax, r3.z, r3.w);
            }
        }
        const float a = fmaxf(round_to_dt<DT>(lmax), clamp_floor<DT>());
        // s = RNE_DT(fl32(a / QMAX)).  a is a DT value of p <= 11 significant
        // bits and QMAX is odd, so a / QMAX is never a DT rounding midpoint and
        // lies at least 2^(-p-1) / QMAX >= 2^-19 (relative) from every one (a
        // midpoint is an odd multiple of a half unit; a * 2^k / QMAX with a
        // multiple of 2 above it is not); fl32(a / QMAX) and a * fl32(1 / QMAX),
        // both within 2^-23 of a / QMAX, round to the same DT value.
        const float s = DT == DT_F32 ? a / QMAX : round_to_dt<DT>(a * (1.0f / QMAX));
        // bf16: v_rcp_f32 is within 1 ulp of 1 / s, so xr * rinv32 stays within
        // 2^-22 of xr / s, inside the 2^-17 the quotient keeps from every bf16
        // midpoint (file header)
        const float rinv32 = __builtin_amdgcn_rcpf(s);
        const double rinv = 1.0 / (double)s;
        // B6T: the codes of flush f (after passes 2f, 2f+1) stay in registers
        // until every flush of the row is converted, then all are stored: a
        // store issued mid-loop would hold back the next flush, whose registers
        // reuse the pending store's data (the wait covers every store in flight).
        constexpr int NF = B6 ? (P + 1) / 2 : 1;
        uint32_t fd[NF][6];
        int fcg[NF];
#pragma unroll
        for (int f = 0; f < NF; ++f) fcg[f] = -1;
        // the other layouts: each pass's 16 code bytes (int8) or 8 packed bytes, and its chunk (-1: none)
        uint32_t pw[P][4] = {};
        int pc[P];
#pragma unroll
        for (int p2 = 0; p2 < P; ++p2) pc[p2] = -1;

#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int c0 = (p * W + wv) * 64;
            if (c0 >= nchunks) continue;
            const int c = c0 + lane;
            const bool ok = c < nchunks;
#pragma unroll
            for (int i = 0; i < 16; i += 2) {
                float z0, z1;
                const int e0 = final_elem<G>(gl, i), e1 = final_elem<G>(gl, i + 1);
                if constexpr (DT == DT_BF16) {
                    // one packed RNE for both quotients; |z| <= QMAX (1 + 2^-9) because
                    // s = RNE(absmax / QMAX), so rint stays in [-QMAX, QMAX]; the int8
                    // clamp only guards non-finite input
                    const uint32_t zz = pack_bf16x2(bf16lo_to_f32(hv[p].w[i >> 1]) * rinv32,
                                                    bf16hi_to_f32(hv[p].w[i >> 1]) * rinv32);
                    if constexpr (B6) {
                        // the bf16 quotients as they are: the BF6 conversion (scale 16)
                        // rounds each to the code of rint_even(z), |z| <= 7 (1 + 2^-9)
                        *b6_slot(gfirst + e0 / kChunk, e0 % kChunk, p & 1) = (uint16_t)zz;
                        *b6_slot(gfirst + e1 / kChunk, e1 % kChunk, p & 1) = (uint16_t)(zz >> 16);
                        continue;
                    }
                    z0 = bf16lo_to_f32(zz);
                    z1 = bf16hi_to_f32(zz);
                    if constexpr (INT8) {
                        z0 = fminf(fmaxf(z0, -QMAX), QMAX);
                        z1 = fminf(fmaxf(z1, -QMAX), QMAX);
                    }
                } else {
                    float zz[2];
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const float xv = held<DT>(hv[p], i + h);
                        float z;
                        if constexpr (DT == DT_F32) z = xv / s;
                        else z = round_to_dt<DT>((float)((double)xv * rinv));
                        if constexpr (DT == DT_F16) z = (z == z) ? z : 0.0f;
                        zz[h] = fminf(fmaxf(z, -QMAX), QMAX);
                    }
                    z0 = zz[0];
                    z1 = zz[1];
                }
                if constexpr (B6) {
                    // f16 / f32 input: the DT-rounded quotient would not survive a bf16
                    // rounding, so rint_even(z) here, kept as its bf16 bits (exact: an
                    // integer of magnitude <= 7; a zero code may carry the sign of z),
                    // which the conversion maps to its code unchanged
                    const float q0 = __builtin_rintf(z0), q1 = __builtin_rintf(z1);
                    *b6_slot(gfirst + e0 / kChunk, e0 % kChunk, p & 1) = (uint16_t)(__float_as_uint(q0) >> 16);
                    *b6_slot(gfirst + e1 / kChunk, e1 % kChunk, p & 1) = (uint16_t)(__float_as_uint(q1) >> 16);
                } else {
                    // low byte of the float bits of z + 1.5*2^23 is rint_even(z) (two's complement)
                    cb[(gfirst + e0 / kChunk) * 16 + (e0 % kChunk)] = (uint8_t)__float_as_uint(z0 + kMagic);
                    cb[(gfirst + e1 / kChunk) * 16 + (e1 % kChunk)] = (uint8_t)__float_as_uint(z1 + kMagic);
                }
            }
            if constexpr (B6) {
                // The 32 codes of one MFMA group are two consecutive chunks of a pass.
                // After every odd pass, and after the wave's last pass, lane L takes
                // group L % 32 of pass (p & ~1) + L / 32: one 32-wide BF6 conversion
                // per two passes, on every lane (lanes of a pass not yet written idle).
                const bool flush = (p & 1) || p + 1 == P || ((p + 1) * W + wv) * 64 >= nchunks;
                if (flush) {
                    wave_sync();
                    const int pp = (p & ~1) + (lane >> 5);
                    const int ch = 2 * (lane & 31);                       // first chunk of the group in pass pp
                    const int cg = (pp * W + wv) * 64 + ch;               // its chunk in the row
                    const bool live = pp <= p && cg < nchunks;
                    uint4 gq[4];
                    if (live) {
#pragma unroll
                        for (int h = 0; h < 4; ++h) gq[h] = reinterpret_cast<const uint4*>(b6_slot(ch, 0, pp & 1))[h];
                    }
                    wave_sync();
                    if (live) {
                        const v16u words = {gq[0].x, gq[0].y, gq[0].z, gq[0].w, gq[1].x, gq[1].y, gq[1].z, gq[1].w,
                                            gq[2].x, gq[2].y, gq[2].z, gq[2].w, gq[3].x, gq[3].y, gq[3].z, gq[3].w};
                        // scale 16: the code of round(value / 16) on E3M2's 1/16 grid = the
                        // B6T code of rint_even(value) (b6t_layout.h)
                        const v6u r = __builtin_amdgcn_cvt_scalef32_pk32_bf6_bf16(__builtin_bit_cast(v32bf, words), 16.0f);
#pragma unroll
                        for (int i = 0; i < 6; ++i) fd[p >> 1][i] = r[i];
                    }
                    fcg[p >> 1] = live ? cg : -1;
                }
                continue;
            }
            wave_sync();
            const uint4 w = reinterpret_cast<const uint4*>(cb)[lane];
            wave_sync();
            if constexpr (!B6) {
                if constexpr (OUT == OUT_PACK4) {
                    const uint32_t ws[4] = {w.x & 0x0f0f0f0fu, w.y & 0x0f0f0f0fu, w.z & 0x0f0f0f0fu,
                                            w.w & 0x0f0f0f0fu};
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const uint32_t t0 = ws[2 * h] | (ws[2 * h] >> 4);
                        const uint32_t t1 = ws[2 * h + 1] | (ws[2 * h + 1] >> 4);
                        pw[p][h] = (t0 & 0xffu) | ((t0 >> 8) & 0xff00u) | ((t1 & 0xffu) << 16) |
                                   ((t1 << 8) & 0xff000000u);
                    }
                } else {
                    pw[p][0] = w.x; pw[p][1] = w.y; pw[p][2] = w.z; pw[p][3] = w.w;
                }
                pc[p] = ok ? c : -1;
            }
        }
        // Every store of the row goes out here, after the last LDS read: the
        // stores' data registers stay live until all are issued (the asm below),
        // so no wait for a store in flight holds back the row's other work.
        if constexpr (B6) {
#pragma unroll
            for (int f = 0; f < NF; ++f)
                if (fcg[f] >= 0) b6_store_group(qout, row, K, fcg[f] * kChunk, fd[f]);
#pragma unroll
            for (int f = 0; f < NF; ++f)
                asm volatile("" :: "v"(fd[f][0]), "v"(fd[f][1]), "v"(fd[f][2]), "v"(fd[f][3]), "v"(fd[f][4]),
                             "v"(fd[f][5]));
        } else {
#pragma unroll
            for (int p = 0; p < P; ++p) {
                if (pc[p] < 0) continue;
                const int k0 = pc[p] * kChunk;
                if constexpr (OUT == OUT_I8) {
                    *reinterpret_cast<uint4*>(qout + (size_t)row * K + k0) =
                        make_uint4(pw[p][0], pw[p][1], pw[p][2], pw[p][3]);
                } else if constexpr (OUT == OUT_I8T) {
                    int8_t* chunk = qout + ((size_t)(row >> 8) * (K >> 6) + (k0 >> 6)) * I8T_CHUNK;
                    *reinterpret_cast<uint4*>(chunk + i8t_off(row & 255, (k0 >> 4) & 3)) =
                        make_uint4(pw[p][0], pw[p][1], pw[p][2], pw[p][3]);
                } else {
                    *reinterpret_cast<uint2*>(qout + (size_t)row * (K / 2) + k0 / 2) = make_uint2(pw[p][0], pw[p][1]);
                }
            }
#pragma unroll
            for (int p = 0; p < P; ++p)
                asm volatile("" :: "v"(pw[p][0]), "v"(pw[p][1]), "v"(pw[p][2]), "v"(pw[p][3]));
        }
        if (wv == 0 && lane == 0) sout[row] = s;
        if constexpr (LR) {
            // t = bf16(part[0] + .. + part[S-1]), the order of lora_reduce_kernel
            if (wv == 0) {
                if (lane < ls.R) {
                    float v = 0.0f;
#pragma unroll
                    for (int s = 0; s < 8; ++s)
                        if (s < ls.S) v += lp[s];
                    ls.t[(size_t)row * ls.R + lane] = (__bf16)v;
                }
                for (int j = lane + 64; j < ls.R; j += 64) {     // ranks above 64
                    float v = 0.0f;
                    for (int s = 0; s < ls.S; ++s) v += ls.part[((size_t)s * M + row) * ls.R + j];
                    ls.t[(size_t)row * ls.R + j] = (__bf16)v;
                }
            }
        }
    }
    if constexpr (OUT == OUT_I8T) {   // zero codes in the padding rows of the last 256-row tile
        const int mpad = (M + 255) & ~255;
        for (int prow = M + blockIdx.x; prow < mpad; prow += gridDim.x)
            for (int k0 = 16 * (wv * 64 + lane); k0 < K; k0 += 16 * 64 * W) {
                int8_t* chunk = qout + ((size_t)(prow >> 8) * (K >> 6) + (k0 >> 6)) * I8T_CHUNK;
                *reinterpret_cast<uint4*>(chunk + i8t_off(prow & 255, (k0 >> 4) & 3)) = make_uint4(0u, 0u, 0u, 0u);
            }
    }
    if constexpr (B6) {   // zero codes in the padding rows of the last 256-row tile
        const int mpad = (M + 255) & ~255;
        const uint32_t z[6] = {0u, 0u, 0u, 0u, 0u, 0u};
        for (int prow = M + blockIdx.x; prow < mpad; prow += gridDim.x)
            for (int k0 = 32 * (wv * 64 + lane); k0 < K; k0 += 32 * 64 * W) b6_store_group(qout, prow, K, k0, z);
    }
}

// Launch shape: a row is np = ceil(K / 1024) passes of 64 lanes; W <= 4 waves
// of a workgroup share it with P = ceil(np / W) passes each.  Rows of up to 4
// passes (K <= 4096) go to one wave each (W = 1, P = np): no barrier between
// waves, and the per-row tail (absmax, scale) is paid once per np passes.
// Longer rows: 2 or 3 passes per wave up to np = 8, beyond that 3 passes on
// each of up to 4 waves (the 3-pass kernel holds fewer registers than the
// 6-pass one: 4 waves per SIMD instead of 3).  Measured (HIP events, bf16 ->
// B6T): M = 4608, K = 3072: 1 wave x 3 passes 17.2 us, 3 x 1 18.3 us; M =
// 16384, K = 3072: 1 x 3 42.5 us, 3 x 1 52.2 us; M = 4608, K = 12288: 2 x 6
// 51.1 us, 1 x 12 54.0 us, and in an interleaved A/B of 4 x 3 against 2 x 6:
// M = 2048 22.5 / 26.3 us, 4096 39.3 / 42.4, 4608 43.4 / 45.4, 16384 142.1 /
// 144.1 (K = 9216: 3 x 3 against 2 x 5, 3-8% faster).  One workgroup per row
// (below).
// Rows of 13 to 32 passes (K in (12288, 32768]): 8 waves of 2 or 3 passes, or
// 16 waves of 2, on the 16-wave instance (8.7 KB of LDS per wave, so one
// 16-wave or two 8-wave workgroups fill a CU's 16 wave slots).
template <int DT, int G, int P, int OUT, bool LR>
static hipError_t rq_wide_launch(const void* x, int8_t* q, float* s, int M, int K, int W, hipStream_t st,
                                 const LoraSum& ls) {
    static std::atomic<bool> attr_set[kMaxDev];
    void (*kern)(const void*, int8_t*, float*, int, int, LoraSum) =
        rotquant_row_kernel<DT, G, P, OUT, LR, kRowWideWaves>;
    int dev = 0;
    hipError_t e = current_device(&dev);
    if (e != hipSuccess) return e;
    e = lds_limit_once(attr_set, dev, reinterpret_cast<const void*>(kern),
                       kRowWideWaves * kRowWaveLds + 32 * (int)sizeof(float));
    if (e != hipSuccess) return e;
    const size_t lds = (size_t)W * kRowWaveLds + 32 * sizeof(float);
    hipLaunchKernelGGL(kern, dim3(M), dim3(64 * W), lds, st, x, q, s, M, K, ls);
    return hipGetLastError();
}

template <int DT, int G, int OUT, bool LR = false>
static hipError_t rq_row_launch(const void* x, int8_t* q, float* s, int M, int K, hipStream_t st,
                                const LoraSum& ls = LoraSum{}) {
    if (M <= 0) return hipSuccess;
    const int np = (K / kChunk + 63) / 64;
    if (np > 3 * kRowMaxWaves) {
        if (np > 2 * kRowWideWaves) return hipErrorInvalidValue;
        if (np <= 16) return rq_wide_launch<DT, G, 2, OUT, LR>(x, q, s, M, K, 8, st, ls);
        if (np <= 24) return rq_wide_launch<DT, G, 3, OUT, LR>(x, q, s, M, K, 8, st, ls);
        return rq_wide_launch<DT, G, 2, OUT, LR>(x, q, s, M, K, 16, st, ls);
    }
    int W, P;
    if (np <= 2 * kRowMaxWaves) {
        P = np <= kRowMaxWaves ? np : (np % 3 != 0 ? 2 : 3);
        if (P == 4) P = 6;                // 4-pass rows: the 6-pass kernel, its last two passes idle
        W = (np + P - 1) / P;
        P = (np + W - 1) / W;
        if (P == 4 || P == 5) P = 6;
    } else {                              // np = 9..12: 3 passes per wave
        W = kRowMaxWaves;
        P = (np + W - 1) / W;
        W = (np + P - 1) / P;
    }
    // Few rows (under two waves per SIMD of the 1024 on MI355X): spread each
    // row over up to 4 waves, so that a row's passes run side by side instead
    // of one after another.
    if ((long long)M * W < 2048 && W < kRowMaxWaves && W < np) {
        W = np < kRowMaxWaves ? np : kRowMaxWaves;
        P = (np + W - 1) / W;
        W = (np + P - 1) / P;
        if (P == 4 || P == 5) P = 6;
    }
    if (W > kRowMaxWaves || P > kRowMaxPass) return hipErrorInvalidValue;
    const size_t lds = (size_t)W * kRowWaveLds + 16 * sizeof(float);
    void (*kern)(const void*, int8_t*, float*, int, int, LoraSum) =
        P == 1 ? rotquant_row_kernel<DT, G, 1, OUT, LR> : P == 2 ? rotquant_row_kernel<DT, G, 2, OUT, LR>
        : P == 3 ? rotquant_row_kernel<DT, G, 3, OUT, LR> : rotquant_row_kernel<DT, G, 6, OUT, LR>;   // 5..6 passes: 6
    // One row per workgroup: the hardware queues the surplus behind the
    // resident workgroups, which beat persistent workgroups walking several
    // rows (A/B on MI355X, HIP events, bf16 -> B6T, 4 interleaved rounds:
    // 16384 x 3072 38.3-42.5 us against 41.1-45.0 with 4 rows per workgroup;
    // 4608 x 12288 45.4-51.5 against 48.0-54.3 with 3; 16384 x 12288
    // 140.9-153.9 against 153.3-201.4 with 11; 4608 x 3072 runs one row per
    // workgroup either way, 16.8-17.4 us).
    const int grid = M;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * W), lds, st, x, q, s, M, K, ls);
    return hipGetLastError();
}

constexpr int kRowMaxK = 2 * kRowWideWaves * 64 * kChunk;   // 32768: 16 waves x 2 passes

// ---------------------------------------------------------------------------
// host-side launch
// ---------------------------------------------------------------------------

struct RQPlan { int npass, tpr, rows_per_wg, grid, block; };

static inline int rq_plan(int M, int K, int G, RQPlan* pl) {
    const int lpg = G / kChunk;
    const int nchunks = K / kChunk;
    int npass = (nchunks + kMaxThreads - 1) / kMaxThreads;
    if (npass < 1) npass = 1;
    int tpr = (nchunks + npass - 1) / npass;
    tpr = ((tpr + lpg - 1) / lpg) * lpg;
    if (tpr > kMaxThreads) return -1;
    int rpw = (npass == 1) ? kMaxThreads / tpr : 1;
    if (rpw < 1) rpw = 1;
    if (rpw > M) rpw = M > 0 ? M : 1;
    pl->npass = npass; pl->tpr = tpr; pl->rows_per_wg = rpw;
    pl->grid = (M + rpw - 1) / rpw;
    pl->block = rpw * tpr;
    return 0;
}

template <int DT, int G, bool STOCH, bool I8 = false>
static hipError_t rq_launch_g(const void* x, const void* noise, int8_t* q, float* s, int M, int K,
                              hipStream_t st) {
    if (M == 0) return hipSuccess;
    if (!STOCH && K <= kRowMaxK) return rq_row_launch<DT, G, I8 ? OUT_I8 : OUT_PACK4>(x, q, s, M, K, st);
    RQPlan pl;
    if (rq_plan(M, K, G, &pl) != 0) return hipErrorInvalidValue;
    dim3 grid(pl.grid), block(pl.block);
#define RQ_CASE(NP)                                                                              \
    case NP:                                                                                     \
        hipLaunchKernelGGL((rotquant_kernel<DT, G, NP, STOCH, I8>), grid, block, 0, st, x, noise, q, s, \
                           M, K, pl.tpr, pl.rows_per_wg);                                        \
        break;
    switch (pl.npass) {
        RQ_CASE(1) RQ_CASE(2) RQ_CASE(3) RQ_CASE(4) RQ_CASE(5) RQ_CASE(6) RQ_CASE(7) RQ_CASE(8)
        default: return hipErrorInvalidValue;
    }
#undef RQ_CASE
    return hipGetLastError();
}

template <int DT, bool STOCH>
static hipError_t rq_launch_dt(const void* x, const void* noise, int8_t* q, float* s, int M, int K, int G,
                               hipStream_t st) {
    switch (G) {
        case 16: return rq_launch_g<DT, 16, STOCH>(x, noise, q, s, M, K, st);
        case 64: return rq_launch_g<DT, 64, STOCH>(x, noise, q, s, M, K, st);
        case 256: return rq_launch_g<DT, 256, STOCH>(x, noise, q, s, M, K, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t rotquant_launch(const void* x, int in_dtype, const void* noise, int8_t* q, float* s,
                           int M, int K, int G, hipStream_t st) {
    const bool stoch = noise != nullptr;
    switch (in_dtype) {
        case DT_F32: return stoch ? rq_launch_dt<DT_F32, true>(x, noise, q, s, M, K, G, st)
                                  : rq_launch_dt<DT_F32, false>(x, noise, q, s, M, K, G, st);
        case DT_BF16: return stoch ? rq_launch_dt<DT_BF16, true>(x, noise, q, s, M, K, G, st)
                                   : rq_launch_dt<DT_BF16, false>(x, noise, q, s, M, K, G, st);
        case DT_F16: return stoch ? rq_launch_dt<DT_F16, true>(x, noise, q, s, M, K, G, st)
                                  : rq_launch_dt<DT_F16, false>(x, noise, q, s, M, K, G, st);
        default: return hipErrorInvalidValue;
    }
}

int rotquant_max_k() { return 8 * kMaxThreads * kChunk; }

// fused rotate + quantize into the B6T layout (K % 128 == 0, K <= 32768)
// With `ls` (not null) the kernel also sums the LoRA partials of every row into ls->t.
hipError_t rotquant_b6_launch(const void* x, int in_dtype, uint8_t* a6, float* s, int M, int K, int G,
                              hipStream_t st, const LoraSum* ls) {
    if (K % 128 != 0 || K > kRowMaxK || M < 0) return hipErrorInvalidValue;
    if (ls != nullptr && (ls->S < 1 || ls->S > 8 || ls->R < 1 || ls->part == nullptr || ls->t == nullptr))
        return hipErrorInvalidValue;
    int8_t* q = reinterpret_cast<int8_t*>(a6);
#define RB6_G(DT)                                                                                   \
    switch (G) {                                                                                    \
        case 16: return ls ? rq_row_launch<DT, 16, OUT_B6T, true>(x, q, s, M, K, st, *ls)          \
                           : rq_row_launch<DT, 16, OUT_B6T>(x, q, s, M, K, st);                    \
        case 64: return ls ? rq_row_launch<DT, 64, OUT_B6T, true>(x, q, s, M, K, st, *ls)          \
                           : rq_row_launch<DT, 64, OUT_B6T>(x, q, s, M, K, st);                    \
        case 256: return ls ? rq_row_launch<DT, 256, OUT_B6T, true>(x, q, s, M, K, st, *ls)        \
                            : rq_row_launch<DT, 256, OUT_B6T>(x, q, s, M, K, st);                  \
        default: return hipErrorInvalidValue;                                                       \
    }
    switch (in_dtype) {
        case DT_F32: RB6_G(DT_F32)
        case DT_BF16: RB6_G(DT_BF16)
        case DT_F16: RB6_G(DT_F16)
        default: return hipErrorInvalidValue;
    }
#undef RB6_G
}

int rotquant_b6_max_k() { return kRowMaxK; }

// fused rotate + int8 quantize into the I8T layout (K % 64 == 0, K <= 32768)
hipError_t rotquant_i8t_launch(const void* x, int in_dtype, int8_t* q, float* s, int M, int K, int G,
                               hipStream_t st) {
    if (K % 64 != 0 || K > kRowMaxK || M < 0) return hipErrorInvalidValue;
#define RI8T_G(DT)                                                                                  \
    switch (G) {                                                                                    \
        case 16: return rq_row_launch<DT, 16, OUT_I8T>(x, q, s, M, K, st);                         \
        case 64: return rq_row_launch<DT, 64, OUT_I8T>(x, q, s, M, K, st);                         \
        case 256: return rq_row_launch<DT, 256, OUT_I8T>(x, q, s, M, K, st);                       \
        default: return hipErrorInvalidValue;                                                       \
    }
    switch (in_dtype) {
        case DT_F32: RI8T_G(DT_F32)
        case DT_BF16: RI8T_G(DT_BF16)
        case DT_F16: RI8T_G(DT_F16)
        default: return hipErrorInvalidValue;
    }
#undef RI8T_G
}

// fused rotate + int8 quantize (W8A8 activations / weights): plain int8 [M, K]
hipError_t rotquant_i8_launch(const void* x, int in_dtype, int8_t* q, float* s, int M, int K, int G,
                              hipStream_t st) {
#define RI8_G(DT)                                                                                   \
    switch (G) {                                                                                    \
        case 16: return rq_launch_g<DT, 16, false, true>(x, nullptr, q, s, M, K, st);               \
        case 64: return rq_launch_g<DT, 64, false, true>(x, nullptr, q, s, M, K, st);               \
        case 256: return rq_launch_g<DT, 256, false, true>(x, nullptr, q, s, M, K, st);             \
        default: return hipErrorInvalidValue;                                                       \
    }
    switch (in_dtype) {
        case DT_F32: RI8_G(DT_F32)
        case DT_BF16: RI8_G(DT_BF16)
        case DT_F16: RI8_G(DT_F16)
        default: return hipErrorInvalidValue;
    }
#undef RI8_G
}

}  // namespace convrot
