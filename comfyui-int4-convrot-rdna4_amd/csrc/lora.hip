// Low-rank "down" projection of the dynamic-LoRA side path (gfx950):
//   t[m, r] = bf16( sum_k x[m, k] * D[r, k] )      x [M, K] bf16/f16, D [R, K] bf16
// The "up" half, scale * t @ U^T, runs inside the W4A4 GEMM epilogue (gemm.hip)
// on the same 32x32 accumulator layout, so the side path costs one extra read
// of x here plus R/16 bf16 MFMAs per 32x32 output tile there.
//
// Reference behaviour being fused: Int4ConvRotOps.Linear._apply_dyn_lora
// (int4_ops.py:181-192) adds, per attached adapter v, v.h(x, out) =
// multiplier * (alpha / rank) * (x @ down^T) @ up^T (ComfyUI's LoRA bypass).
// Several adapters are one LoRA whose D / U are the concatenation of theirs
// along the rank (the per-adapter scales folded into U on the host).
//
// Work layout: one workgroup (4 waves) per 32 rows; wave w accumulates the
// k-quarter w of every 32x32 (rows x rank) tile with v_mfma_f32_32x32x16_bf16,
// the quarters are summed through LDS and wave 0 stores the bf16 result.

#include "common.h"

namespace convrot {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

template <int DT>
__device__ __forceinline__ bf16x8_t load8_as_bf16(const void* __restrict__ p, size_t elem) {
    if constexpr (DT == DT_BF16) {
        return *reinterpret_cast<const bf16x8_t*>(reinterpret_cast<const uint16_t*>(p) + elem);
    } else {
        const uint4 w = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p) + elem);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
        bf16x8_t o;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            o[2 * i] = (__bf16)f16bits_to_f32(ws[i]);
            o[2 * i + 1] = (__bf16)f16bits_to_f32(ws[i] >> 16);
        }
        return o;
    }
}

template <int DT, int RT>
__global__ __launch_bounds__(256) void lora_down_kernel(const void* __restrict__ x, const __bf16* __restrict__ D,
                                                        __bf16* __restrict__ t, int M, int K) {
    __shared__ float red[3][RT][16][64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row0 = blockIdx.x * 32;
    const int row = row0 + (lane & 31);
    const int half = lane >> 5;
    const int nsteps = K / 16;
    const int s0 = (nsteps * wave) / 4, s1 = (nsteps * (wave + 1)) / 4;

    f32x16_t acc[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) acc[r] = (f32x16_t){0};
    const bool row_ok = row < M;
#pragma unroll 4
    for (int s = s0; s < s1; ++s) {
        const int k = s * 16 + 8 * half;                 // same k slice for A and B lanes
        bf16x8_t a = row_ok ? load8_as_bf16<DT>(x, (size_t)row * K + k) : (bf16x8_t){0};
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const bf16x8_t b = *reinterpret_cast<const bf16x8_t*>(D + (size_t)(r * 32 + (lane & 31)) * K + k);
            acc[r] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[r], 0, 0, 0);
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
            for (int e = 0; e < 16; ++e) red[wave - 1][r][e][lane] = acc[r][e];
    }
    __syncthreads();
    if (wave == 0) {
        const int R = RT * 32;
#pragma unroll
        for (int r = 0; r < RT; ++r) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float v = (acc[r][e] + red[0][r][e][lane]) + (red[1][r][e][lane] + red[2][r][e][lane]);
                const int orow = row0 + 8 * (e >> 2) + 4 * half + (e & 3);   // 32x32 accumulator layout
                if (orow < M) t[(size_t)orow * R + r * 32 + (lane & 31)] = (__bf16)v;
            }
        }
    }
}

hipError_t lora_down_launch(const void* x, int in_dtype, const void* D, void* t, int M, int K, int R,
                            hipStream_t st) {
    if (M == 0) return hipSuccess;
    dim3 grid((M + 31) / 32), block(256);
    const __bf16* d = reinterpret_cast<const __bf16*>(D);
    __bf16* o = reinterpret_cast<__bf16*>(t);
#define LD_CASE(RT)                                                                                     \
    case RT:                                                                                            \
        if (in_dtype == DT_BF16)                                                                        \
            hipLaunchKernelGGL((lora_down_kernel<DT_BF16, RT>), grid, block, 0, st, x, d, o, M, K);     \
        else                                                                                            \
            hipLaunchKernelGGL((lora_down_kernel<DT_F16, RT>), grid, block, 0, st, x, d, o, M, K);      \
        break;
    switch (R / 32) {
        LD_CASE(1) LD_CASE(2) LD_CASE(3) LD_CASE(4)
        default: return hipErrorInvalidValue;
    }
#undef LD_CASE
    return hipGetLastError();
}

}  // namespace convrot
