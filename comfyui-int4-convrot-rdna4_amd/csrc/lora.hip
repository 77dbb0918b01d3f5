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
// Work layout: one 512-lane workgroup per 16 rows of x (M = 4096 gives 256
// workgroups) over the whole of K, so no partial sums leave the workgroup.
// Every workgroup needs all of D (R x K bf16), which makes D, read from L2,
// the larger part of its traffic; both operands are therefore staged in LDS by
// the global->LDS DMA (one contiguous row chunk per instruction), the fastest
// path from L2 and HBM into a CU.  A stage holds KC k of the 16 x rows and the
// R D rows (row stride KC*2 + 16 bytes, so the fragment reads below hit 64
// distinct banks); a ring of three stages (two for R > 64) keeps two blocks in
// flight while one is consumed.  In a stage the 8 waves take
// different 32-k steps and accumulate 16 x R (rows x rank) with
// v_mfma_f32_16x16x32_bf16; the eight partial sums meet in LDS and are added
// in a fixed order (deterministic) before the bf16 store.

#include "gemm_common.h"

namespace convrot {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int LD_ROWS = 16;
constexpr int LD_WAVES = 8;

template <int CT> struct LoraDownCfg {
    static constexpr int R = CT * 16;
    static constexpr int KC = CT <= 2 ? 512 : 256;          // k per stage
    static constexpr int RB = KC * 2;                       // bytes of a row chunk (one DMA instruction)
    static constexpr int RS = RB + 16;                      // LDS row stride
    static constexpr int ROWS = LD_ROWS + R;                // x rows then D rows
    static constexpr int STAGE = ROWS * RS;
    static constexpr int LOADS = ROWS / LD_WAVES;           // DMA instructions per wave and stage
    static constexpr int NST = 3 * STAGE <= 160 * 1024 ? 3 : 2;   // stages in the ring
    static constexpr int RED = LD_WAVES * CT * 64 * 16;     // partial sums of the 8 waves
    static constexpr int LDS = NST * STAGE > RED ? NST * STAGE : RED;
    static_assert(ROWS % LD_WAVES == 0 && (NST - 2) * LOADS <= 63, "DMA split");
    static_assert(NST * STAGE <= 160 * 1024, "LDS");
};

template <int DT>
__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 w) {
    if constexpr (DT == DT_BF16) {
        return __builtin_bit_cast(bf16x8_t, w);
    } else {
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

template <int DT, int CT>
__global__ __launch_bounds__(64 * LD_WAVES) void lora_down_kernel(const void* __restrict__ x, const __bf16* __restrict__ D,
                                                                  __bf16* __restrict__ t, int M, int K) {
    using C = LoraDownCfg<CT>;
    extern __shared__ __attribute__((aligned(16))) uint8_t ldsl[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row0 = blockIdx.x * LD_ROWS;
    const int nkb = (K + C::KC - 1) / C::KC;

    // DMA: wave w copies stage rows w, w + 8, ...; lane l the 16 bytes at l * 16
    // of the row's chunk (lanes past the chunk or past K stay idle).  x rows past
    // M re-read row M - 1: they only feed output rows that are never stored.
    auto issue = [&](int kb) {
        const uint32_t st = (uint32_t)(uintptr_t)ldsl + (kb % C::NST) * C::STAGE;
        const int k = kb * C::KC + lane * 8;
        if (lane * 16 < C::RB && k < K) {
#pragma unroll
            for (int j = 0; j < C::LOADS; ++j) {
                const int r = wave + j * LD_WAVES;
                const uint16_t* src = r < LD_ROWS
                        ? reinterpret_cast<const uint16_t*>(x) + (size_t)min(row0 + r, M - 1) * K + k
                        : reinterpret_cast<const uint16_t*>(D) + (size_t)(r - LD_ROWS) * K + k;
                dma16(st + r * C::RS, src);
            }
        }
    };

    const int r16 = lane & 15;
    const int kq = (lane >> 4) * 8;                     // this lane's 8 k of each 32-k step (same for x and D)
    f32x4_t acc[CT];
#pragma unroll
    for (int c = 0; c < CT; ++c) acc[c] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    constexpr int STEPS = C::KC / 32;                   // 32-k steps per stage
    constexpr int SPW = STEPS / LD_WAVES;               // per wave (1 or 2)

    // Block kb lives in stage kb % NST.  Iteration kb: wait for block kb (exact
    // vmcnt: the blocks issued after it are still counted), one barrier (every
    // wave's copy of block kb has landed and every wave has finished block
    // kb - 1), refill the stage of block kb - 1 with block kb + NST - 1, compute.
    for (int j = 0; j < C::NST - 1 && j < nkb; ++j) issue(j);
    for (int kb = 0; kb < nkb; ++kb) {
        wait_block_landed<C::NST - 2, C::LOADS>(min(C::NST - 2, nkb - 1 - kb));
        __syncthreads();
        if (kb + C::NST - 1 < nkb) issue(kb + C::NST - 1);
        const uint8_t* st = ldsl + (kb % C::NST) * C::STAGE;
#pragma unroll
        for (int u = 0; u < SPW; ++u) {
            const int s = wave * SPW + u;
            const int kin = s * 32 + kq;                          // k inside the stage
            const bool kok = kb * C::KC + kin < K;                // K % 16 == 0: whole 8-k pieces
            const uint4 araw = *reinterpret_cast<const uint4*>(st + r16 * C::RS + kin * 2);
            const bf16x8_t a = kok ? as_bf16x8<DT>(araw) : (bf16x8_t){0};
#pragma unroll
            for (int c = 0; c < CT; ++c) {
                // past K the stage holds stale bytes (possibly NaN patterns): zero both operands
                const uint4 braw = *reinterpret_cast<const uint4*>(st + (LD_ROWS + c * 16 + r16) * C::RS + kin * 2);
                const bf16x8_t b = kok ? __builtin_bit_cast(bf16x8_t, braw) : (bf16x8_t){0};
                acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[c], 0, 0, 0);
            }
        }
    }
    __syncthreads();                                              // every wave is done with the stages

    f32x4_t* red = reinterpret_cast<f32x4_t*>(ldsl);               // [wave][c][lane]; the stages are free now
#pragma unroll
    for (int c = 0; c < CT; ++c) red[(wave * CT + c) * 64 + lane] = acc[c];
    __syncthreads();

    // output (i, j): row i of the tile, rank column j; the 16x16 accumulator of
    // column tile c = j / 16 holds it in lane (i / 4) * 16 + j % 16, element i % 4
    for (int o = threadIdx.x; o < LD_ROWS * C::R; o += 64 * LD_WAVES) {
        const int i = o / C::R, j = o - i * C::R;
        const int c = j >> 4, l = (i >> 2) * 16 + (j & 15), e = i & 3;
        const float* base = reinterpret_cast<const float*>(red + c * 64 + l) + e;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < LD_WAVES; ++w) v += base[w * CT * 64 * 4];
        if (row0 + i < M) t[(size_t)(row0 + i) * C::R + j] = (__bf16)v;
    }
}

template <int DT, int CT>
static hipError_t launch_lora_down(const void* x, const __bf16* d, __bf16* o, int M, int K, hipStream_t st) {
    static std::atomic<bool> attr_set[kMaxDev];
    int dev = 0;
    hipError_t e = current_device(&dev);
    if (e != hipSuccess) return e;
    e = lds_limit_once(attr_set, dev, reinterpret_cast<const void*>(&lora_down_kernel<DT, CT>),
                       LoraDownCfg<CT>::LDS);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((lora_down_kernel<DT, CT>), dim3((M + LD_ROWS - 1) / LD_ROWS), dim3(64 * LD_WAVES),
                       LoraDownCfg<CT>::LDS, st, x, d, o, M, K);
    return hipGetLastError();
}

hipError_t lora_down_launch(const void* x, int in_dtype, const void* D, void* t, int M, int K, int R,
                            hipStream_t st) {
    if (M == 0) return hipSuccess;
    const __bf16* d = reinterpret_cast<const __bf16*>(D);
    __bf16* o = reinterpret_cast<__bf16*>(t);
    const bool bf = in_dtype == DT_BF16;
    switch (R / 32) {
        case 1: return bf ? launch_lora_down<DT_BF16, 2>(x, d, o, M, K, st) : launch_lora_down<DT_F16, 2>(x, d, o, M, K, st);
        case 2: return bf ? launch_lora_down<DT_BF16, 4>(x, d, o, M, K, st) : launch_lora_down<DT_F16, 4>(x, d, o, M, K, st);
        case 3: return bf ? launch_lora_down<DT_BF16, 6>(x, d, o, M, K, st) : launch_lora_down<DT_F16, 6>(x, d, o, M, K, st);
        case 4: return bf ? launch_lora_down<DT_BF16, 8>(x, d, o, M, K, st) : launch_lora_down<DT_F16, 8>(x, d, o, M, K, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace convrot
