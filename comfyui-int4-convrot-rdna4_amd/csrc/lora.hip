// Low-rank "down" projection of the dynamic-LoRA side path (gfx950):
//   t[m, r] = bf16( sum_k x[m, k] * D[r, k] )      x [M, K] bf16/f16, D [R, K] bf16
// The "up" half, scale * t @ U^T, runs inside the W4A4 GEMM epilogue on the
// GEMM's own accumulator layout, so the side path costs one extra read of x
// here plus R/16 bf16 MFMAs per 32x32 output tile there.
//
// Reference behaviour being fused: Int4ConvRotOps.Linear._apply_dyn_lora
// (int4_ops.py:181-192) adds, per attached adapter v, v.h(x, out) =
// multiplier * (alpha / rank) * (x @ down^T) @ up^T (ComfyUI's LoRA bypass).
// Several adapters are one LoRA whose D / U are the concatenation of theirs
// along the rank (the per-adapter scales folded into U on the host).
//
// Work split.  Every workgroup that covers XR rows of x over a k range reads
// those rows and the same k range of all of D, so D's share of the bytes a CU
// pulls from L2 is R / (XR + R).  lora_plan picks, per shape: XR = 64 rows
// and S k ranges for large M and long rows (the image stream's K = 12288:
// 64 x 4 workgroups), 16 rows over the whole of K for large M and short rows
// (one workgroup per 16 rows already fills the chip), and 16 rows over S k
// ranges for small M (the text stream's M = 512: 32 x 8 workgroups).  With one
// k range the kernel writes t itself (the f32 sum of its 8 waves, rounded
// once).  With S > 1 each workgroup writes its f32 partial sums part[s, m, r]
// (plain stores, no atomics); they are summed in the fixed order s = 0, 1, ..,
// S-1 and rounded once to bf16 by whoever reads them next: the rotate+quant
// kernel of the linear (which walks every row anyway, rotquant.hip) or
// lora_reduce_kernel for the standalone call.  Both add in the same order, so
// the two give the same t bit for bit, and t does not depend on the device.
// (Measured on MI355X, R = 32, x from HBM, HIP events per launch: M = 4096,
// K = 3072: 16 rows x 1 range 11.0 us, 64 x 4 12.0 us; K = 12288: 64 x 4 24.0
// us, 16 x 1 28.0 us; M = 512, K = 12288: 16 x 8 9.6 us.)
//
// Inside a workgroup both operands are staged in LDS by the global->LDS DMA
// (one contiguous row chunk per instruction: 1 KB for KC = 512 k per stage,
// 512 B for KC = 256; the full-width copies move more bytes per instruction).
// A stage holds KC k of the XR x rows and the R D rows (row stride KC*2 + 16
// bytes, so the fragment reads below hit distinct banks); a ring of up to
// three stages keeps blocks in flight while one is consumed.  The 8 waves take
// different 32-k steps of a stage (KC / 256 each) and accumulate XR x R with
// v_mfma_f32_16x16x32_bf16; their partial sums meet in LDS and are added in a
// fixed order (deterministic).

#include "gemm_common.h"

namespace convrot {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int LD_WAVES = 8;
constexpr int LD_MAX_SPLITS = 8;           // the rotate+quant kernel holds up to 8 partials per rank column
constexpr int LD_TARGET_WGS = 256;

template <int CT, int XR, int KC_> struct LoraDownCfg {
    static constexpr int KC = KC_;                          // k per stage: 256 or 512
    static constexpr int SPW = KC / 256;                    // 32-k steps per wave and stage
    static constexpr int R = CT * 16;
    static constexpr int RF = XR / 16;                      // 16-row fragments of x
    static constexpr int RB = KC * 2;                       // bytes of a row chunk (one DMA instruction)
    static constexpr int RS = RB + 16;                      // LDS row stride
    static constexpr int ROWS = XR + R;                     // x rows then D rows
    static constexpr int STAGE = ROWS * RS;
    static constexpr int LOADS = ROWS / LD_WAVES;           // DMA instructions per wave and stage
    static constexpr int NST = 3 * STAGE <= 160 * 1024 ? 3 : 2;   // stages in the ring
    static constexpr int RED = LD_WAVES * RF * CT * 64 * 16;      // partial sums of the 8 waves
    static constexpr int LDS = NST * STAGE > RED ? NST * STAGE : RED;
    static_assert(ROWS % LD_WAVES == 0 && (NST - 2) * LOADS <= 63, "DMA split");
    static_assert(NST * STAGE <= 160 * 1024 && RED <= 160 * 1024, "LDS");
};

// Rows per workgroup, k splits and k per split for an [M, K] x and rank R.  A
// pure function of the shape: t must not depend on the device it runs on.
LoraPlan lora_plan(int M, int K, int R) {
    LoraPlan p{};
    const bool big = M >= 1024;
    p.xr = (big && R <= 64 && (K > 4096 || R > 32)) ? 64 : 16;
    int s = 1;
    if (!big || p.xr == 64) {
        const int blocks = (M + p.xr - 1) / p.xr;
        s = (LD_TARGET_WGS + blocks / 2) / blocks;
        const int smax = K / 256 > 1 ? K / 256 : 1;          // a split covers at least 256 k
        s = s < 1 ? 1 : s > LD_MAX_SPLITS ? LD_MAX_SPLITS : s;
        s = s > smax ? smax : s;
    }
    const int steps = (K + 31) / 32;
    p.krange = (steps + s - 1) / s * 32;
    p.splits = (K + p.krange - 1) / p.krange;               // no empty split
    return p;
}

// k per stage of the plan's kernel: full 1 KB row chunks where the ring of
// three stages fits (rank 32 with 16 rows), else 512-byte chunks
static int lora_kc(const LoraPlan& p, int R) { return (p.xr == 16 && R == 32) ? 512 : 256; }

size_t lora_part_bytes(int M, int K, int R) {
    const LoraPlan p = lora_plan(M, K, R);
    return p.splits > 1 ? (size_t)p.splits * (size_t)M * (size_t)R * sizeof(float) : 0;
}

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

// grid (ceil(M / XR), S): workgroup (b, s) sums k in [s * krange, min(K, (s +
// 1) * krange)) for rows b*XR .. +XR-1 into part[s, row, 0..R-1] (f32), or, with
// t given (S = 1), into t[row, 0..R-1] rounded once to bf16.
template <int DT, int CT, int XR, int KC>
__global__ __launch_bounds__(64 * LD_WAVES) void lora_part_kernel(const void* __restrict__ x,
                                                                  const __bf16* __restrict__ D,
                                                                  float* __restrict__ part, __bf16* __restrict__ t,
                                                                  int M, int K, int krange) {
    using C = LoraDownCfg<CT, XR, KC>;
    extern __shared__ __attribute__((aligned(16))) uint8_t ldsl[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row0 = blockIdx.x * XR;
    const int split = blockIdx.y;
    const int k0 = split * krange;                               // < K: lora_plan leaves no empty split
    const int k1 = min(K, k0 + krange);
    const int nkb = (k1 - k0 + C::KC - 1) / C::KC;

    // DMA: wave w copies stage rows w, w + 8, ...; lane l the 16 bytes at l * 16
    // of the row's chunk (lanes past the chunk or past the k range stay idle;
    // lane 0 never does, so every wave issues LOADS instructions per block).
    // x rows past M re-read row M - 1: they only feed partial sums never stored.
    auto issue = [&](int kb) {
        const uint32_t st = (uint32_t)(uintptr_t)ldsl + (kb % C::NST) * C::STAGE;
        const int k = k0 + kb * C::KC + lane * 8;
        if (lane * 16 < C::RB && k < k1) {
#pragma unroll
            for (int j = 0; j < C::LOADS; ++j) {
                const int r = wave + j * LD_WAVES;
                const uint16_t* src = r < XR
                        ? reinterpret_cast<const uint16_t*>(x) + (size_t)min(row0 + r, M - 1) * K + k
                        : reinterpret_cast<const uint16_t*>(D) + (size_t)(r - XR) * K + k;
                dma16(st + r * C::RS, src);
            }
        }
    };

    const int r16 = lane & 15;
    const int kq = (lane >> 4) * 8;                     // this lane's 8 k of the wave's 32-k step (x and D alike)
    f32x4_t acc[C::RF][CT];
#pragma unroll
    for (int f = 0; f < C::RF; ++f)
#pragma unroll
        for (int c = 0; c < CT; ++c) acc[f][c] = (f32x4_t){0.f, 0.f, 0.f, 0.f};

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
        for (int u = 0; u < C::SPW; ++u) {
            const int kin = (wave * C::SPW + u) * 32 + kq;           // k inside the stage
            // past the k range the stage holds stale bytes (possibly NaN patterns):
            // zero both operands (k1 % 8 == 0, so 8-k pieces are wholly in or out)
            const bool kok = k0 + kb * C::KC + kin < k1;
            bf16x8_t b[CT];
#pragma unroll
            for (int c = 0; c < CT; ++c) {
                const uint4 braw = *reinterpret_cast<const uint4*>(st + (XR + c * 16 + r16) * C::RS + kin * 2);
                b[c] = kok ? __builtin_bit_cast(bf16x8_t, braw) : (bf16x8_t){0};
            }
#pragma unroll
            for (int f = 0; f < C::RF; ++f) {
                const uint4 araw = *reinterpret_cast<const uint4*>(st + (f * 16 + r16) * C::RS + kin * 2);
                const bf16x8_t a = kok ? as_bf16x8<DT>(araw) : (bf16x8_t){0};
#pragma unroll
                for (int c = 0; c < CT; ++c)
                    acc[f][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[c], acc[f][c], 0, 0, 0);
            }
        }
    }
    __syncthreads();                                              // every wave is done with the stages

    f32x4_t* red = reinterpret_cast<f32x4_t*>(ldsl);               // [wave][f][c][lane]; the stages are free now
#pragma unroll
    for (int f = 0; f < C::RF; ++f)
#pragma unroll
        for (int c = 0; c < CT; ++c) red[((wave * C::RF + f) * CT + c) * 64 + lane] = acc[f][c];
    __syncthreads();

    // output (i, j): row i of the workgroup's XR, rank column j; fragment f = i / 16
    // and column tile c = j / 16 hold it in lane ((i % 16) / 4) * 16 + j % 16,
    // element i % 4
    for (int o = threadIdx.x; o < XR * C::R; o += 64 * LD_WAVES) {
        const int i = o / C::R, j = o - i * C::R;
        const int f = i >> 4, c = j >> 4, l = ((i & 15) >> 2) * 16 + (j & 15), e = i & 3;
        const float* base = reinterpret_cast<const float*>(red + (f * CT + c) * 64 + l) + e;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < LD_WAVES; ++w) v += base[w * C::RF * CT * 64 * 4];
        if (row0 + i >= M) continue;
        const size_t o2 = (size_t)(row0 + i) * C::R + j;
        if (t != nullptr) t[o2] = (__bf16)v;
        else part[(size_t)split * M * C::R + o2] = v;
    }
}

// t[m, r] = bf16(sum_s part[s, m, r]) in the order s = 0 .. S-1 (the same sum
// as the rotate+quant kernel's, lora_reduce_row)
__global__ __launch_bounds__(256) void lora_reduce_kernel(const float* __restrict__ part, __bf16* __restrict__ t,
                                                          int M, int R, int S) {
    const size_t n = (size_t)M * R;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        float v = 0.f;
        for (int s = 0; s < S; ++s) v += part[(size_t)s * n + i];
        t[i] = (__bf16)v;
    }
}

template <int DT, int CT, int XR, int KC>
static hipError_t launch_lora_part(const void* x, const __bf16* d, float* part, __bf16* t, int M, int K,
                                   const LoraPlan& p, hipStream_t st) {
    using C = LoraDownCfg<CT, XR, KC>;
    static std::atomic<bool> attr_set[kMaxDev];
    int dev = 0;
    hipError_t e = current_device(&dev);
    if (e != hipSuccess) return e;
    e = lds_limit_once(attr_set, dev, reinterpret_cast<const void*>(&lora_part_kernel<DT, CT, XR, KC>), C::LDS);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((lora_part_kernel<DT, CT, XR, KC>), dim3((M + XR - 1) / XR, p.splits), dim3(64 * LD_WAVES),
                       (C::LDS), st, x, d, part, t, M, K, p.krange);
    return hipGetLastError();
}

template <int DT, int CT>
static hipError_t launch_lora_part_ct(const void* x, const __bf16* d, float* part, __bf16* t, int M, int K,
                                      const LoraPlan& p, hipStream_t st) {
    if constexpr (CT <= 4) {
        if (p.xr == 64) return launch_lora_part<DT, CT, 64, 256>(x, d, part, t, M, K, p, st);
    }
    if constexpr (CT == 2) {
        if (lora_kc(p, 32) == 512) return launch_lora_part<DT, CT, 16, 512>(x, d, part, t, M, K, p, st);
    }
    return launch_lora_part<DT, CT, 16, 256>(x, d, part, t, M, K, p, st);
}

// The split projection's first launch: f32 partials into `part`
// (lora_part_bytes(M, K, R) bytes) when the plan has several k ranges, else t
// itself.  Returns the plan's split count in *splits.
hipError_t lora_part_launch(const void* x, int in_dtype, const void* D, float* part, void* t, int M, int K, int R,
                            int* splits, hipStream_t st) {
    const LoraPlan p = lora_plan(M, K, R);
    *splits = p.splits;
    if (M == 0) return hipSuccess;
    const __bf16* d = reinterpret_cast<const __bf16*>(D);
    __bf16* tt = p.splits == 1 ? reinterpret_cast<__bf16*>(t) : nullptr;
    const bool bf = in_dtype == DT_BF16;
    switch (R / 32) {
        case 1: return bf ? launch_lora_part_ct<DT_BF16, 2>(x, d, part, tt, M, K, p, st) : launch_lora_part_ct<DT_F16, 2>(x, d, part, tt, M, K, p, st);
        case 2: return bf ? launch_lora_part_ct<DT_BF16, 4>(x, d, part, tt, M, K, p, st) : launch_lora_part_ct<DT_F16, 4>(x, d, part, tt, M, K, p, st);
        case 3: return bf ? launch_lora_part_ct<DT_BF16, 6>(x, d, part, tt, M, K, p, st) : launch_lora_part_ct<DT_F16, 6>(x, d, part, tt, M, K, p, st);
        case 4: return bf ? launch_lora_part_ct<DT_BF16, 8>(x, d, part, tt, M, K, p, st) : launch_lora_part_ct<DT_F16, 8>(x, d, part, tt, M, K, p, st);
        default: return hipErrorInvalidValue;
    }
}

// the standalone projection: t directly (one k range), or the partials and
// then their sum rounded to bf16 into t
hipError_t lora_down_launch(const void* x, int in_dtype, const void* D, void* t, int M, int K, int R,
                            float* part, hipStream_t st) {
    if (M == 0) return hipSuccess;
    int splits = 1;
    hipError_t e = lora_part_launch(x, in_dtype, D, part, t, M, K, R, &splits, st);
    if (e != hipSuccess || splits == 1) return e;
    const size_t n = (size_t)M * R;
    const int grid = (int)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
    hipLaunchKernelGGL(lora_reduce_kernel, dim3(grid), dim3(256), 0, st, part, reinterpret_cast<__bf16*>(t), M, R,
                       splits);
    return hipGetLastError();
}

}  // namespace convrot
