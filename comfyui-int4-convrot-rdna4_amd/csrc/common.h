// Shared device helpers for the gfx950 W4A4 ConvRot kernels.
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace convrot {

// dtype codes of the C-ABI (reference: _int4/hip_loader.py:38-39)
enum : int { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };

// ---------------------------------------------------------------------------
// host-side per-device set-up.  Launch helpers may be called from several
// host threads at once, so their caches are atomics: concurrent first calls
// on a device may each do the set-up, which is idempotent.
// ---------------------------------------------------------------------------

constexpr int kMaxDev = 64;

// Index of the current device, checked against kMaxDev.
inline hipError_t current_device(int* dev) {
    hipError_t e = hipGetDevice(dev);
    if (e != hipSuccess) return e;
    return (*dev < 0 || *dev >= kMaxDev) ? hipErrorInvalidDevice : hipSuccess;
}

// Raises a kernel's dynamic-LDS limit to `bytes` on the current device, once.
// A failed attempt leaves the flag clear, so the next call tries again.
inline hipError_t lds_limit_once(std::atomic<bool> (&done)[kMaxDev], int dev, const void* kernel, int bytes) {
    if (done[dev].load(std::memory_order_acquire)) return hipSuccess;
    hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess) done[dev].store(true, std::memory_order_release);
    return e;
}

// Bytes 0 .. 2047 of every workspace the library takes hold the split
// counters of the bf6 GEMM's small-tile kernel (one per tile, at most 512):
// zero when a workspace is first used and zero again after every call; no
// other intermediate is ever written there.
constexpr size_t kSplitCounterBytes = 2048;

// The split LoRA down projection (lora.hip): x rows per workgroup, k splits,
// k per split.  lora_plan is a pure function of the shape.
struct LoraPlan { int xr, splits, krange; };
LoraPlan lora_plan(int M, int K, int R);
size_t lora_part_bytes(int M, int K, int R);

// What the rotate+quant kernel sums for the linear's LoRA side path: t[m, r] =
// bf16(part[0, m, r] + .. + part[S-1, m, r]) in that order (S <= 8).
struct LoraSum { const float* part; __bf16* t; int S, R; };

__device__ __forceinline__ float bf16lo_to_f32(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi_to_f32(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ float f16bits_to_f32(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short)(h & 0xffffu)));
}

// float -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    return (uint32_t)__bfloat16_as_ushort(__float2bfloat16(f));
}

// Round a float once to the element dtype and widen it back (RNE).
template <int DT>
__device__ __forceinline__ float round_to_dt(float f) {
    if constexpr (DT == DT_BF16) {
        return __uint_as_float(f32_to_bf16_bits(f) << 16);
    } else if constexpr (DT == DT_F16) {
        return __half2float(__float2half_rn(f));
    } else {
        return f;
    }
}

// Round an fp64 value ONCE to the element dtype (RNE), returned as float.
// bf16 / f16: the low 32 bits of the double are folded into a sticky bit at
// mantissa bit 32 ("jamming"); the result then has at most 21 significant bits
// and converts to float exactly, and the single float -> dtype rounding sees
// the same guard bit and the same sticky predicate as the exact value, so it
// rounds the same way.  f32: one fp64 -> fp32 conversion.
template <int DT>
__device__ __forceinline__ float round_f64_to_dt(double d) {
    if constexpr (DT == DT_F32) {
        return (float)d;
    } else {
        uint64_t u = (uint64_t)__double_as_longlong(d);
        uint32_t hi = (uint32_t)(u >> 32), lo = (uint32_t)u;
        hi |= (lo != 0u) ? 1u : 0u;
        float f = (float)__longlong_as_double((long long)((uint64_t)hi << 32));
        return round_to_dt<DT>(f);
    }
}

// Order LDS accesses of the lanes of one wave: every lane's earlier LDS
// writes are visible to every lane's later LDS reads.  A wave issues its LDS
// operations in program order; the fences keep the compiler from moving LDS
// accesses across this point.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two floats -> packed bf16 pair (a in the low half), both rounded to nearest
// even by one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    const bf16x2_t h = __builtin_convertvector((f32x2_t){a, b}, bf16x2_t);
    return __builtin_bit_cast(uint32_t, h);
}

}  // namespace convrot
