// extern "C" boundary of libconvrot_gfx950.so; declarations and contracts in
// include/convrot_mi355x.h.

#include "../../include/convrot_mi355x.h"
#include "common.h"

namespace convrot {
hipError_t rotquant_launch(const void* x, int in_dtype, const void* noise, int8_t* q, float* s,
                           int M, int K, int G, hipStream_t st);
int rotquant_max_k();
hipError_t gemm_launch(const int8_t* Xp, const int8_t* Wp, const float* xs, const float* ws,
                       const float* bias, void* out, int M, int N, int K, int epi, hipStream_t st);
hipError_t gemm_lora_launch(const int8_t* Xp, const int8_t* Wp, const float* xs, const float* ws,
                            const float* bias, const void* t, const void* U, int R, float scale, void* out,
                            int M, int N, int K, int epi, hipStream_t st);
hipError_t lora_down_launch(const void* x, int in_dtype, const void* D, void* t, int M, int K, int R,
                            float* part, hipStream_t st);
hipError_t lora_part_launch(const void* x, int in_dtype, const void* D, float* part, void* t, int M, int K, int R,
                            int* splits, hipStream_t st);
hipError_t int4_to_bf6_launch(const void* src, void* dst, int rows, int K, hipStream_t st);
hipError_t bf6_to_int4_launch(const void* src, void* dst, int rows, int K, hipStream_t st);
hipError_t i8t_to_int8_launch(const void* src, void* dst, int rows, int K, hipStream_t st);
hipError_t rotquant_b6_launch(const void* x, int in_dtype, uint8_t* a6, float* s, int M, int K, int G,
                              hipStream_t st, const LoraSum* ls);
int rotquant_b6_max_k();
hipError_t rotquant_i8_launch(const void* x, int in_dtype, int8_t* q, float* s, int M, int K, int G,
                              hipStream_t st);
hipError_t gemm_i8_launch(const int8_t* X, const int8_t* W, const float* xs, const float* ws,
                          const float* bias, void* out, int M, int N, int K, int epi, hipStream_t st);
hipError_t gemm_bf6_launch(const void* A6, const void* W6, const float* xs, const float* ws, const void* bias,
                           int bias_dt, const void* t, const void* U, int R, float scale, void* out, int M, int N,
                           int K, int epi, int nsplit, void* workspace, hipStream_t st);
int gemm_bf6_choose_nsplit(int M, int N, int K);
hipError_t rotquant_i8t_launch(const void* x, int in_dtype, int8_t* q, float* s, int M, int K, int G,
                               hipStream_t st);
hipError_t int8_to_i8t_launch(const void* src, void* dst, int rows, int K, hipStream_t st);
hipError_t gemm_i8t_launch(const int8_t* X, const int8_t* W, const float* xs, const float* ws,
                           const float* bias, void* out, int M, int N, int K, int epi, hipStream_t st);
size_t gemm_bf6_splitk_workspace(int M, int N, int nsplit);
void gemm_bf6_tile(int M, int N, int K, int nsplit, int* bm, int* bn);
hipError_t gemm_splitk_launch(const int8_t* Xp, const int8_t* Wp, const float* xs, const float* ws, float* accum,
                              int M, int N, int K, int nsplit, hipStream_t st);
}  // namespace convrot

#define API extern "C" __attribute__((visibility("default")))

using convrot::kSplitCounterBytes;   // the workspaces' leading counter region (common.h)

static int quant_args_ok(int in_dtype, int M, int K, int G) {
    if (!(G == 16 || G == 64 || G == 256)) return 0;
    if (M < 0 || K <= 0 || K % G != 0) return 0;
    if (K > convrot::rotquant_max_k()) return 0;
    if (in_dtype < 0 || in_dtype > 2) return 0;
    return 1;
}

API int ck_convrot_quant_int4(const void* x, int in_dtype, void* qout, void* scaleout,
                              int M, int K, int G, void* stream) {
    if (!quant_args_ok(in_dtype, M, K, G)) return -1;
    hipError_t e = convrot::rotquant_launch(x, in_dtype, nullptr, reinterpret_cast<int8_t*>(qout),
                                            reinterpret_cast<float*>(scaleout), M, K, G,
                                            reinterpret_cast<hipStream_t>(stream));
    return (int)e;
}

API int cr_convrot_quant_int4_stochastic(const void* x, int in_dtype, const void* noise, void* qout,
                                         void* scaleout, int M, int K, int G, void* stream) {
    if (!quant_args_ok(in_dtype, M, K, G) || noise == nullptr) return -1;
    hipError_t e = convrot::rotquant_launch(x, in_dtype, noise, reinterpret_cast<int8_t*>(qout),
                                            reinterpret_cast<float*>(scaleout), M, K, G,
                                            reinterpret_cast<hipStream_t>(stream));
    return (int)e;
}

API int cr_int4_convrot_gemm_ex(const void* Xp, const void* Wp, const void* xscale, const void* wscale,
                                const void* bias, void* out, int M, int N, int K, int epilogue,
                                void* stream) {
    if (K % 32 != 0 || K <= 0 || K >= 131072 || M < 0 || N < 0) return -1;
    if (epilogue < 0 || epilogue > 3) return -1;
    hipError_t e = convrot::gemm_launch(reinterpret_cast<const int8_t*>(Xp), reinterpret_cast<const int8_t*>(Wp),
                                        reinterpret_cast<const float*>(xscale), reinterpret_cast<const float*>(wscale),
                                        reinterpret_cast<const float*>(bias), out, M, N, K, epilogue,
                                        reinterpret_cast<hipStream_t>(stream));
    return (int)e;
}

API int ck_int4_convrot_gemm(const void* Xp, const void* Wp, const void* xscale, const void* wscale,
                             const void* bias, void* out, int M, int N, int K, int out_dtype,
                             void* stream) {
    if (out_dtype != 0 && out_dtype != 1) return -1;
    return cr_int4_convrot_gemm_ex(Xp, Wp, xscale, wscale, bias, out, M, N, K, out_dtype, stream);
}

API int ck_int4_convrot_gemm_splitk(const void* Xp, const void* Wp, const void* xscale, const void* wscale,
                                    void* accum, int M, int N, int K, int nsplit, void* stream) {
    if (K % 32 != 0 || K <= 0 || K >= 131072 || M < 0 || N < 0 || nsplit < 1) return -1;
    return (int)convrot::gemm_splitk_launch(reinterpret_cast<const int8_t*>(Xp), reinterpret_cast<const int8_t*>(Wp),
                                            reinterpret_cast<const float*>(xscale),
                                            reinterpret_cast<const float*>(wscale), reinterpret_cast<float*>(accum),
                                            M, N, K, nsplit, reinterpret_cast<hipStream_t>(stream));
}

static int lora_rank_ok(int R) { return R >= 32 && R <= 128 && R % 32 == 0; }

// the partials follow the counter region (untouched here)
API size_t cr_lora_down_workspace(int M, int K, int R) {
    if (M <= 0 || K <= 0 || K % 16 != 0 || !lora_rank_ok(R)) return 0;
    const size_t need = convrot::lora_part_bytes(M, K, R);
    return need > 0 ? kSplitCounterBytes + need : 0;
}

API int cr_lora_down(const void* x, int in_dtype, const void* D, void* t, int M, int K, int R, void* workspace,
                     size_t workspace_bytes, void* stream) {
    if ((in_dtype != 1 && in_dtype != 2) || M < 0 || K <= 0 || K % 16 != 0 || !lora_rank_ok(R)) return -1;
    if (M == 0) return 0;
    const size_t need = convrot::lora_part_bytes(M, K, R);
    if (need > 0 && (workspace == nullptr || workspace_bytes < kSplitCounterBytes + need)) return -1;
    float* part = need > 0 ? reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) + kSplitCounterBytes)
                           : nullptr;
    hipError_t e = convrot::lora_down_launch(x, in_dtype, D, t, M, K, R, part, reinterpret_cast<hipStream_t>(stream));
    return (int)e;
}

API int cr_int4_convrot_gemm_lora(const void* Xp, const void* Wp, const void* xscale, const void* wscale,
                                  const void* bias, const void* t, const void* U, int R, float scale,
                                  void* out, int M, int N, int K, int epilogue, void* stream) {
    if (K % 32 != 0 || K <= 0 || K >= 131072 || M < 0 || N < 0) return -1;
    if (epilogue < 0 || epilogue > 2 || !lora_rank_ok(R) || t == nullptr || U == nullptr) return -1;
    hipError_t e = convrot::gemm_lora_launch(reinterpret_cast<const int8_t*>(Xp), reinterpret_cast<const int8_t*>(Wp),
                                             reinterpret_cast<const float*>(xscale),
                                             reinterpret_cast<const float*>(wscale),
                                             reinterpret_cast<const float*>(bias), t, U, R, scale, out, M, N, K,
                                             epilogue, reinterpret_cast<hipStream_t>(stream));
    return (int)e;
}

static int bf6_k_ok(int K) { return K > 0 && K % 128 == 0 && K < 131072; }

API int cr_int4_to_bf6(const void* src, void* dst, int rows, int K, void* stream) {
    if (rows < 0 || !bf6_k_ok(K)) return -1;
    return (int)convrot::int4_to_bf6_launch(src, dst, rows, K, reinterpret_cast<hipStream_t>(stream));
}

API int cr_bf6_to_int4(const void* src, void* dst, int rows, int K, void* stream) {
    if (rows < 0 || !bf6_k_ok(K)) return -1;
    return (int)convrot::bf6_to_int4_launch(src, dst, rows, K, reinterpret_cast<hipStream_t>(stream));
}

API int cr_convrot_quant_bf6(const void* x, int in_dtype, void* a6out, void* scaleout, int M, int K, int G,
                             void* stream) {
    if (!quant_args_ok(in_dtype, M, K, G) || K % 128 != 0 || K > convrot::rotquant_b6_max_k()) return -1;
    return (int)convrot::rotquant_b6_launch(x, in_dtype, reinterpret_cast<uint8_t*>(a6out),
                                            reinterpret_cast<float*>(scaleout), M, K, G,
                                            reinterpret_cast<hipStream_t>(stream), nullptr);
}

API int cr_max_quant_bf6_k(void) { return convrot::rotquant_b6_max_k(); }

API int cr_int4_convrot_gemm_bf6(const void* A6, const void* W6, const void* xscale, const void* wscale,
                                 const void* bias, void* out, int M, int N, int K, int epilogue, void* stream) {
    if (!bf6_k_ok(K) || M < 0 || N < 0 || epilogue < 0 || epilogue > 3) return -1;
    return (int)convrot::gemm_bf6_launch(A6, W6, reinterpret_cast<const float*>(xscale),
                                         reinterpret_cast<const float*>(wscale),
                                         bias, 0, nullptr, nullptr, 0, 0.0f, out,
                                         M, N, K, epilogue, 1, nullptr, reinterpret_cast<hipStream_t>(stream));
}

API int cr_int4_convrot_gemm_bf6_lora(const void* A6, const void* W6, const void* xscale, const void* wscale,
                                      const void* bias, const void* t, const void* U, int R, float scale,
                                      void* out, int M, int N, int K, int epilogue, void* stream) {
    if (!bf6_k_ok(K) || M < 0 || N < 0 || epilogue < 0 || epilogue > 2) return -1;
    if (!lora_rank_ok(R) || t == nullptr || U == nullptr) return -1;
    return (int)convrot::gemm_bf6_launch(A6, W6, reinterpret_cast<const float*>(xscale),
                                         reinterpret_cast<const float*>(wscale),
                                         bias, 0, t, U, R, scale, out, M, N, K,
                                         epilogue, 1, nullptr, reinterpret_cast<hipStream_t>(stream));
}

API int cr_gemm_bf6_choose_nsplit(int M, int N, int K) {
    if (M <= 0 || N <= 0 || !bf6_k_ok(K)) return 1;
    return convrot::gemm_bf6_choose_nsplit(M, N, K);
}

API int cr_gemm_bf6_tile(int M, int N, int K, int nsplit, int* bm, int* bn) {
    if (M <= 0 || N <= 0 || !bf6_k_ok(K) || nsplit < 1 || nsplit > K / 128 || bm == nullptr || bn == nullptr)
        return -1;
    convrot::gemm_bf6_tile(M, N, K, nsplit, bm, bn);
    return 0;
}

API size_t cr_gemm_bf6_splitk_workspace(int M, int N, int nsplit) {
    if (M <= 0 || N <= 0 || nsplit < 1) return 0;
    return convrot::gemm_bf6_splitk_workspace(M, N, nsplit);
}

API int cr_int4_convrot_gemm_bf6_splitk(const void* A6, const void* W6, const void* xscale, const void* wscale,
                                        const void* bias, const void* t, const void* U, int R, float scale,
                                        void* out, int M, int N, int K, int epilogue, int nsplit,
                                        void* workspace, size_t workspace_bytes, void* stream) {
    if (!bf6_k_ok(K) || M < 0 || N < 0 || nsplit < 1 || nsplit > K / 128) return -1;
    if (t != nullptr && (epilogue < 0 || epilogue > 2 || !lora_rank_ok(R) || U == nullptr)) return -1;
    if (t == nullptr && (epilogue < 0 || epilogue > 3)) return -1;
    if (nsplit > 1 && M > 0 && N > 0 &&
        (workspace == nullptr || workspace_bytes < convrot::gemm_bf6_splitk_workspace(M, N, nsplit)))
        return -1;
    return (int)convrot::gemm_bf6_launch(A6, W6, reinterpret_cast<const float*>(xscale),
                                         reinterpret_cast<const float*>(wscale),
                                         bias, 0, t, U, R, scale, out, M, N, K,
                                         epilogue, nsplit, workspace, reinterpret_cast<hipStream_t>(stream));
}

API int ck_convrot_quant_int8(const void* x, int in_dtype, void* qout, void* scaleout,
                              int M, int K, int G, void* stream) {
    if (!quant_args_ok(in_dtype, M, K, G)) return -1;
    return (int)convrot::rotquant_i8_launch(x, in_dtype, reinterpret_cast<int8_t*>(qout),
                                            reinterpret_cast<float*>(scaleout), M, K, G,
                                            reinterpret_cast<hipStream_t>(stream));
}

API int cr_int8_convrot_gemm_ex(const void* X, const void* W, const void* xscale, const void* wscale,
                                const void* bias, void* out, int M, int N, int K, int epilogue, void* stream) {
    if (K % 16 != 0 || K <= 0 || K >= 131072 || M < 0 || N < 0) return -1;
    if (epilogue != 0 && epilogue != 1 && epilogue != 3) return -1;
    return (int)convrot::gemm_i8_launch(reinterpret_cast<const int8_t*>(X), reinterpret_cast<const int8_t*>(W),
                                        reinterpret_cast<const float*>(xscale), reinterpret_cast<const float*>(wscale),
                                        reinterpret_cast<const float*>(bias), out, M, N, K, epilogue,
                                        reinterpret_cast<hipStream_t>(stream));
}

API int ck_int8_convrot_gemm(const void* X, const void* W, const void* xscale, const void* wscale,
                             const void* bias, void* out, int M, int N, int K, int out_dtype, void* stream) {
    if (out_dtype != 0 && out_dtype != 1) return -1;
    return cr_int8_convrot_gemm_ex(X, W, xscale, wscale, bias, out, M, N, K, out_dtype, stream);
}

static int i8t_k_ok(int K) { return K > 0 && K % 64 == 0 && K < 131072; }

API int cr_convrot_quant_int8_i8t(const void* x, int in_dtype, void* qout, void* scaleout, int M, int K, int G,
                                  void* stream) {
    if (!quant_args_ok(in_dtype, M, K, G) || !i8t_k_ok(K) || K > convrot::rotquant_b6_max_k()) return -1;
    return (int)convrot::rotquant_i8t_launch(x, in_dtype, reinterpret_cast<int8_t*>(qout),
                                             reinterpret_cast<float*>(scaleout), M, K, G,
                                             reinterpret_cast<hipStream_t>(stream));
}

API int cr_int8_to_i8t(const void* src, void* dst, int rows, int K, void* stream) {
    if (rows < 0 || !i8t_k_ok(K)) return -1;
    return (int)convrot::int8_to_i8t_launch(src, dst, rows, K, reinterpret_cast<hipStream_t>(stream));
}

API int cr_i8t_to_int8(const void* src, void* dst, int rows, int K, void* stream) {
    if (rows < 0 || !i8t_k_ok(K)) return -1;
    return (int)convrot::i8t_to_int8_launch(src, dst, rows, K, reinterpret_cast<hipStream_t>(stream));
}

API int cr_int8_convrot_gemm_i8t(const void* X, const void* W, const void* xscale, const void* wscale,
                                 const void* bias, void* out, int M, int N, int K, int epilogue, void* stream) {
    if (!i8t_k_ok(K) || M < 0 || N < 0) return -1;
    if (epilogue != 0 && epilogue != 1 && epilogue != 3) return -1;
    return (int)convrot::gemm_i8t_launch(reinterpret_cast<const int8_t*>(X), reinterpret_cast<const int8_t*>(W),
                                         reinterpret_cast<const float*>(xscale), reinterpret_cast<const float*>(wscale),
                                         reinterpret_cast<const float*>(bias), out, M, N, K, epilogue,
                                         reinterpret_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// The whole bf6 linear in one call: rotate + quantize x into B6T, the LoRA down
// projection (R > 0), the GEMM (k-split when the library chooses it) with the
// epilogue and the LoRA term.  Intermediates live in the caller's workspace.
// ---------------------------------------------------------------------------
namespace {
// Workspace layout: the GEMM's split region first (its counters at bytes
// 0 .. 2047 of every workspace, whatever the shape and split, so that no
// other intermediate of any call ever overwrites them), then the B6T codes,
// the row scales, t and the LoRA partials.
struct LinPlan { size_t part, a6, xs, t, lpart, total; int nsplit; };
size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }
LinPlan lin_plan(int M, int N, int K, int R) {
    LinPlan p{};
    const size_t rows = (size_t)((M + 255) / 256) * 256;
    p.nsplit = convrot::gemm_bf6_choose_nsplit(M, N, K);
    p.part = 0;
    const size_t split_bytes = convrot::gemm_bf6_splitk_workspace(M, N, p.nsplit);
    p.a6 = al256(split_bytes > kSplitCounterBytes ? split_bytes : kSplitCounterBytes);
    p.xs = p.a6 + al256(rows * (size_t)K / 4 * 3);
    p.t = p.xs + al256((size_t)M * 4);
    p.lpart = p.t + al256((size_t)M * R * 2);
    p.total = p.lpart + (R > 0 ? al256(convrot::lora_part_bytes(M, K, R)) : 0);
    return p;
}
}  // namespace

API size_t cr_convrot_w4a4_linear_bf6_workspace(int M, int N, int K, int R) {
    if (M <= 0 || N <= 0 || !bf6_k_ok(K) || R < 0) return 0;
    return lin_plan(M, N, K, R).total;
}

static int linear_bf6_args_ok(int in_dtype, int bias_dtype, const void* D, const void* U, int R, int epilogue,
                              int M, int N, int K, int G) {
    if (!quant_args_ok(in_dtype, M, K, G) || !bf6_k_ok(K) || K > convrot::rotquant_b6_max_k() || N < 0) return 0;
    if (bias_dtype < 0 || bias_dtype > 2) return 0;
    if (epilogue < 0 || epilogue > 2) return 0;
    if (R != 0 && (!lora_rank_ok(R) || D == nullptr || U == nullptr || in_dtype == 0)) return 0;
    return 1;
}

// The linear's launches with its intermediates at `workspace` (p.total bytes).
static int linear_bf6_run(const void* x, int in_dtype, const void* W6, const void* wscale, const void* bias,
                          int bias_dtype, const void* D, const void* U, int R, float scale, void* out, int epilogue,
                          int M, int N, int K, int G, const LinPlan& p, void* workspace, void* stream) {
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
    float* xs = reinterpret_cast<float*>(ws + p.xs);
    // LoRA (R > 0).  A projection split over k ranges runs first, and the
    // rotate+quant kernel adds its partial sums up row by row into t.  An
    // unsplit one writes t itself and runs after rotate+quant, which has just
    // read x: its own read of x then comes from the Infinity Cache (burst-timed
    // pair on MI355X, 4096 x 3072, rank 32: 18.35 us against 19.77 in the
    // other order).
    float* lpart = reinterpret_cast<float*>(ws + p.lpart);
    const bool lora_split = R != 0 && convrot::lora_part_bytes(M, K, R) > 0;
    int splits = 1;
    if (lora_split) {
        hipError_t e = convrot::lora_part_launch(x, in_dtype, D, lpart, ws + p.t, M, K, R, &splits, st);
        if (e != hipSuccess) return (int)e;
    }
    convrot::LoraSum ls{lpart, reinterpret_cast<__bf16*>(ws + p.t), splits, R};
    hipError_t e = convrot::rotquant_b6_launch(x, in_dtype, ws + p.a6, xs, M, K, G, st,
                                               splits > 1 ? &ls : nullptr);
    if (e != hipSuccess) return (int)e;
    if (R != 0 && !lora_split) {
        e = convrot::lora_part_launch(x, in_dtype, D, lpart, ws + p.t, M, K, R, &splits, st);
        if (e != hipSuccess) return (int)e;
    }
    return (int)convrot::gemm_bf6_launch(ws + p.a6, W6, xs, reinterpret_cast<const float*>(wscale), bias, bias_dtype,
                                         R ? ws + p.t : nullptr, U, R, scale, out, M, N, K, epilogue, p.nsplit,
                                         ws + p.part, st);
}

API int cr_convrot_w4a4_linear_bf6(const void* x, int in_dtype, const void* W6, const void* wscale, const void* bias,
                                   int bias_dtype, const void* D, const void* U, int R, float scale, void* out,
                                   int epilogue, int M, int N, int K, int G, void* workspace, size_t workspace_bytes,
                                   void* stream) {
    if (!linear_bf6_args_ok(in_dtype, bias_dtype, D, U, R, epilogue, M, N, K, G)) return -1;
    if (M == 0 || N == 0) return 0;
    const LinPlan p = lin_plan(M, N, K, R);
    if (workspace == nullptr || workspace_bytes < p.total) return -1;
    return linear_bf6_run(x, in_dtype, W6, wscale, bias, bias_dtype, D, U, R, scale, out, epilogue, M, N, K, G, p,
                          workspace, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free form of cr_convrot_w4a4_linear_bf6.  The intermediates live
// in `scratch`, a file-scope device array of kScratchBytes that every GPU the
// library runs on holds until the process ends.  In host code `scratch` names
// a host-side stand-in, so its device address is looked up once per device
// (hipGetSymbolAddress with that device current, on the first call there) and
// only that address is passed to kernels.  Nothing here allocates; every byte
// the kernels read from the scratch is written earlier in the same call
// (codes and padding rows, scales, LoRA t, split partials), so nothing needs
// clearing between calls.  Calls that overlap on one GPU share the array and
// race.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = size_t(64) << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

static hipError_t scratch_address(void** out) {
    static std::atomic<void*> addr[convrot::kMaxDev];
    int dev = 0;
    hipError_t e = convrot::current_device(&dev);
    if (e != hipSuccess) return e;
    void* p = addr[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (p == nullptr) return hipErrorInvalidSymbol;
        addr[dev].store(p, std::memory_order_release);
    }
    *out = p;
    return hipSuccess;
}

API int cr_convrot_w4a4_linear_bf6_noalloc(const void* x, int in_dtype, const void* W6, const void* wscale,
                                           const void* bias, int bias_dtype, const void* D, const void* U, int R,
                                           float scale, void* out, int epilogue, int M, int N, int K, int G,
                                           void* stream) {
    if (!linear_bf6_args_ok(in_dtype, bias_dtype, D, U, R, epilogue, M, N, K, G)) return -1;
    if (M == 0 || N == 0) return 0;
    const LinPlan p = lin_plan(M, N, K, R);
    if (p.total > kScratchBytes) return -1;       // this shape needs more than the library's scratch
    void* ws = nullptr;
    hipError_t e = scratch_address(&ws);
    if (e != hipSuccess) return (int)e;
    return linear_bf6_run(x, in_dtype, W6, wscale, bias, bias_dtype, D, U, R, scale, out, epilogue, M, N, K, G, p, ws,
                          stream);
}

API int cr_max_quant_k(void) { return convrot::rotquant_max_k(); }

API int cr_abi_version(void) { return 13; }
