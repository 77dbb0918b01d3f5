/*
 * C-ABI of the gfx950 (MI355X) W4A4 ConvRot linear path.
 *
 * Library: comfyui-int4-convrot-rdna4_amd/_int4/libconvrot_gfx950.so
 *
 * Conventions: those of the reference's ctypes boundary.  The five exports the
 * reference's loader binds (_int4/hip_loader.py:42-71: ck_int4_convrot_gemm,
 * ck_int4_convrot_gemm_splitk, ck_convrot_quant_int4, ck_int8_convrot_gemm,
 * ck_convrot_quant_int8) exist here with the same names, argument lists and
 * contracts, so that loader binds this library unchanged:
 *   - all pointers are device pointers; the caller allocates every buffer
 *     (outputs included) and every entry point works in caller memory only,
 *     except cr_convrot_w4a4_linear_bf6_noalloc, whose intermediates live in
 *     a 64 MiB static device array that the library's code object holds on
 *     every GPU it is loaded on (whether or not that entry point is called);
 *   - work is enqueued asynchronously on `stream` (a hipStream_t, e.g.
 *     torch.cuda.current_stream().cuda_stream); nothing synchronises;
 *   - dtype codes: input 0 = f32, 1 = bf16, 2 = f16; output 0 = f32, 1 = bf16
 *     (reference _int4/hip_loader.py:38-39);
 *   - return value: 0 on success, -1 on invalid arguments, otherwise the
 *     hipError_t of the launch (no device synchronisation).
 *   - packed int4 layout: int8 [rows, K/2], element 2j in the low nibble of
 *     byte j, 2j+1 in the high nibble (reference _int4/_codec.py:19-25).
 *   - workspaces (cr_lora_down, cr_int4_convrot_gemm_bf6_splitk,
 *     cr_convrot_w4a4_linear_bf6): bytes 0..2047 of every workspace hold the
 *     split counters of the bf6 GEMM.  They must be zero when a workspace is
 *     first used (clear them once after allocating it); every call leaves them
 *     zero, and no call writes anything else there, so one workspace can serve
 *     every entry point and shape in stream order.  The sizes returned by the
 *     *_workspace queries include these 2048 bytes.  The no-allocation entry
 *     point's static array starts zeroed and keeps the same rule.
 */
#ifndef CONVROT_MI355X_H
#define CONVROT_MI355X_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Fused ConvRot rotation + rowwise int4 quantization + nibble packing.
 *   x        [M, K] in_dtype (row-major, contiguous)
 *   qout     int8 [M, K/2]  packed codes in [-7, 7]
 *   scaleout f32 [M]        per-row scale, an exact value of in_dtype
 * G in {16, 64, 256}, K % G == 0, K <= 32768.
 * Arithmetic: the reference eager path (_int4/eager.py:65-79, 104-120):
 * exactly rounded rotation, s = dt(fl32(absmax/7)), q = rint_even(dt(fl32(x/s))).
 * Replaces: ck_convrot_quant_int4, reference _int4/int4_gemm.hip:650-660
 * (bound at _int4/hip_loader.py:56-61, called at :74-92).
 */
int ck_convrot_quant_int4(const void* x, int in_dtype, void* qout, void* scaleout,
                          int M, int K, int G, void* stream);

/*
 * W4A4 GEMM with int32 accumulation and the dequant epilogue:
 *   out[m, n] = fl32(fl32(fl32(acc * xscale[m]) * wscale[n]) + bias[n])
 *   acc[m, n] = sum_k qx[m, k] * qw[n, k]
 * Xp int8 [M, K/2], Wp int8 [N, K/2], xscale f32 [M], wscale f32 [N],
 * bias f32 [N] or NULL, out [M, N] f32 (out_dtype 0) or bf16 (out_dtype 1,
 * one RNE of the f32 value).  K % 32 == 0.
 * Replaces: ck_int4_convrot_gemm, reference _int4/int4_gemm.hip:711-741
 * (bound at _int4/hip_loader.py:50-52, called at :158-207).
 */
int ck_int4_convrot_gemm(const void* Xp, const void* Wp, const void* xscale, const void* wscale,
                         const void* bias, void* out, int M, int N, int K, int out_dtype,
                         void* stream);

/*
 * Split-K form of ck_int4_convrot_gemm for small output grids (the reference
 * chooses it for few tiles and large K, _int4/hip_loader.py:20-36).
 *   accum f32 [M, N], zeroed by the caller; on return it holds
 *   fl32(fl32(acc * xscale[m]) * wscale[n]), the scaled product WITHOUT bias;
 *   the caller adds the bias and casts (_int4/hip_loader.py:176-192).
 * The k blocks are split over min(nsplit, ceil(K / 128)) workgroups per tile;
 * each adds its exact integer partial into accum (viewed as int32, which is 0
 * for a zeroed float buffer) with atomics, and one more kernel scales the sum
 * in place.  The result is therefore bit-identical to ck_int4_convrot_gemm's
 * f32 epilogue (bias NULL) for every nsplit.  A non-zeroed accum gives
 * undefined results.  K % 32 == 0, nsplit >= 1; otherwise -1.
 * Replaces: ck_int4_convrot_gemm_splitk, reference _int4/int4_gemm.hip:634-645
 * (bound at _int4/hip_loader.py:53-56, called at :176-192), whose partials are
 * rounded per split and added in an order the atomics decide.
 */
int ck_int4_convrot_gemm_splitk(const void* Xp, const void* Wp, const void* xscale, const void* wscale,
                                void* accum, int M, int N, int K, int nsplit, void* stream);

/*
 * ck_int4_convrot_gemm with an explicit epilogue:
 *   epilogue 0: f32 output, as ck_int4_convrot_gemm out_dtype 0
 *   epilogue 1: bf16 output, as ck_int4_convrot_gemm out_dtype 1
 *   epilogue 2: bf16 output through the eager bf16 rounding chain
 *               o1 = bf16(acc), o2 = bf16(o1*bf16(xs)), o3 = bf16(o2*bf16(ws)),
 *               o4 = bf16(o3 + bf16(bias))  (_int4/eager.py:162-168)
 *   epilogue 3: int32 accumulators only (out is int32 [M, N]; scales unused)
 * Extends the same reference export (_int4/int4_gemm.hip:711-741); epilogue 3
 * is the accumulator dump used to prove the integer stage bit-exact.
 */
int cr_int4_convrot_gemm_ex(const void* Xp, const void* Wp, const void* xscale, const void* wscale,
                            const void* bias, void* out, int M, int N, int K, int epilogue,
                            void* stream);

/*
 * ck_convrot_quant_int4 with stochastic rounding: q = clamp(floor(dt(t + u)), -7, 7)
 * with t = dt(fl32(xr/s)) and u = noise [M, K] (in_dtype, uniform [0, 1)), the
 * weight-quantization mode of _int4/eager.py:92-109 (the caller draws u with the
 * same generator call as the reference, _int4/eager.py:92-101).
 * Replaces the torch stochastic branch of quantize_convrot_w4a4_weight
 * (_int4/eager.py:123-135), which has no native counterpart in the reference.
 */
int cr_convrot_quant_int4_stochastic(const void* x, int in_dtype, const void* noise, void* qout,
                                     void* scaleout, int M, int K, int G, void* stream);

/*
 * Down projection of the dynamic-LoRA side path: t = bf16(x @ D^T).
 *   x [M, K] bf16 (in_dtype 1) or f16 (2), D [R, K] bf16, t [M, R] bf16;
 *   R in {32, 64, 96, 128}, K % 16 == 0.
 * Depending on the shape (never on the device) the projection is split over
 * k: f32 partial sums go to `workspace` after its counter region
 * (cr_lora_down_workspace(M, K, R) bytes; 0 bytes, and workspace may be NULL,
 * for an unsplit shape), then their
 * sum in split order is rounded once to bf16.  The linear
 * (cr_convrot_w4a4_linear_bf6) computes the same t bit for bit.
 * Together with cr_int4_convrot_gemm_lora it replaces the per-adapter
 * v.h(x, out) side path of Int4ConvRotOps.Linear._apply_dyn_lora
 * (reference int4_ops.py:181-192), which has no native counterpart there.
 */
int cr_lora_down(const void* x, int in_dtype, const void* D, void* t, int M, int K, int R, void* workspace,
                 size_t workspace_bytes, void* stream);

/* Workspace bytes of cr_lora_down for this shape (0: none needed, or invalid arguments). */
size_t cr_lora_down_workspace(int M, int K, int R);

/*
 * cr_int4_convrot_gemm_ex (epilogue 0, 1 or 2) plus the LoRA up projection in
 * the epilogue:  out = epilogue + scale * (t @ U^T), with t from cr_lora_down
 * and U [N, R] bf16 (several adapters: D and U concatenated along R, each
 * adapter's multiplier * alpha / rank folded into its rows of U).  The term is
 * added in fp32 before the output rounding (epilogue 2: rounded to bf16 and
 * added in the bf16 chain).
 */
int cr_int4_convrot_gemm_lora(const void* Xp, const void* Wp, const void* xscale, const void* wscale,
                              const void* bias, const void* t, const void* U, int R, float scale,
                              void* out, int M, int N, int K, int epilogue, void* stream);

/*
 * bf6 operand path.  CDNA4's v_mfma_scale_f32_32x32x64_f8f6f4 runs BF6 (E3M2)
 * operands at twice the int8 rate and BF6 holds every int4 value exactly; the
 * products are integers and the fp32 accumulation of a K < 131072 dot product
 * is exact, so these entry points return the same accumulators (and, through
 * the same epilogues, the same outputs) as cr_int4_convrot_gemm_ex.  They
 * have no counterpart in the reference: the Linear replacement converts each
 * weight once at load time and uses them on its forward path
 * (reference _int4/__init__.py:94-138 is the call they serve).
 *
 * "B6T" layout of a [rows, K] operand (K % 128 == 0): rows padded to
 * R = ceil(rows / 256) * 256 with zero codes; R * 3K/4 bytes stored as
 * [R / 256][K / 128] chunks of 24576 bytes (256 rows x 128 k).  An int4
 * value q is held as the BF6 code of q / 16, which is |q| with the sign in bit
 * 5 (E3M2's subnormals and first binade are 1/16 apart; -0, 0x20, may stand
 * for 0); the GEMMs scale both operands by 2^4.  Group g of a row is the 32
 * codes of k = 128 kb + 32 g .. +31, code e at bits 6e..6e+5 of the group's
 * 6 little-endian dwords d0..d5.  In a chunk, with
 * rr = r % 32 and f(rr) = ((rr >> 1 ^ rr >> 3) & 1) | (rr >> 1 & 2):
 *   bytes 0..16383: row r at r * 64; 16-byte piece g ^ f(rr) holds d0..d3 of
 *     group g when r / 32 is even, d2..d5 when it is odd;
 *   bytes 16384..24575: pair p = r / 64 at 16384 + (p * 32 + rr) * 64;
 *     16-byte piece g ^ f(rr) holds d4..d5 of group g of row 64p + rr
 *     (bytes 0..7) and d0..d1 of group g of row 64p + 32 + rr (bytes 8..15).
 */

/* Packed int4 [rows, K/2] (the _int4/_codec.py layout) -> B6T (dst holds
 * ceil(rows / 256) * 256 * 3K/4 bytes). */
int cr_int4_to_bf6(const void* src, void* dst, int rows, int K, void* stream);

/* B6T -> packed int4 [rows, K/2]: the inverse of cr_int4_to_bf6 on the first
 * `rows` rows, bit for bit.  Lets a layer keep only its B6T weight on the
 * device and hand out the checkpoint layout (the reference's Save node reads
 * it, int4_save.py:114-118) when asked.  No counterpart in the reference. */
int cr_bf6_to_int4(const void* src, void* dst, int rows, int K, void* stream);

/* ck_convrot_quant_int4 writing the codes in the B6T layout (a6out holds
 * ceil(M / 256) * 256 * 3K/4 bytes, padding rows zero) instead of packed
 * nibbles; same codes and scales.  K % 128 == 0 and K <= cr_max_quant_bf6_k(). */
int cr_convrot_quant_bf6(const void* x, int in_dtype, void* a6out, void* scaleout, int M, int K, int G,
                         void* stream);

/* Largest K accepted by cr_convrot_quant_bf6. */
int cr_max_quant_bf6_k(void);

/* cr_int4_convrot_gemm_ex on B6T operands (A6 from M rows, W6 from N rows); epilogue 0..3.
 * Grids of at most 512 128 x 128 output tiles with K <= 4096 run on 128 x 128
 * tiles, larger ones on 256 x 256 tiles; the outputs are the same bits. */
int cr_int4_convrot_gemm_bf6(const void* A6, const void* W6, const void* xscale, const void* wscale,
                             const void* bias, void* out, int M, int N, int K, int epilogue, void* stream);

/* cr_int4_convrot_gemm_lora on B6T operands; epilogue 0..2. */
int cr_int4_convrot_gemm_bf6_lora(const void* A6, const void* W6, const void* xscale, const void* wscale,
                                  const void* bias, const void* t, const void* U, int R, float scale,
                                  void* out, int M, int N, int K, int epilogue, void* stream);

/*
 * Split-K form of the bf6 GEMM for small tile grids (few rows, large K): S
 * workgroups per output tile each take 1/S of the 128-k blocks and store their
 * raw accumulators (exact integers) in `workspace`.  On grids of 128 x 128 or
 * 128 x 192 tiles the split that finishes last sums the S partials in the same kernel
 * (a ticket from the tile's counter in the workspace's counter region decides
 * which); on 256 x 256 tiles a second kernel sums them.  Integer partials sum
 * exactly in any order, so the outputs are bit-identical to
 * cr_int4_convrot_gemm_bf6 / _lora for every S.
 *   t == NULL: no LoRA term, epilogue 0..3; else LoRA as cr_int4_convrot_gemm_bf6_lora
 *   (epilogue 0..2).  1 <= nsplit <= K / 128; nsplit == 1 needs no workspace,
 *   otherwise workspace_bytes >= cr_gemm_bf6_splitk_workspace(M, N, nsplit).
 * The bf6 counterpart of ck_int4_convrot_gemm_splitk (reference
 * _int4/int4_gemm.hip:634-645, which adds rounded fp32 partials into a zeroed
 * [M, N] buffer with atomics and leaves bias and cast to torch): this one owns
 * its workspace layout, sums the partials in a fixed order and finishes the
 * epilogue itself.
 */
int cr_int4_convrot_gemm_bf6_splitk(const void* A6, const void* W6, const void* xscale, const void* wscale,
                                    const void* bias, const void* t, const void* U, int R, float scale,
                                    void* out, int M, int N, int K, int epilogue, int nsplit,
                                    void* workspace, size_t workspace_bytes, void* stream);

/* The library's k-split count for an M x N x K bf6 GEMM (1 = no split). */
int cr_gemm_bf6_choose_nsplit(int M, int N, int K);

/* The workgroup tile (*bm rows of A x *bn rows of B) of a bf6 GEMM launch of
 * M x N x K split nsplit ways: 256 x 256 on large grids, 128 x 128 or 128 x 192
 * on small ones (the outputs are the same bits whichever runs).  0, or -1 for
 * arguments no launch accepts.  No counterpart in the reference: for tests and
 * measurement reports that name the kernel which ran. */
int cr_gemm_bf6_tile(int M, int N, int K, int nsplit, int* bm, int* bn);

/* Workspace bytes of cr_int4_convrot_gemm_bf6_splitk: 2048 counter bytes plus
 * one f32 per output of every tile and split for the largest of the tile
 * shapes (nsplit * tiles * bm * bn * 4 over 256 x 256, 128 x 128, 128 x 192;
 * 0 when nsplit == 1). */
size_t cr_gemm_bf6_splitk_workspace(int M, int N, int nsplit);

/*
 * The whole W4A4 linear of the Linear replacement's forward in one call:
 *   out = epilogue(x_rot_quant @ W^T) [+ scale * (x @ D^T) @ U^T]
 * = cr_convrot_quant_bf6 on x, cr_lora_down when R > 0 (x bf16/f16), then the
 * bf6 GEMM (k-split when cr_gemm_bf6_choose_nsplit says so) with epilogue 0..2;
 * the same bits as those calls made one by one (here the LoRA partial sums are
 * added up by the rotate+quant kernel, in cr_lora_down's order).  W6 is the
 * weight in B6T (cr_int4_to_bf6), wscale f32 [N], bias [N] of bias_dtype (0 f32,
 * 1 bf16, 2 f16: the Linear keeps biases in fp16) or NULL, D
 * [R, K] / U [N, R] bf16 (R = 0: no LoRA).  The activation codes, scales, t and
 * split partials live in `workspace` (>= cr_convrot_w4a4_linear_bf6_workspace
 * bytes, reused by the next call on the same stream).  K % 128 == 0,
 * K <= cr_max_quant_bf6_k().  No counterpart in the reference's ABI: it serves
 * the per-call sequence of _int4/__init__.py:94-138 with one FFI crossing.
 */
int cr_convrot_w4a4_linear_bf6(const void* x, int in_dtype, const void* W6, const void* wscale, const void* bias,
                               int bias_dtype, const void* D, const void* U, int R, float scale, void* out,
                               int epilogue, int M, int N, int K, int G, void* workspace, size_t workspace_bytes,
                               void* stream);

/* Workspace bytes of cr_convrot_w4a4_linear_bf6 for this shape and LoRA rank. */
size_t cr_convrot_w4a4_linear_bf6_workspace(int M, int N, int K, int R);

/*
 * cr_convrot_w4a4_linear_bf6 without the workspace argument: the library
 * allocates nothing during the call (no hipMalloc, no allocating library
 * routine).  The intermediates live in a 64 MiB device array that the library
 * holds on every GPU it runs on until the process ends; the caller passes
 * inputs and outputs only.  Same kernels, same bits as
 * cr_convrot_w4a4_linear_bf6.  Returns -1 (no device work) when the shape's
 * cr_convrot_w4a4_linear_bf6_workspace(M, N, K, R) exceeds 64 MiB (e.g. M =
 * 4608 fits for K <= 12288; M = 16384, K = 12288 does not), and for the same
 * argument errors as cr_convrot_w4a4_linear_bf6.  The array is shared by all
 * calls on one GPU and holds the last call's contents: calls that overlap on
 * one GPU (different streams, or host threads) race.  The first call on a
 * device looks the array's address up and sets the kernels' LDS limits (not
 * stream operations): make one call per device before capturing the entry
 * point into a HIP graph; captured calls then replay like eager ones.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory during a forward (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation).
 */
int cr_convrot_w4a4_linear_bf6_noalloc(const void* x, int in_dtype, const void* W6, const void* wscale,
                                       const void* bias, int bias_dtype, const void* D, const void* U, int R,
                                       float scale, void* out, int epilogue, int M, int N, int K, int G,
                                       void* stream);

/*
 * W8A8 tier (the reference's int8 ConvRot layers, _int4/int8_eager.py).
 *
 * Fused ConvRot rotation + rowwise int8 quantization:
 *   qout     int8 [M, K]  plain codes in [-127, 127]
 *   scaleout f32 [M]      per-row scale, an exact value of in_dtype
 * G in {16, 64, 256}, K % G == 0, K <= 32768.  Arithmetic: the reference eager
 * path (_int4/int8_eager.py:22-28 on _int4/eager.py:65-79): exactly rounded
 * rotation, s = dt(fl32(absmax/127)), q = clamp(rint_even(dt(fl32(x/s))), +-127).
 * Replaces: ck_convrot_quant_int8, reference _int4/int4_gemm.hip:664-676
 * (bound at _int4/hip_loader.py:66-71, called at :95-113).
 */
int ck_convrot_quant_int8(const void* x, int in_dtype, void* qout, void* scaleout,
                          int M, int K, int G, void* stream);

/*
 * W8A8 GEMM: out[m, n] = fl32(fl32(fl32(float(acc) * xscale[m]) * wscale[n]) + bias[n]),
 * acc[m, n] = sum_k x[m, k] * w[n, k] exact in int32 (float(acc) rounds to
 * nearest even once |acc| >= 2^24).  X int8 [M, K], W int8 [N, K], K % 16 == 0.
 * Replaces: ck_int8_convrot_gemm, reference _int4/int4_gemm.hip:678-709
 * (bound at _int4/hip_loader.py:63-65, called at :116-147).
 */
int ck_int8_convrot_gemm(const void* X, const void* W, const void* xscale, const void* wscale,
                         const void* bias, void* out, int M, int N, int K, int out_dtype, void* stream);

/* ck_int8_convrot_gemm with epilogue 0 (f32), 1 (bf16) or 3 (int32 accumulators). */
int cr_int8_convrot_gemm_ex(const void* X, const void* W, const void* xscale, const void* wscale,
                            const void* bias, void* out, int M, int N, int K, int epilogue, void* stream);

/*
 * The W8A8 tier on the I8T operand layout (no counterpart in the reference: a
 * gfx950 layout of the same int8 codes).  An int8 matrix [rows, K], K % 64 == 0,
 * is stored as ceil(rows/256) x K/64 chunks of 16384 bytes, the rows padded
 * with zero codes: chunk (t, kb) holds rows 256t..256t+255, k = 64kb..64kb+63,
 * row r at byte r*64, its 16-byte piece c at (c ^ f(r))*16 with
 * f(r) = (((r >> 1) ^ (r >> 3)) & 1) | ((r >> 1) & 2).  Size: ceil(rows/256)*256*K.
 *
 * cr_convrot_quant_int8_i8t: ck_convrot_quant_int8 (same codes and scales, the
 *   reference _int4/int4_gemm.hip:664-676 path) written in I8T; K <= cr_max_quant_bf6_k().
 * cr_int8_to_i8t: re-lays row-major int8 codes (a quantized weight) into I8T.
 * cr_i8t_to_int8: the inverse of cr_int8_to_i8t on the first `rows` rows.
 * cr_int8_convrot_gemm_i8t: cr_int8_convrot_gemm_ex on I8T operands; the
 *   accumulators and outputs equal the row-major call's bit for bit.
 */
int cr_convrot_quant_int8_i8t(const void* x, int in_dtype, void* qout, void* scaleout, int M, int K, int G,
                              void* stream);
int cr_int8_to_i8t(const void* src, void* dst, int rows, int K, void* stream);
int cr_i8t_to_int8(const void* src, void* dst, int rows, int K, void* stream);
int cr_int8_convrot_gemm_i8t(const void* X, const void* W, const void* xscale, const void* wscale,
                             const void* bias, void* out, int M, int N, int K, int epilogue, void* stream);

/* Largest K accepted by the quantization entry points. */
int cr_max_quant_k(void);

/* ABI version of this library (increments on any signature change). */
int cr_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* CONVROT_MI355X_H */
