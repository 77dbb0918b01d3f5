/*
 * CPU oracle for the W4A4 ConvRot linear path.  TEST INFRASTRUCTURE ONLY:
 * nothing in the shipped package links, loads or calls this file; only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it,
 * and only as the checker.  Row loops run in parallel with OpenMP (rows are
 * independent; the arithmetic of every row is unchanged).
 *
 * It restates the reference eager path (pure torch) in plain C, with every
 * rounding step made explicit.  Each function names the reference lines it
 * follows (paths relative to the reference repository root).
 *
 * Number formats: bf16 / f16 values travel as their uint16 bit patterns, f32 as
 * float.  dtype codes follow the reference C-ABI: 0 = f32, 1 = bf16, 2 = f16
 * (_int4/hip_loader.py:38-39).
 *
 * Rotation semantics: the eager path computes x.reshape(-1,K/G,G) @ H in the
 * input dtype (_int4/eager.py:65-79), i.e. a dot product of G inputs with
 * entries +-1/sqrt(G), accumulated by the BLAS library and rounded once to the
 * input dtype.  The oracle returns the CORRECTLY ROUNDED value of that dot
 * product: the exact sum, rounded once (RNE).  It is exact for every finite
 * input: a group whose nonzero magnitudes span few enough binades is summed in
 * fp64 (provably exact), any other group goes through an exact multi-limb
 * integer accumulator.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define DT_F32 0
#define DT_BF16 1
#define DT_F16 2

/* ----------------------------------------------------------------------- */
/* scalar format helpers                                                    */
/* ----------------------------------------------------------------------- */

static float u32_as_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f32_as_u32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float orc_bf16_to_f32(uint16_t b) { return u32_as_f32((uint32_t)b << 16); }

/* float -> bf16, round to nearest even (torch's c10::BFloat16 conversion). */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u = f32_as_u32(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40); /* quiet NaN */
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t s = (uint32_t)(h >> 15) << 31;
    int e = (h >> 10) & 0x1f;
    uint32_t m = h & 0x3ff;
    if (e == 0x1f) return u32_as_f32(s | 0x7f800000u | (m << 13));
    if (e == 0) {
        float v = ldexpf((float)m, -24);
        return s ? -v : v;
    }
    return u32_as_f32(s | ((uint32_t)(e - 15 + 127) << 23) | (m << 13));
}

/* ----------------------------------------------------------------------- */
/* exact rounding of mag * 2^exp2 (mag an unsigned 64-bit integer) to a    */
/* binary format with p significant bits and minimum normal exponent emin  */
/* (value range [2^emin, ...)).  Returns the rounded value as a double,     */
/* which is exact because p <= 24 and the exponent range fits a double.     */
/* ----------------------------------------------------------------------- */

typedef struct { int p; int emin; int emax; } fmt_t;
static const fmt_t FMT_F32 = {24, -126, 127};
static const fmt_t FMT_BF16 = {8, -126, 127};
static const fmt_t FMT_F16 = {11, -14, 15};

static fmt_t fmt_of(int dt) { return dt == DT_F32 ? FMT_F32 : (dt == DT_F16 ? FMT_F16 : FMT_BF16); }

/* Round (mag, exp2, sticky_in) once to nearest-even in format f.  sticky_in
 * says that the true magnitude is strictly above mag*2^exp2 (by less than one
 * unit of mag's last bit).  */
static double round_mag(uint64_t mag, int exp2, int sticky_in, int neg, fmt_t f) {
    if (mag == 0) return neg ? -0.0 : 0.0;
    int top = 63 - __builtin_clzll(mag);        /* index of leading bit */
    int e_lead = top + exp2;                    /* value in [2^e_lead, 2^(e_lead+1)) */
    int lsb_exp = e_lead - (f.p - 1);           /* exponent of the last kept bit */
    if (lsb_exp < f.emin - (f.p - 1)) lsb_exp = f.emin - (f.p - 1); /* subnormal */
    int shift = lsb_exp - exp2;                 /* bits of mag to drop */
    uint64_t kept;
    int guard = 0, sticky = sticky_in;
    if (shift <= 0) {
        kept = mag << (-shift);                 /* exact, no rounding */
        if (sticky_in) { /* below the last bit by less than one mag unit */
            /* remaining bits are zero, sticky only; no round-up possible */
        }
    } else if (shift > 64) {
        kept = 0; guard = 0; sticky = 1;
    } else {
        kept = (shift == 64) ? 0 : (mag >> shift);
        uint64_t rem = (shift == 64) ? mag : (mag & ((1ull << shift) - 1));
        uint64_t half = 1ull << (shift - 1);
        guard = (rem & half) != 0;
        sticky = sticky || ((rem & (half - 1)) != 0);
    }
    if (guard && (sticky || (kept & 1))) kept += 1;
    double v = ldexp((double)kept, lsb_exp);
    if (v >= ldexp(1.0, f.emax + 1)) v = INFINITY;
    return neg ? -v : v;
}

/* Round an exact double once to format f (RNE), returning the result as a double. */
static double round_double(double d, fmt_t f) {
    if (d == 0.0 || isnan(d) || isinf(d)) return d;
    int e;
    double m = frexp(fabs(d), &e);              /* |d| = m*2^e, m in [0.5,1) */
    uint64_t mag = (uint64_t)ldexp(m, 53);      /* exact: 53-bit integer */
    return round_mag(mag, e - 53, 0, d < 0, f);
}

static uint16_t double_to_bf16_bits(double v) { /* v exactly representable in bf16 */
    return orc_f32_to_bf16((float)v);
}

static uint16_t double_to_f16_bits(double v) { /* v exactly representable in f16 (or inf/nan) */
    uint16_t s = signbit(v) ? 0x8000 : 0;
    double a = fabs(v);
    if (isnan(v)) return 0x7e00;
    if (isinf(a)) return s | 0x7c00;
    if (a == 0.0) return s;
    int e;
    frexp(a, &e);                               /* a in [2^(e-1), 2^e) */
    int E = e - 1;
    if (E < -14) {                              /* subnormal: a = m * 2^-24 */
        return s | (uint16_t)ldexp(a, 24);
    }
    uint32_t m = (uint32_t)ldexp(a, 10 - E) - 1024u;
    return s | (uint16_t)((E + 15) << 10) | (uint16_t)m;
}

/* Round a float once to dtype dt and return it widened back to float. */
float orc_round_to(float x, int dt) {
    if (dt == DT_F32) return x;
    if (dt == DT_BF16) return orc_bf16_to_f32(orc_f32_to_bf16(x));
    return (float)round_double((double)x, FMT_F16);
}

/* ----------------------------------------------------------------------- */
/* exact multi-limb accumulator: value = sum(limb[i] * 2^(32 i + ACC_EBASE)) */
/* ----------------------------------------------------------------------- */

#define ACC_LIMBS 12
#define ACC_EBASE (-200)

typedef struct { int64_t limb[ACC_LIMBS + 2]; } bigacc_t;

static void acc_add(bigacc_t* a, int64_t m, int e) {   /* a += m * 2^e, |m| < 2^40 */
    if (m == 0) return;
    int sh = e - ACC_EBASE;
    int li = sh >> 5, off = sh & 31;
    __int128 v = (__int128)m * ((__int128)1 << off);
    int64_t lo = (int64_t)(v & 0xffffffff);
    __int128 hi = (v - lo) >> 32;
    a->limb[li] += lo;
    a->limb[li + 1] += (int64_t)(hi & 0xffffffff);
    a->limb[li + 2] += (int64_t)((hi - (hi & 0xffffffff)) >> 32);
}

/* Round the accumulator (times 2^scale_exp) to format f. */
static double acc_round(const bigacc_t* a, int scale_exp, fmt_t f) {
    uint32_t d[ACC_LIMBS + 2];
    __int128 carry = 0;
    for (int i = 0; i < ACC_LIMBS + 2; ++i) {
        __int128 t = (__int128)a->limb[i] + carry;
        int64_t low = (int64_t)(t & 0xffffffff);
        d[i] = (uint32_t)low;
        carry = (t - low) >> 32;
    }
    int neg = carry < 0;
    if (neg) { /* two's complement negate over the limbs */
        uint64_t c = 1;
        for (int i = 0; i < ACC_LIMBS + 2; ++i) {
            uint64_t t = (uint64_t)(uint32_t)~d[i] + c;
            d[i] = (uint32_t)t;
            c = t >> 32;
        }
    }
    int hi = -1;
    for (int i = ACC_LIMBS + 1; i >= 0; --i) if (d[i]) { hi = i; break; }
    if (hi < 0) return 0.0;
    /* take the top 64 bits (three limbs) and a sticky from the rest */
    uint64_t mag = 0;
    int used = 0;
    int base = hi;
    for (int i = hi; i >= 0 && used < 2; --i, ++used) { mag = (mag << 32) | d[i]; base = i; }
    int sticky = 0;
    for (int i = base - 1; i >= 0; --i) if (d[i]) { sticky = 1; break; }
    return round_mag(mag, 32 * base + ACC_EBASE + scale_exp, sticky, neg, f);
}

/* decompose a finite value of dtype dt into m * 2^e with an integer m */
static void decompose(float v, int* m, int* e) {
    if (v == 0.0f) { *m = 0; *e = 0; return; }
    int ex;
    float fr = frexpf(v, &ex);                  /* v = fr * 2^ex, |fr| in [0.5,1) */
    *m = (int)ldexpf(fr, 24);                   /* exact for any float */
    *e = ex - 24;
}

static float load_val(const void* x, int dt, size_t i) {
    if (dt == DT_F32) return ((const float*)x)[i];
    if (dt == DT_BF16) return orc_bf16_to_f32(((const uint16_t*)x)[i]);
    return orc_f16_to_f32(((const uint16_t*)x)[i]);
}

static void store_val(void* y, int dt, size_t i, double v) { /* v representable in dt */
    if (dt == DT_F32) ((float*)y)[i] = (float)v;
    else if (dt == DT_BF16) ((uint16_t*)y)[i] = double_to_bf16_bits(v);
    else ((uint16_t*)y)[i] = double_to_f16_bits(v);
}

/* ----------------------------------------------------------------------- */
/* Hadamard                                                                 */
/* ----------------------------------------------------------------------- */

/* H4 of _int4/eager.py:32-36; H_G = kron^(log4 G)(H4) / sqrt(G)
 * (_int4/eager.py:38-44).  Entry (i, j) is the product over base-4 digits of
 * H4[i_d][j_d], divided by sqrt(G).  Returns the +-1 sign (as int). */
static const int H4[4][4] = {{1, 1, 1, -1}, {1, 1, -1, 1}, {1, -1, 1, 1}, {-1, 1, 1, 1}};

int orc_hadamard_sign(int G, int i, int j) {
    int s = 1;
    for (int g = G; g > 1; g >>= 2) { s *= H4[i & 3][j & 3]; i >>= 2; j >>= 2; }
    return s;
}

static int log4i(int G) { int n = 0; while ((1 << (2 * n)) < G) ++n; return n; }

/* Dense H_G (float, entries +-1/sqrt(G)), row-major [G, G]. */
void orc_hadamard(int G, float* out) {
    float inv = 1.0f / sqrtf((float)G);
    for (int i = 0; i < G; ++i)
        for (int j = 0; j < G; ++j) out[(size_t)i * G + j] = orc_hadamard_sign(G, i, j) * inv;
}

/* ----------------------------------------------------------------------- */
/* a5: rotation, _int4/eager.py:65-79 (activation) and :49-62 (weight;      */
/* identical because H is symmetric).  out[m, gG+j] = RNE_dt(sum_i x[m,gG+i] */
/* * H[i,j]), exactly rounded.  Returns the number of groups that needed    */
/* the exact integer accumulator.                                           */
/* ----------------------------------------------------------------------- */

static void fwht_exact_f64(double* v, int G) {
    /* radix-4 stages over base-4 digits; each stage out_j = S - 2*v[3-j]
     * (H4 v = (sum v) 1 - 2 reverse(v)); exact in fp64 when the caller's
     * span check holds. */
    for (int stride = 1; stride < G; stride <<= 2) {
        for (int base = 0; base < G; ++base) {
            if ((base / stride) & 3) continue;
            double a = v[base], b = v[base + stride], c = v[base + 2 * stride], d = v[base + 3 * stride];
            double S = a + b + c + d;
            v[base] = S - 2.0 * d;
            v[base + stride] = S - 2.0 * c;
            v[base + 2 * stride] = S - 2.0 * b;
            v[base + 3 * stride] = S - 2.0 * a;
        }
    }
}

int orc_rotate(const void* x, int dt, int M, int K, int G, void* out) {
    int nexact = 0;
    fmt_t f = fmt_of(dt);
    int lg = log4i(G);
    int halflog = lg;                          /* sqrt(G) = 2^lg */
#pragma omp parallel reduction(+ : nexact)
    {
    double* v = (double*)malloc(sizeof(double) * G);
    int* mm = (int*)malloc(sizeof(int) * G);
    int* ee = (int*)malloc(sizeof(int) * G);
#pragma omp for schedule(static)
    for (int m = 0; m < M; ++m) {
        for (int g = 0; g < K / G; ++g) {
            size_t base = (size_t)m * K + (size_t)g * G;
            int emax = -100000, emin = 100000;
            for (int i = 0; i < G; ++i) {
                float xv = load_val(x, dt, base + i);
                decompose(xv, &mm[i], &ee[i]);
                if (mm[i] != 0) {
                    unsigned am = (unsigned)abs(mm[i]);
                    int lead = ee[i] + 31 - __builtin_clz(am);   /* leading set bit */
                    int low = ee[i] + __builtin_ctz(am);         /* lowest set bit */
                    if (lead > emax) emax = lead;
                    if (low < emin) emin = low;
                }
                v[i] = (double)xv;
            }
            /* every partial sum is a multiple of 2^emin and below 2^(emax+1+2*lg);
             * it fits 53 bits iff (emax + 1 + 2*lg) - emin <= 53 */
            int exact64 = (emax == -100000) || ((emax + 1 + 2 * lg) - emin <= 53);
            if (exact64) {
                fwht_exact_f64(v, G);
                for (int j = 0; j < G; ++j) {
                    double s = ldexp(v[j], -halflog); /* exact */
                    store_val(out, dt, base + j, round_double(s, f));
                }
            } else {
                ++nexact;
                for (int j = 0; j < G; ++j) {
                    bigacc_t a;
                    memset(&a, 0, sizeof(a));
                    for (int i = 0; i < G; ++i)
                        acc_add(&a, (int64_t)orc_hadamard_sign(G, i, j) * mm[i], ee[i]);
                    store_val(out, dt, base + j, acc_round(&a, -halflog, f));
                }
            }
        }
    }
    free(v); free(mm); free(ee);
    }
    return nexact;
}

/* Reference-free exact dot product of one output element (for self-checks). */
double orc_rotate_one_exact(const void* x, int dt, int K, int G, int m, int col) {
    int g = col / G, j = col % G;
    bigacc_t a;
    memset(&a, 0, sizeof(a));
    for (int i = 0; i < G; ++i) {
        int mi, ei;
        decompose(load_val(x, dt, (size_t)m * K + (size_t)g * G + i), &mi, &ei);
        acc_add(&a, (int64_t)orc_hadamard_sign(G, i, j) * mi, ei);
    }
    return acc_round(&a, -log4i(G), fmt_of(dt));
}

/* ----------------------------------------------------------------------- */
/* a6 / a7: quantize_signed_int4_rowwise + _round_int4 + pack               */
/* (_int4/eager.py:104-120, _int4/_codec.py:19-25).                         */
/*   absmax = max|x| clamped to dt(1e-10)           eager.py:117            */
/*   s      = RNE_dt(fl32(absmax / 7))              eager.py:118            */
/*   q      = clamp(rint_even(RNE_dt(fl32(x/s))), -7, 7)  eager.py:119,109  */
/*   stochastic (noise u != NULL): q = clamp(floor(RNE_dt(fl32(t + u))))    */
/*   with t = RNE_dt(fl32(x/s))                     eager.py:105-108        */
/* A NaN quotient (0/0 when the dtype flushes the 1e-10 clamp to 0, as f16  */
/* does) converts to code 0, as float->int8 does on the GPU.                */
/* ----------------------------------------------------------------------- */

static float clamp_floor_value(int dt) {
    /* the python scalar 1e-10 converted to the tensor dtype */
    if (dt == DT_F32) return 1e-10f;
    if (dt == DT_BF16) return (float)round_double(1e-10, FMT_BF16);
    return (float)round_double(1e-10, FMT_F16);  /* underflows to 0 */
}

static int code_of(float t, int stochastic, float u, int dt) {
    float r;
    if (stochastic) {
        r = floorf(orc_round_to(t + u, dt));
    } else {
        r = nearbyintf(t);                     /* default mode: ties to even */
    }
    if (isnan(r)) return 0;
    if (r < -7.0f) r = -7.0f;
    if (r > 7.0f) r = 7.0f;
    return (int)r;
}

void orc_quant_rows(const void* xr, int dt, int M, int K, const void* noise,
                    int8_t* packed, float* scales, int8_t* codes /* nullable, [M,K] */) {
    float lo = clamp_floor_value(dt);
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; ++m) {
        size_t base = (size_t)m * K;
        float a = 0.0f;
        for (int k = 0; k < K; ++k) {
            float v = fabsf(load_val(xr, dt, base + k));
            if (v > a) a = v;
        }
        if (a < lo) a = lo;
        float s = orc_round_to(a / 7.0f, dt);
        scales[m] = s;
        for (int k = 0; k < K; k += 2) {
            int q2[2];
            for (int h = 0; h < 2; ++h) {
                float t = orc_round_to(load_val(xr, dt, base + k + h) / s, dt);
                float u = noise ? load_val(noise, dt, base + k + h) : 0.0f;
                q2[h] = code_of(t, noise != NULL, u, dt);
                if (codes) codes[base + k + h] = (int8_t)q2[h];
            }
            packed[base / 2 + k / 2] = (int8_t)((q2[0] & 0xF) | ((q2[1] & 0xF) << 4));
        }
    }
}

/* a3 activation half: rotate then quantize (_int4/eager.py:191-195). */
int orc_rotquant(const void* x, int dt, int M, int K, int G, const void* noise,
                 int8_t* packed, float* scales, void* xr_out /* nullable */) {
    size_t esz = dt == DT_F32 ? 4 : 2;
    void* xr = xr_out ? xr_out : malloc((size_t)M * K * esz);
    int n = orc_rotate(x, dt, M, K, G, xr);
    orc_quant_rows(xr, dt, M, K, noise, packed, scales, NULL);
    if (!xr_out) free(xr);
    return n;
}

/* ----------------------------------------------------------------------- */
/* W8A8 tier: quantize_signed_int8_rowwise (_int4/int8_eager.py:22-28)     */
/*   a = max(max_k |xr|, dt(1e-10));  s = RNE_dt(fl32(a / 127))            */
/*   q = clamp(rint_even(RNE_dt(fl32(xr / s))), -127, 127)                 */
/* stored as plain int8 [M, K] (_int4/int8_eager.py:31-47).  A NaN quotient */
/* (0/0 for an f16 row of zeros) gives code 0.                             */
/* ----------------------------------------------------------------------- */

void orc_quant_rows8(const void* xr, int dt, int M, int K, int8_t* q8, float* scales) {
    float lo = clamp_floor_value(dt);
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; ++m) {
        size_t base = (size_t)m * K;
        float a = 0.0f;
        for (int k = 0; k < K; ++k) {
            float v = fabsf(load_val(xr, dt, base + k));
            if (v > a) a = v;
        }
        if (a < lo) a = lo;
        float s = orc_round_to(a / 127.0f, dt);
        scales[m] = s;
        for (int k = 0; k < K; ++k) {
            float t = orc_round_to(load_val(xr, dt, base + k) / s, dt);
            float r = nearbyintf(t);               /* ties to even */
            int c = 0;
            if (!isnan(r)) c = r < -127.0f ? -127 : (r > 127.0f ? 127 : (int)r);
            q8[base + k] = (int8_t)c;
        }
    }
}

/* convrot_w8a8_linear's activation half / quantize_convrot_w8a8_weight     */
/* (_int4/int8_eager.py:31-47, 81-83): rotate then quantize to int8.        */
int orc_rotquant8(const void* x, int dt, int M, int K, int G, int8_t* q8, float* scales,
                  void* xr_out /* nullable */) {
    size_t esz = dt == DT_F32 ? 4 : 2;
    void* xr = xr_out ? xr_out : malloc((size_t)M * K * esz);
    int n = orc_rotate(x, dt, M, K, G, xr);
    orc_quant_rows8(xr, dt, M, K, q8, scales);
    if (!xr_out) free(xr);
    return n;
}

/* W8A8 accumulators acc[m,n] = sum_k x[m,k] * w[n,k], exact in int64 and    */
/* returned as int32 (|acc| <= 127^2 K < 2^31 for K < 133000).              */
void orc_int8_gemm(const int8_t* X, const int8_t* W, int M, int N, int K, int32_t* acc) {
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; ++m) {
        const int8_t* a = X + (size_t)m * K;
        for (int n = 0; n < N; ++n) {
            const int8_t* b = W + (size_t)n * K;
            int64_t s = 0;
            for (int k = 0; k < K; ++k) s += (int32_t)a[k] * b[k];
            acc[(size_t)m * N + n] = (int32_t)s;
        }
    }
}

/* ----------------------------------------------------------------------- */
/* a7 unpack (_int4/_codec.py:28-36) and a8 int GEMM (_int4/eager.py:160-162) */
/* ----------------------------------------------------------------------- */

void orc_unpack(const int8_t* packed, size_t nbytes, int8_t* codes) {
    for (size_t j = 0; j < nbytes; ++j) {
        int b = (uint8_t)packed[j];
        int lo = b & 0xF, hi = (b >> 4) & 0xF;
        codes[2 * j] = (int8_t)(lo >= 8 ? lo - 16 : lo);
        codes[2 * j + 1] = (int8_t)(hi >= 8 ? hi - 16 : hi);
    }
}

/* acc[m,n] = sum_k qx[m,k] * qw[n,k], exact (|acc| <= 64 K). */
void orc_int_gemm(const int8_t* Xp, const int8_t* Wp, int M, int N, int K, int32_t* acc) {
    int8_t* xc = (int8_t*)malloc((size_t)M * K);
    int8_t* wc = (int8_t*)malloc((size_t)N * K);
    orc_unpack(Xp, (size_t)M * K / 2, xc);
    orc_unpack(Wp, (size_t)N * K / 2, wc);
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; ++m) {
        const int8_t* a = xc + (size_t)m * K;
        for (int n = 0; n < N; ++n) {
            const int8_t* b = wc + (size_t)n * K;
            int32_t s = 0;
            for (int k = 0; k < K; ++k) s += (int32_t)a[k] * b[k];
            acc[(size_t)m * N + n] = s;
        }
    }
    free(xc); free(wc);
}

/* ----------------------------------------------------------------------- */
/* a8 epilogues                                                             */
/* ----------------------------------------------------------------------- */

/* fp32 chain: o = fl32(fl32(fl32(acc*xs)*ws) + b).  For out_dtype f32 this is
 * the eager int4_linear computation exactly (_int4/eager.py:164-168 with
 * out_dtype f32: the integer matmul is exact in f32 because |acc| < 2^24).
 * For the W8A8 tier it is the reference kernel's epilogue
 * ((float)acc * xscale * ws + bias, _int4/int4_gemm.hip:555-558) and the eager
 * one (_int4/int8_eager.py:87-91) whenever its fp32 matmul is exact
 * (|partial sums| < 2^24); (float)acc rounds to nearest even above that.
 * out_bf16 != 0 rounds the final value once to bf16 (bits in out16). */
void orc_epilogue_f32(const int32_t* acc, const float* xs, const float* ws, const float* bias,
                      int M, int N, int out_bf16, float* out32, uint16_t* out16) {
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            volatile float t = (float)acc[(size_t)m * N + n] * xs[m];
            volatile float u = t * ws[n];
            float v = bias ? (float)(u + bias[n]) : u;
            if (out_bf16) out16[(size_t)m * N + n] = orc_f32_to_bf16(v);
            else out32[(size_t)m * N + n] = v;
        }
}

/* bf16 chain of the eager path with out_dtype bf16 (_int4/eager.py:162-168):
 *   o1 = RNE(acc); o2 = RNE(o1*bf16(xs)); o3 = RNE(o2*bf16(ws)); o4 = RNE(o3+bf16(b))
 * each product/sum formed in fp32 and rounded to bf16, as torch does. */
void orc_epilogue_eager_bf16(const int32_t* acc, const float* xs, const float* ws, const float* bias,
                             int M, int N, uint16_t* out16) {
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; ++m) {
        float xsb = orc_round_to(xs[m], DT_BF16);
        for (int n = 0; n < N; ++n) {
            float wsb = orc_round_to(ws[n], DT_BF16);
            float o1 = orc_round_to((float)acc[(size_t)m * N + n], DT_BF16);
            float o2 = orc_round_to(o1 * xsb, DT_BF16);
            float o3 = orc_round_to(o2 * wsb, DT_BF16);
            float o4 = bias ? orc_round_to(o3 + orc_round_to(bias[n], DT_BF16), DT_BF16) : o3;
            out16[(size_t)m * N + n] = orc_f32_to_bf16(o4);
        }
    }
}

/* threads the row loops above use (OpenMP; OMP_NUM_THREADS) */
int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* scalar conversion entry points for the python side */
uint16_t orc_round_double_bits(double v, int dt) {
    double r = round_double(v, fmt_of(dt));
    return dt == DT_F16 ? double_to_f16_bits(r) : double_to_bf16_bits(r);
}
