/* iro_oracle.c -- CPU restatement of irodori-c's int8 W8A8 path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker): never linked into, loaded by or
 * called from the HIP product library.
 *
 * Build with -ffp-contract=off and without -ffast-math: every float
 * operation below rounds exactly where it is written.  Where the reference's
 * fast-math build fuses a multiply-add, this file calls fmaf() explicitly.
 * Each function cites the reference lines it restates.
 */
#include "iro_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* Constants GCC 11 folds into the fast-math build of ops.c/dacvae.c:
 *   x / 255.0f   ->  x * fl(1/255)            0x3B808081
 *   1 / (d/255)  ->  fl(1/fl(1/255)) / d       0x437EFFFF (254.99998)
 *   255 / (d/255)->  fl(255/fl(1/255)) / d     0x477E00FF (65024.996)
 *   x / 127.0f   ->  x * fl(1/127)            0x3C010204
 *   1 / (a/127)  ->  127 / a                   0x42FE0000
 */
static float f32_bits(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}
#define C_INV255 f32_bits(0x3B808081u)
#define C_255_OVER_INV255 f32_bits(0x437EFFFFu)
#define C_255_OVER_INV255_B f32_bits(0x477E00FFu)
#define C_INV127 f32_bits(0x3C010204u)

static int clamp_i(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* Round-to-nearest-even, as nearbyintf / cvtss2si / vrndscaleps $12 under
   the default MXCSR. */
static float rne(float v) { return rintf(v); }

/* ---- weights: ops.c:259-293 ------------------------------------------ */

static void weight_row(int conv, const float *row, int K, int8_t *q,
                       float *scale_out, int32_t *colsum_out) {
    float amax = 0.0f;
    for (int k = 0; k < K; k++) {
        float a = fabsf(row[k]);
        if (a > amax) amax = a;
    }
    float scale, inv;
    if (conv == ORC_GCC_FASTMATH) {
        if (amax > 0.0f) {
            scale = amax * C_INV127;
            inv = 127.0f / amax;
        } else {
            scale = 1.0f;
            inv = 1.0f;
        }
    } else {
        scale = amax > 0.0f ? amax / 127.0f : 1.0f;
        inv = 1.0f / scale;
    }
    int32_t sum = 0;
    for (int k = 0; k < K; k++) {
        int v = (int)rne(row[k] * inv);
        v = clamp_i(v, -127, 127);
        q[k] = (int8_t)v;
        sum += v;
    }
    *scale_out = scale;
    *colsum_out = sum;
}

int orc_weight_quantize(int conv, const float *w, int N, int K,
                        int8_t *q, float *scale, int32_t *colsum) {
    if (!w || !q || !scale || !colsum || N <= 0 || K <= 0) return -1;
    for (int n = 0; n < N; n++)
        weight_row(conv, w + (size_t)n * K, K, q + (size_t)n * K, &scale[n],
                   &colsum[n]);
    return 0;
}

int orc_weight_quantize_transposed(int conv, const float *w, int N, int K,
                                   int8_t *q, float *scale, int32_t *colsum) {
    if (!w || N <= 0 || K <= 0) return -1;
    float *t = malloc(sizeof(float) * (size_t)N * K);
    if (!t) return -1;
    for (int k = 0; k < K; k++)
        for (int n = 0; n < N; n++) t[(size_t)n * K + k] = w[(size_t)k * N + n];
    int rc = orc_weight_quantize(conv, t, N, K, q, scale, colsum);
    free(t);
    return rc;
}

/* ---- activations: ops.c:321-348 -------------------------------------- */

typedef struct {
    float s, inv, zpf;
    int zp;
} RowQuant;

/* Scale and zero point of a row whose range (with zero) is [lo, hi]. */
static RowQuant row_params(int conv, float lo, float hi) {
    RowQuant r;
    float d = hi - lo;
    if (conv == ORC_GCC_FASTMATH) {
        r.s = d * C_INV255;
        if (!(r.s > 0.0f)) {
            r.s = 1.0f;
            r.inv = 1.0f;
            r.zp = clamp_i((int)rne(-lo), 0, 255);
        } else {
            r.inv = C_255_OVER_INV255 / d;
            r.zp = clamp_i((int)rne(-(lo * r.inv)), 0, 255);
        }
    } else {
        r.s = d / 255.0f;
        if (!(r.s > 0.0f)) r.s = 1.0f;
        r.inv = 1.0f / r.s;
        r.zp = clamp_i((int)rne(-lo * r.inv), 0, 255);
    }
    r.zpf = (float)r.zp;
    return r;
}

static uint8_t quant_code(int conv, float x, const RowQuant *r) {
    float v = conv == ORC_GCC_FASTMATH ? rne(fmaf(x, r->inv, r->zpf))
                                        : rne(x * r->inv + r->zpf);
    v = v < 0.0f ? 0.0f : v;
    v = v > 255.0f ? 255.0f : v;
    return (uint8_t)v;
}

static void row_range(const float *row, int K, float *lo_out, float *hi_out) {
    float lo = 0.0f, hi = 0.0f;
    for (int k = 0; k < K; k++) {
        lo = row[k] < lo ? row[k] : lo;
        hi = row[k] > hi ? row[k] : hi;
    }
    *lo_out = lo;
    *hi_out = hi;
}

void orc_quantize_rows(int conv, const float *x, int M, int K,
                       uint8_t *q, float *scale, int32_t *zero) {
    for (int m = 0; m < M; m++) {
        const float *row = x + (size_t)m * K;
        uint8_t *qrow = q + (size_t)m * K;
        float lo, hi;
        row_range(row, K, &lo, &hi);
        RowQuant r = row_params(conv, lo, hi);
        for (int k = 0; k < K; k++) qrow[k] = quant_code(conv, row[k], &r);
        scale[m] = r.s;
        zero[m] = r.zp;
    }
}

/* ops.c:427-442: r = x - s1*(q1 - zp1), then requantize r. */
void orc_quantize_rows_residual(int conv, const float *x, int M, int K,
                                uint8_t *q1, float *scale1, int32_t *zero1,
                                float *residual,
                                uint8_t *q2, float *scale2, int32_t *zero2) {
    float *r = residual;
    float *own = NULL;
    if (!r) {
        own = malloc(sizeof(float) * (size_t)K);
        if (!own) return;
    }
    orc_quantize_rows(conv, x, M, K, q1, scale1, zero1);
    for (int m = 0; m < M; m++) {
        const float *row = x + (size_t)m * K;
        const uint8_t *qrow = q1 + (size_t)m * K;
        float *rrow = own ? own : r + (size_t)m * K;
        const float s = scale1[m];
        const float zp = (float)zero1[m];
        for (int k = 0; k < K; k++) {
            if (conv == ORC_GCC_FASTMATH)
                rrow[k] = fmaf(s, zp - (float)qrow[k], row[k]);
            else
                rrow[k] = row[k] - s * ((float)qrow[k] - zp);
        }
        if (own)
            orc_quantize_rows(conv, own, 1, K, q2 + (size_t)m * K, scale2 + m,
                              zero2 + m);
    }
    if (!own) orc_quantize_rows(conv, r, M, K, q2, scale2, zero2);
    free(own);
}

/* ---- integer GEMM: ops.c:351-364 ------------------------------------- */

void orc_gemm_u8s8(const uint8_t *a, const int8_t *b, int32_t *c,
                   int M, int N, int K, int threads) {
#ifdef _OPENMP
    if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) num_threads(threads)
#else
    (void)threads;
#endif
    for (int m = 0; m < M; m++) {
        const uint8_t *arow = a + (size_t)m * K;
        int32_t *crow = c + (size_t)m * N;
        for (int n = 0; n < N; n++) {
            const int8_t *brow = b + (size_t)n * K;
            int32_t acc = 0;
            for (int k = 0; k < K; k++) acc += (int32_t)arow[k] * (int32_t)brow[k];
            crow[n] = acc;
        }
    }
}

/* ---- epilogue: ops.c:468-490 ------------------------------------------ */

void orc_epilogue(int conv, const int32_t *acc, const float *sx,
                  const int32_t *zx, const float *sw, const int32_t *colsum,
                  const float *bias, float *y, int M, int N, int accumulate) {
    const int fast = conv == ORC_GCC_FASTMATH;
    for (int m = 0; m < M; m++) {
        const int32_t *crow = acc + (size_t)m * N;
        float *yrow = y + (size_t)m * N;
        for (int n = 0; n < N; n++) {
            const float t = (float)(crow[n] - zx[m] * colsum[n]);
            const float c = sx[m] * sw[n];
            if (accumulate && bias) {
                yrow[n] = fast ? fmaf(t, c, yrow[n] + bias[n])
                               : yrow[n] + (t * c + bias[n]);
            } else if (accumulate) {
                yrow[n] = fast ? fmaf(t, c, yrow[n]) : yrow[n] + t * c;
            } else if (bias) {
                yrow[n] = fast ? fmaf(t, c, bias[n]) : t * c + bias[n];
            } else {
                yrow[n] = t * c;
            }
        }
    }
}

void orc_int8_linear_ex(int conv, const uint8_t *q, const float *sx,
                        const int32_t *zx, const int8_t *wq, const float *sw,
                        const int32_t *colsum, int N, int K,
                        const float *bias, float *y, int M, int32_t *work,
                        int accumulate, int threads) {
    orc_gemm_u8s8(q, wq, work, M, N, K, threads);
    orc_epilogue(conv, work, sx, zx, sw, colsum, bias, y, M, N, accumulate);
}

/* ---- known answer: ops.c:375-398 ---------------------------------------- */

void orc_selfcheck_kat(uint8_t *a, int8_t *b, int32_t *want) {
    enum { M = 3, N = 5, K = 64 };
    for (int i = 0; i < M * K; i++) a[i] = (uint8_t)(i % 3 == 0 ? 255 : 200 + i % 50);
    for (int i = 0; i < N * K; i++)
        b[i] = (int8_t)(i % 4 == 0 ? 127 : (i % 4 == 1 ? -127 : 90 - i % 60));
    orc_gemm_u8s8(a, b, want, M, N, K, 1);
}

/* ---- SwiGLU gate: ops.c:781-784 (strict build) ------------------------ */

void orc_silu_mul(float *x, const float *g, size_t n) {
    for (size_t i = 0; i < n; i++) x[i] = (x[i] / (1.0f + expf(-x[i]))) * g[i];
}

/* ---- glibc expf restated ------------------------------------------------ */

/* 2^(i/32) as doubles, minus i << 47 so the exponent of k can be added. */
static const uint64_t EXP2_TAB[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

float orc_expf_restated(float x) {
    if (x != x) return x + x;
    if (x > 0x1.62e42ep6f) return INFINITY;
    if (x < -0x1.9fe368p6f) return 0.0f;
    const double invln2n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    double kd = fma(invln2n, xd, shift);
    uint64_t ki;
    memcpy(&ki, &kd, sizeof ki);
    kd -= shift;
    const double r = fma(invln2n, xd, -kd);
    uint64_t t = EXP2_TAB[ki % 32] + (ki << 47);
    double s;
    memcpy(&s, &t, sizeof s);
    const double z = fma(c0, r, c1);
    const double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    return (float)(y * s);
}

long long orc_expf_mismatches(int threads) {
    long long bad = 0;
#ifdef _OPENMP
    if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) reduction(+ : bad) num_threads(threads)
#else
    (void)threads;
#endif
    for (long long hi = 0; hi < 65536; hi++) {
        for (uint32_t lo = 0; lo < 65536; lo++) {
            const uint32_t u = ((uint32_t)hi << 16) | lo;
            float x;
            memcpy(&x, &u, sizeof x);
            const float a = orc_expf_restated(x), b = expf(x);
            uint32_t ua, ub;
            memcpy(&ua, &a, 4);
            memcpy(&ub, &b, 4);
            if (ua != ub && !(a != a && b != b)) bad++;
        }
    }
    return bad;
}

/* Order-independent digest of orc_expf_restated over every float input:
   the sum (mod 2^64) of (bits(x) * 0x9E3779B97F4A7C15) ^ (bits(e) *
   0xC2B2AE3D27D4EB4F), with every NaN result counted as 0x7FC00000.  The
   device restatement's self-check computes the same sum. */
unsigned long long orc_expf_digest(int threads) {
    unsigned long long sum = 0;
#ifdef _OPENMP
    if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) reduction(+ : sum) num_threads(threads)
#else
    (void)threads;
#endif
    for (long long hi = 0; hi < 65536; hi++) {
        for (uint32_t lo = 0; lo < 65536; lo++) {
            const uint32_t u = ((uint32_t)hi << 16) | lo;
            float x;
            memcpy(&x, &u, sizeof x);
            const float e = orc_expf_restated(x);
            uint32_t ue;
            memcpy(&ue, &e, 4);
            if (e != e) ue = 0x7FC00000u;
            sum += ((unsigned long long)u * 0x9E3779B97F4A7C15ull) ^
                   ((unsigned long long)ue * 0xC2B2AE3D27D4EB4Full);
        }
    }
    return sum;
}

/* The same digest form for the host's sqrtf(x) and 1.0f / x (IEEE, as the
   strict reference computes them) over every float input. */
void orc_fp32_digests(int threads, unsigned long long *sqrt_digest,
                      unsigned long long *recip_digest) {
    unsigned long long hs = 0, hq = 0;
#ifdef _OPENMP
    if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) reduction(+ : hs, hq) num_threads(threads)
#else
    (void)threads;
#endif
    for (long long hi = 0; hi < 65536; hi++) {
        for (uint32_t lo = 0; lo < 65536; lo++) {
            const uint32_t u = ((uint32_t)hi << 16) | lo;
            float x;
            memcpy(&x, &u, sizeof x);
            const float r = sqrtf(x), q = 1.0f / x;
            uint32_t ur, uq;
            memcpy(&ur, &r, 4);
            memcpy(&uq, &q, 4);
            if (r != r) ur = 0x7FC00000u;
            if (q != q) uq = 0x7FC00000u;
            hs += ((unsigned long long)u * 0x9E3779B97F4A7C15ull) ^
                  ((unsigned long long)ur * 0xC2B2AE3D27D4EB4Full);
            hq += ((unsigned long long)u * 0x9E3779B97F4A7C15ull) ^
                  ((unsigned long long)uq * 0xC2B2AE3D27D4EB4Full);
        }
    }
    *sqrt_digest = hs;
    *recip_digest = hq;
}

/* ---- adaLN RMSNorm modulate: dit.c:593-606 ------------------------------ */

/* h = x * inv * (1 + scale[b]) + shift[b] for the rows of branch b = row / S,
   inv = 1 / sqrtf(ms / D + eps), ms the row's sum of squares accumulated in
   order d = 0 .. D-1 (each square rounded, then added), as the strict build
   evaluates dit.c:597-603. */
void orc_adaln_apply(const float *x, const float *shift, const float *scale, int B, int S, int D,
                     float eps, float *h) {
    for (int b = 0; b < B; b++) {
        for (int s = 0; s < S; s++) {
            const float *row = x + ((size_t)b * S + s) * D;
            float *out = h + ((size_t)b * S + s) * D;
            float ms = 0.0f;
            for (int d = 0; d < D; d++) {
                const float sq = row[d] * row[d];
                ms = ms + sq;
            }
            const float inv = 1.0f / sqrtf(ms / (float)D + eps);
            const float *sh = shift + (size_t)b * D, *sc = scale + (size_t)b * D;
            for (int d = 0; d < D; d++) {
                const float t = row[d] * inv;
                const float m = t * (1.0f + sc[d]);
                out[d] = m + sh[d];
            }
        }
    }
}

/* ---- glibc expm1f / tanhf and the adaLN parameters: dit.c:543-588 ------- */

static inline uint32_t orc_fbits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static inline float orc_bitsf(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* The expm1f / tanhf below follow fdlibm's s_expm1f.c and s_tanhf.c, whose
 * notice is preserved as its licence asks:
 *
 * ====================================================
 * Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
 *
 * Developed at SunPro, a Sun Microsystems, Inc. business.
 * Permission to use, copy, modify, and distribute this
 * software is freely granted, provided that this notice
 * is preserved.
 * ====================================================
 *
 * (float conversion by Ian Lance Taylor, Cygnus Support.)
 */
/* expm1f and tanhf as glibc 2.35 computes them: the float port of fdlibm 5.3's
   s_expm1f.c (argument reduction by ln2 in two pieces, a degree-5 rational
   correction in x^2/2 with the published Q1..Q5) and s_tanhf.c (tanh through
   expm1 of 2|x|).  Equal to libm on every float input
   (tests/test_oracle_pins.py::test_tanhf_restatement_equals_libm_on_every_float). */
float orc_expm1f(float x) {
    const float one = 1.0f, tiny = 1.0e-30f, huge = 1.0e+30f;
    const float o_threshold = 8.8721679688e+01f, ln2_hi = 6.9313812256e-01f,
                ln2_lo = 9.0580006145e-06f, invln2 = 1.4426950216e+00f;
    const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f,
                Q4 = 4.0082177293e-06f, Q5 = -2.0109921195e-07f;
    float y, hi, lo, c = 0, t, e, hxs, hfx, r1;
    int32_t k, xsb;
    uint32_t hx = orc_fbits(x);
    xsb = hx & 0x80000000;
    y = xsb == 0 ? x : -x;
    hx &= 0x7fffffff;
    if (hx >= 0x4195b844) {
        if (hx >= 0x42b17218) {
            if (hx > 0x7f800000) return x + x;
            if (hx == 0x7f800000) return xsb == 0 ? x : -1.0f;
            if (x > o_threshold) return huge * huge;
        }
        if (xsb != 0) return tiny - one;
    }
    if (hx > 0x3eb17218) {
        if (hx < 0x3F851592) {
            if (xsb == 0) { hi = x - ln2_hi; lo = ln2_lo; k = 1; }
            else { hi = x + ln2_hi; lo = -ln2_lo; k = -1; }
        } else {
            k = invln2 * x + (xsb == 0 ? 0.5f : -0.5f);
            t = k;
            hi = x - t * ln2_hi;
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000) {
        t = huge + x;
        return x - (t - (huge + x));
    } else k = 0;
    hfx = 0.5f * x;
    hxs = x * hfx;
    r1 = one + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    t = 3.0f - r1 * hfx;
    e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = (x * (e - c) - c);
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) {
        if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
        return one + 2.0f * (x - e);
    }
    if (k <= -2 || k > 56) {
        y = one - (e - x);
        y = orc_bitsf(orc_fbits(y) + ((uint32_t)k << 23));
        return y - one;
    }
    t = one;
    if (k < 23) {
        t = orc_bitsf(0x3f800000 - (0x1000000 >> k));
        y = t - (e - x);
        y = orc_bitsf(orc_fbits(y) + ((uint32_t)k << 23));
    } else {
        t = orc_bitsf((uint32_t)(0x7f - k) << 23);
        y = x - (e + t);
        y += one;
        y = orc_bitsf(orc_fbits(y) + ((uint32_t)k << 23));
    }
    return y;
}
float orc_tanhf(float x) {
    const float one = 1.0f, two = 2.0f, tiny = 1.0e-30f;
    float t, z;
    int32_t jx = (int32_t)orc_fbits(x), ix = jx & 0x7fffffff;
    if (ix >= 0x7f800000) return jx >= 0 ? one / x + one : one / x - one;
    if (ix < 0x41b00000) {
        if (ix == 0) return x;
        if (ix < 0x24000000) return x * (one + x);
        if (ix >= 0x3f800000) {
            t = orc_expm1f(two * fabsf(x));
            z = one - two / (t + two);
        } else {
            t = orc_expm1f(-two * fabsf(x));
            z = -t / (t + two);
        }
    } else z = one - tiny;
    return jx >= 0 ? z : -z;
}

long long orc_tanhf_mismatches(int threads) {
    long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static) num_threads(threads)
    for (long long i = 0; i < (1LL << 32); i++) {
        const float x = orc_bitsf((uint32_t)i);
        const float a = orc_tanhf(x), b = tanhf(x);
        if (orc_fbits(a) != orc_fbits(b) && !(a != a && b != b)) bad++;
    }
    return bad;
}

/* The tanhf digest of the device self-check: sum over all 2^32 inputs u of
   (u * K1) ^ (bits(tanhf(u)) * K2), NaN results as 0x7FC00000. */
unsigned long long orc_tanhf_digest(int threads) {
    unsigned long long h = 0;
#pragma omp parallel for reduction(+ : h) schedule(static) num_threads(threads)
    for (long long i = 0; i < (1LL << 32); i++) {
        const float t = orc_tanhf(orc_bitsf((uint32_t)i));
        const uint32_t ut = t != t ? 0x7FC00000u : orc_fbits(t);
        h += ((unsigned long long)(uint32_t)i * 0x9E3779B97F4A7C15ull) ^
             ((unsigned long long)ut * 0xC2B2AE3D27D4EB4Full);
    }
    return h;
}

/* sinf and cosf as glibc 2.35 computes them on x86-64 (the FMA ifunc
   variant libm's sinf/cosf resolve to on this host): ARM optimized-routines'
   sincosf method.  |x| < pi/4: an odd (sin) or even (cos) polynomial in
   double; |x| < 120: x - n*pi/2 with n from x * 2/pi scaled by 2^24
   (fnmadd), then the polynomial of the quadrant with its sign; larger |x|:
   a 32 x 96-bit product with 4/pi (192-bit table, 8 new bits per word)
   gives the quadrant and a 2.62 fixed-point remainder.  In the FMA build
   each "a + b * c" of the polynomials and the reduction is one fma.  The
   constants are the published ones (sincosf_data.c); the restatement is
   checked against libm on every float input
   (tests/test_oracle_pins.py::test_sinf_cosf_restatement_equals_libm_on_every_float). */
typedef struct {
    double sign[4], hpi_inv, hpi, c0, c1, c2, c3, c4, s1, s2, s3;
} orc_sincos_t;
static const orc_sincos_t orc_sincos_tab[2] = {
    {{1.0, -1.0, -1.0, 1.0}, 0x1.45F306DC9C883p+23, 0x1.921FB54442D18p0, 0x1p0,
     -0x1.ffffffd0c621cp-2, 0x1.55553e1068f19p-5, -0x1.6c087e89a359dp-10,
     0x1.99343027bf8c3p-16, -0x1.555545995a603p-3, 0x1.1107605230bc4p-7,
     -0x1.994eb3774cf24p-13},
    {{1.0, -1.0, -1.0, 1.0}, 0x1.45F306DC9C883p+23, 0x1.921FB54442D18p0, -0x1p0,
     0x1.ffffffd0c621cp-2, -0x1.55553e1068f19p-5, 0x1.6c087e89a359dp-10,
     -0x1.99343027bf8c3p-16, -0x1.555545995a603p-3, 0x1.1107605230bc4p-7,
     -0x1.994eb3774cf24p-13}};
static const uint32_t orc_inv_pio4[24] = {
    0xa2,       0xa2f9,     0xa2f983,   0xa2f9836e, 0xf9836e4e, 0x836e4e44,
    0x6e4e4415, 0x4e441529, 0x441529fc, 0x1529fc27, 0x29fc2757, 0xfc2757d1,
    0x2757d1f5, 0x57d1f534, 0xd1f534dd, 0xf534ddc0, 0x34ddc0db, 0xddc0db62,
    0xc0db6295, 0xdb629599, 0x6295993c, 0x95993c43, 0x993c4390, 0x3c439041};

static inline uint32_t orc_abstop12(float x) { return (orc_fbits(x) >> 20) & 0x7ff; }

static inline float orc_sincos_poly(double x, double x2, const orc_sincos_t *p, int n) {
    if ((n & 1) == 0) {
        const double x3 = x * x2;
        const double s1 = fma(x2, p->s3, p->s2);
        const double x7 = x3 * x2;
        const double s = fma(x3, p->s1, x);
        return (float)fma(x7, s1, s);
    }
    const double x4 = x2 * x2;
    const double c2 = fma(x2, p->c4, p->c3);
    const double c1 = fma(x2, p->c1, p->c0);
    const double x6 = x4 * x2;
    const double c = fma(x4, p->c2, c1);
    return (float)fma(x6, c2, c);
}

static inline double orc_reduce_fast(double x, const orc_sincos_t *p, int *np) {
    const double r = x * p->hpi_inv;
    const int n = ((int32_t)r + 0x800000) >> 24;
    *np = n;
    return fma(-(double)n, p->hpi, x);
}

static inline double orc_reduce_large(uint32_t xi, int *np) {
    const uint32_t *arr = &orc_inv_pio4[(xi >> 26) & 15];
    const int shift = (xi >> 23) & 7;
    xi = (xi & 0xffffff) | 0x800000;
    xi <<= shift;
    uint64_t res0 = (uint32_t)(xi * arr[0]);
    const uint64_t res1 = (uint64_t)xi * arr[4];
    const uint64_t res2 = (uint64_t)xi * arr[8];
    res0 = (res2 >> 32) | (res0 << 32);
    res0 += res1;
    const uint64_t n = (res0 + (1ULL << 61)) >> 62;
    res0 -= n << 62;
    const double x = (double)(int64_t)res0;
    *np = (int)n;
    return x * 0x1.921FB54442D18p-62;
}

/* cosine = 0: sinf; 1: cosf. */
static float orc_sincosf(float y, int cosine) {
    double x = y;
    int n;
    const orc_sincos_t *p = &orc_sincos_tab[0];
    if (orc_abstop12(y) < orc_abstop12(0x1.921FB6p-1f)) {
        const double x2 = x * x;
        if (orc_abstop12(y) < orc_abstop12(0x1p-12f)) return cosine ? 1.0f : y;
        return orc_sincos_poly(x, x2, p, cosine);
    }
    if (orc_abstop12(y) < orc_abstop12(120.0f)) {
        x = orc_reduce_fast(x, p, &n);
        const double s = p->sign[n & 3];
        if (n & 2) p = &orc_sincos_tab[1];
        return orc_sincos_poly(x * s, x * x, p, n ^ cosine);
    }
    if (orc_abstop12(y) < orc_abstop12(INFINITY)) {
        const uint32_t xi = orc_fbits(y);
        const int sign = xi >> 31;
        x = orc_reduce_large(xi, &n);
        const double s = p->sign[(n + sign) & 3];
        if ((n + sign) & 2) p = &orc_sincos_tab[1];
        return orc_sincos_poly(x * s, x * x, p, n ^ cosine);
    }
    return (y - y) / (y - y);
}

float orc_sinf(float x) { return orc_sincosf(x, 0); }
float orc_cosf(float x) { return orc_sincosf(x, 1); }

/* Inputs whose restated sinf (which = 0) or cosf (1) differs from libm's
   (NaN == NaN), over all 2^32 floats. */
long long orc_sincosf_mismatches(int which, int threads) {
    long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static) num_threads(threads)
    for (long long i = 0; i < (1LL << 32); i++) {
        const float x = orc_bitsf((uint32_t)i);
        const float a = which ? orc_cosf(x) : orc_sinf(x);
        const float b = which ? cosf(x) : sinf(x);
        if (orc_fbits(a) != orc_fbits(b) && !(a != a && b != b)) bad++;
    }
    return bad;
}

/* Digest of the restated sinf (which = 0) or cosf (1) over all 2^32 inputs,
   in the form of orc_tanhf_digest. */
unsigned long long orc_sincosf_digest(int which, int threads) {
    unsigned long long h = 0;
#pragma omp parallel for reduction(+ : h) schedule(static) num_threads(threads)
    for (long long i = 0; i < (1LL << 32); i++) {
        const float x = orc_bitsf((uint32_t)i);
        const float t = which ? orc_cosf(x) : orc_sinf(x);
        const uint32_t ut = t != t ? 0x7FC00000u : orc_fbits(t);
        h += ((unsigned long long)(uint32_t)i * 0x9E3779B97F4A7C15ull) ^
             ((unsigned long long)ut * 0xC2B2AE3D27D4EB4Full);
    }
    return h;
}

/* The snake activations of the decoder (dacvae.c:803-931) on time-major
   [T, C] rows: v = x (+ bias[c] when bias is not NULL), y = v + sin(a v)^2
   / a with sinf = orc_sinf.  inv_form: the hoisted reciprocal
   inv = 1 / (a + 1e-9), y = v + (s * s) * inv (iro_snake_forward up to 1536
   channels, snake_bias_forward in place up to 1536 channels); otherwise the
   quotient y = v + (s * s) / (a + 1e-9).  conv ORC_GCC_FASTMATH contracts the
   reciprocal form's final add into fma(s * s, inv, v); the fast build's
   libmvec sinf is not restated, so that convention is parity unpinned here.
   y may be x. */
void orc_snake(int conv, const float *x, int T, int C, const float *bias, const float *alpha,
               int inv_form, float *y) {
    for (long long t = 0; t < T; t++)
        for (int c = 0; c < C; c++) {
            const size_t i = (size_t)t * C + c;
            const float v = bias ? x[i] + bias[c] : x[i];
            const float a = alpha[c];
            const float s = orc_sinf(a * v);
            const float ss = s * s;
            if (inv_form) {
                const float inv = 1.0f / (a + 1e-9f);
                y[i] = conv == ORC_GCC_FASTMATH ? fmaf(ss, inv, v) : v + ss * inv;
            } else {
                y[i] = v + ss / (a + 1e-9f);
            }
        }
}

/* dit.c:543-558 adaln_branch for branches 0..2 of one adaLN, then the gate's
   tanhf (dit.c:588): act = silu(cond slice) as x / (1 + expf(-x));
   low[r] = sum_d act[d] down[r][d] in index order (+ 0, the scalar linear's
   absent bias); out[n] = (sum_r low[r] up[n][r] in index order) + bias[n],
   then + cond slice[n]; gate = tanhf(out).  cond [B, 3D]; down[i] [R, D],
   up[i] [D, R], bias[i] [D]; out [3, B, D]: shift, scale, gate. */
void orc_adaln_params(const float *cond, int B, int D, int R, const float *const *down,
                      const float *const *up, const float *const *bias, float *out) {
    float *act = malloc(sizeof(float) * (size_t)D);
    float *low = malloc(sizeof(float) * (size_t)R);
    for (int br = 0; br < 3; br++)
        for (int b = 0; b < B; b++) {
            const float *in = cond + (size_t)b * 3 * D + (size_t)br * D;
            for (int d = 0; d < D; d++) act[d] = in[d] / (1.0f + expf(-in[d]));
            for (int r = 0; r < R; r++) {
                float acc = 0.0f;
                for (int d = 0; d < D; d++) {
                    const float p = act[d] * down[br][(size_t)r * D + d];
                    acc = acc + p;
                }
                low[r] = acc + 0.0f;
            }
            float *o = out + ((size_t)br * B + b) * D;
            for (int n = 0; n < D; n++) {
                float acc = 0.0f;
                for (int r = 0; r < R; r++) {
                    const float p = low[r] * up[br][(size_t)n * R + r];
                    acc = acc + p;
                }
                const float y = acc + bias[br][n];
                o[n] = y + in[n];
                if (br == 2) o[n] = orc_tanhf(o[n]);
            }
        }
    free(act);
    free(low);
}

/* ---- per-head RMSNorm and half-RoPE: dit.c:619-706 ---------------------- */

/* The rotation table of head_rmsnorm_rope_pair (dit.c:641-657, 697-703): per
   pair p of a 64-wide head, the angle step 1 / 10000^(2p/64) as a double
   cosine/sine pair from libm, and position s's rotation advanced from
   position s-1 by one complex multiplication in double (each product rounded,
   no fused multiply-add), rounded to float for use.  cos_t/sin_t are
   [S][32]. */
void orc_rope_table(int S, float *cos_t, float *sin_t) {
    double cs[32], sn[32], c[32], s[32];
    for (int p = 0; p < 32; p++) {
        const double theta = 1.0 / pow(10000.0, (double)(2 * p) / 64.0);
        cs[p] = cos(theta);
        sn[p] = sin(theta);
        c[p] = 1.0;
        s[p] = 0.0;
    }
    for (int t = 0; t < S; t++) {
        for (int p = 0; p < 32; p++) {
            cos_t[(size_t)t * 32 + p] = (float)c[p];
            sin_t[(size_t)t * 32 + p] = (float)s[p];
        }
        for (int p = 0; p < 32; p++) {
            const double a = c[p] * cs[p], b = s[p] * sn[p];
            const double e = s[p] * cs[p], f = c[p] * sn[p];
            c[p] = a - b;
            s[p] = e + f;
        }
    }
}

/* One 64-wide head row: mean square in index order, inv = 1/sqrtf(ms/64 +
   eps), then either y = x * (inv * w) or, for a rotated head, the pairs
   (y0, y1) = (x0' c - x1' s, x0' s + x1' c) with x' = x * (inv * w)
   (dit.c:619-636, 666-695). */
static void orc_head_row(float *row, const float *w, float eps, const float *ct, const float *st) {
    float ms = 0.0f;
    for (int d = 0; d < 64; d++) {
        const float sq = row[d] * row[d];
        ms = ms + sq;
    }
    const float inv = 1.0f / sqrtf(ms / 64.0f + eps);
    if (!ct) {
        for (int d = 0; d < 64; d++) row[d] = row[d] * (inv * w[d]);
        return;
    }
    for (int p = 0; p < 32; p++) {
        const float x0 = row[2 * p] * (inv * w[2 * p]);
        const float x1 = row[2 * p + 1] * (inv * w[2 * p + 1]);
        const float a = x0 * ct[p], b = x1 * st[p];
        const float e = x0 * st[p], f = x1 * ct[p];
        row[2 * p] = a - b;
        row[2 * p + 1] = e + f;
    }
}

/* q, k [B*S, heads*64] in place.  rope != 0: head_rmsnorm_rope_pair
   (dit.c:638-706), the first heads/2 heads rotated by position s; rope == 0:
   head_rmsnorm (dit.c:619-636) on q alone (k may be NULL). */
int orc_head_norm_rope(float *q, const float *qw, float *k, const float *kw, int B, int S,
                       int heads, float eps, int rope) {
    float *ct = NULL, *st = NULL;
    if (rope) {
        ct = malloc(sizeof(float) * (size_t)S * 32);
        st = malloc(sizeof(float) * (size_t)S * 32);
        if (!ct || !st) {
            free(ct);
            free(st);
            return -1;
        }
        orc_rope_table(S, ct, st);
    }
    const int D = heads * 64;
    for (int b = 0; b < B; b++)
        for (int s = 0; s < S; s++)
            for (int h = 0; h < heads; h++) {
                const size_t off = ((size_t)b * S + s) * D + (size_t)h * 64;
                const int rot = rope && h < heads / 2;
                const float *c = rot ? ct + (size_t)s * 32 : NULL;
                const float *sn = rot ? st + (size_t)s * 32 : NULL;
                orc_head_row(q + off, qw + h * 64, eps, c, sn);
                if (k) orc_head_row(k + off, kw + h * 64, eps, c, sn);
            }
    free(ct);
    free(st);
    return 0;
}

/* ---- attention core: dit.c:808-870 with the scalar ops (ops.c:577-600,
   681-703, 754-766, 786-789) ---------------------------------------------- */

/* Per batch b and head h: the joined keys are the S latent tokens of b, then
   the context rows ci < C whose mask[b*C + ci] is set, in order (context row
   ci of batch b is row ci of the shared context when context_batch == 1, else
   row b*C + ci).  score = sum_d q[d] k[d] in index order, times 1/sqrtf(64);
   softmax per query row: max by strict replacement from the first score,
   p = expf(score - max), sum of p in key order, p / sum; out[n] = sum_j p_j
   v_j[n] in key order; mix = out * (1 / (1 + expf(-gate))).  q, k, v, gate,
   mix [B*S, D]; ck, cv [(context_batch == 1 ? 1 : B) * C, D]. */
int orc_attention_core(const float *q, const float *k, const float *v, const float *gate, int B,
                       int S, int D, const float *ck, const float *cv, const uint8_t *mask, int C,
                       int context_batch, float *mix, int threads) {
    const int heads = D / 64;
    const float scale = 1.0f / sqrtf(64.0f);
    int fail = 0;
    /* (b, h) pairs are independent; each thread keeps its own key lists. */
#pragma omp parallel num_threads(threads)
    {
        const float **kr = malloc(sizeof(float *) * (size_t)(S + C));
        const float **vr = malloc(sizeof(float *) * (size_t)(S + C));
        float *sc = malloc(sizeof(float) * (size_t)(S + C));
        if (!kr || !vr || !sc) {
#pragma omp atomic write
            fail = 1;
        }
#pragma omp for collapse(2) schedule(dynamic)
        for (int b = 0; b < B; b++) {
            for (int h = 0; h < heads; h++) {
                if (!kr || !vr || !sc) continue;
                int J = 0;
                for (int t = 0; t < S; t++) {
                    kr[J] = k + ((size_t)b * S + t) * D + h * 64;
                    vr[J++] = v + ((size_t)b * S + t) * D + h * 64;
                }
                const size_t crow = context_batch == 1 ? 0 : (size_t)b * C;
                for (int ci = 0; ci < C; ci++) {
                    if (!mask[(size_t)b * C + ci]) continue;
                    kr[J] = ck + (crow + ci) * D + h * 64;
                    vr[J++] = cv + (crow + ci) * D + h * 64;
                }
                for (int s = 0; s < S; s++) {
                    const float *qs = q + ((size_t)b * S + s) * D + h * 64;
                    for (int j = 0; j < J; j++) {
                        float acc = 0.0f;
                        for (int d = 0; d < 64; d++) {
                            const float pr = qs[d] * kr[j][d];
                            acc = acc + pr;
                        }
                        sc[j] = acc * scale;
                    }
                    float mx = sc[0];
                    for (int j = 1; j < J; j++)
                        if (sc[j] > mx) mx = sc[j];
                    float sum = 0.0f;
                    for (int j = 0; j < J; j++) {
                        sc[j] = expf(sc[j] - mx);
                        sum = sum + sc[j];
                    }
                    for (int j = 0; j < J; j++) sc[j] = sc[j] / sum;
                    float *out = mix + ((size_t)b * S + s) * D + h * 64;
                    for (int n = 0; n < 64; n++) {
                        float acc = 0.0f;
                        for (int j = 0; j < J; j++) {
                            const float pr = sc[j] * vr[j][n];
                            acc = acc + pr;
                        }
                        out[n] = acc;
                    }
                }
            }
        }
        free(kr);
        free(vr);
        free(sc);
    }
    if (fail) return -1;
    const size_t n = (size_t)B * S * D;
    for (size_t i = 0; i < n; i++) {
        const float r = 1.0f / (1.0f + expf(-gate[i]));
        mix[i] = mix[i] * r;
    }
    return 0;
}

/* ---- fp32 linear and RMSNorm of the scalar build: ops.c:221-234, 738-747 */

void orc_linear_f32(const float *x, int M, int K, const float *w, int N, const float *bias,
                    float *y) {
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float acc = 0.0f;
            for (int k = 0; k < K; k++) {
                const float p = x[(size_t)m * K + k] * w[(size_t)n * K + k];
                acc = acc + p;
            }
            y[(size_t)m * N + n] = acc + (bias ? bias[n] : 0.0f);
        }
}

void orc_rmsnorm(const float *x, int M, int D, const float *w, float eps, float *y) {
    for (int m = 0; m < M; m++) {
        const float *r = x + (size_t)m * D;
        float ms = 0.0f;
        for (int d = 0; d < D; d++) {
            const float sq = r[d] * r[d];
            ms = ms + sq;
        }
        const float inv = 1.0f / sqrtf(ms / (float)D + eps);
        for (int d = 0; d < D; d++) {
            const float t = r[d] * inv;
            y[(size_t)m * D + d] = t * w[d];
        }
    }
}

/* ---- gated residual: dit.c:1013-1020, 1032-1039 ------------------------ */

void orc_gated_residual(int conv, float *x, const float *gate,
                        const float *branch, int B, int S, int D) {
    for (int b = 0; b < B; b++) {
        const float *grow = gate + (size_t)b * D;
        for (int s = 0; s < S; s++) {
            size_t row = ((size_t)b * S + s) * D;
            for (int i = 0; i < D; i++) {
                if (conv == ORC_GCC_FASTMATH)
                    x[row + i] = fmaf(grow[i], branch[row + i], x[row + i]);
                else
                    x[row + i] = x[row + i] + grow[i] * branch[row + i];
            }
        }
    }
}

/* ---- int8 Conv1d: dacvae.c:340-348, 543-688 ----------------------------- */

int orc_conv1d_output_length(int T, int kernel, int stride, int dilation,
                             int padding) {
    if (T <= 0 || stride <= 0 || kernel <= 0 || dilation <= 0) return -1;
    long long effective = (long long)dilation * (kernel - 1) + 1;
    long long num = (long long)T + 2LL * padding - effective;
    long long out = num < 0 ? -1 : num / stride + 1;
    return out <= 0 || out > 0x7fffffffLL ? -1 : (int)out;
}

/* The quantized im2col rows of the conv (dacvae.c:607-673): per input row
   the range over channels, per output row the window range over the taps
   inside [0, T), then the u8 row [tap*C + c] (padding taps = zero point) and,
   with c2 != NULL, the fixed-scale second plane (dacvae.c:637-663).
   Returns T_out, or -1 on bad shapes or allocation failure. */
int orc_conv1d_quantize(int conv, const float *input, int T, int C, int kernel,
                        int stride, int dilation, int padding, uint8_t *c1,
                        float *s1, int32_t *z1, uint8_t *c2, float *s2,
                        int32_t *z2) {
    const int T_out = orc_conv1d_output_length(T, kernel, stride, dilation, padding);
    if (T_out <= 0 || C <= 0) return -1;
    const int inner = kernel * C;
    const int fast = conv == ORC_GCC_FASTMATH;
    const int residual = c2 != NULL;
    /* Per input row (time step) range over channels, with zero included
       (dacvae.c:607-616). */
    float *row_lo = malloc(sizeof(float) * (size_t)T);
    float *row_hi = malloc(sizeof(float) * (size_t)T);
    if (!row_lo || !row_hi) {
        free(row_lo); free(row_hi);
        return -1;
    }
    for (int t = 0; t < T; t++) row_range(input + (size_t)t * C, C, &row_lo[t], &row_hi[t]);
    for (int r = 0; r < T_out; r++) {
        /* Window range over the taps that land inside [0, T)
           (dacvae.c:617-627); padding taps do not widen it. */
        float lo = 0.0f, hi = 0.0f;
        for (int tap = 0; tap < kernel; tap++) {
            int it = r * stride - padding + tap * dilation;
            if (it < 0 || it >= T) continue;
            lo = row_lo[it] < lo ? row_lo[it] : lo;
            hi = row_hi[it] > hi ? row_hi[it] : hi;
        }
        RowQuant q = row_params(conv, lo, hi);
        float sc2, inv2;
        if (fast) {
            /* dacvae.c:637-638 under fast-math: s/255 -> s*fl(1/255),
               255/s -> 0x477E00FF/(hi-lo) (s=1 rows are all-zero windows
               whose plane-2 codes are 128 regardless of inv2). */
            sc2 = q.s * C_INV255;
            float d = hi - lo;
            inv2 = (hi - lo) * C_INV255 > 0.0f ? C_255_OVER_INV255_B / d : 255.0f;
        } else {
            sc2 = q.s / 255.0f;
            inv2 = 255.0f / q.s;
        }
        s1[r] = q.s;
        z1[r] = q.zp;
        if (residual) {
            s2[r] = sc2;
            z2[r] = 128;
        }
        uint8_t *dst = c1 + (size_t)r * inner;
        uint8_t *dst2 = residual ? c2 + (size_t)r * inner : NULL;
        for (int tap = 0; tap < kernel; tap++) {
            int it = r * stride - padding + tap * dilation;
            uint8_t *td = dst + (size_t)tap * C;
            if (it < 0 || it >= T) {
                memset(td, q.zp, (size_t)C);
                if (residual) memset(dst2 + (size_t)tap * C, 128, (size_t)C);
                continue;
            }
            const float *row = input + (size_t)it * C;
            for (int c = 0; c < C; c++) {
                uint8_t code = quant_code(conv, row[c], &q);
                td[c] = code;
                if (residual) {
                    float v = (float)code;
                    float rem, v2;
                    if (fast) {
                        rem = fmaf(q.s, q.zpf - v, row[c]);
                        v2 = rne(fmaf(rem, inv2, 128.0f));
                    } else {
                        rem = row[c] - q.s * (v - q.zpf);
                        v2 = rne(rem * inv2 + 128.0f);
                    }
                    v2 = v2 < 0.0f ? 0.0f : v2;
                    v2 = v2 > 255.0f ? 255.0f : v2;
                    dst2[(size_t)tap * C + c] = (uint8_t)v2;
                }
            }
        }
    }
    free(row_lo); free(row_hi);
    return T_out;
}

int orc_conv1d_int8(int conv, const float *input, int T, int C,
                    const int8_t *wq, const float *sw, const int32_t *colsum,
                    int N, int kernel, int stride, int dilation, int padding,
                    const float *bias, int residual, float *output,
                    uint8_t *cols, float *row_scale, int32_t *row_zero,
                    int threads) {
    const int T_out = orc_conv1d_output_length(T, kernel, stride, dilation, padding);
    if (T_out <= 0 || C <= 0 || N <= 0) return -1;
    const int inner = kernel * C;
    uint8_t *c1 = cols ? cols : malloc((size_t)T_out * inner);
    uint8_t *c2 = residual ? malloc((size_t)T_out * inner) : NULL;
    float *s1 = malloc(sizeof(float) * (size_t)T_out);
    int32_t *z1 = malloc(sizeof(int32_t) * (size_t)T_out);
    float *s2 = residual ? malloc(sizeof(float) * (size_t)T_out) : NULL;
    int32_t *z2 = residual ? malloc(sizeof(int32_t) * (size_t)T_out) : NULL;
    int32_t *work = malloc(sizeof(int32_t) * (size_t)T_out * N);
    int ok = c1 && s1 && z1 && work && (!residual || (c2 && s2 && z2));
    if (ok)
        ok = orc_conv1d_quantize(conv, input, T, C, kernel, stride, dilation, padding,
                                 c1, s1, z1, c2, s2, z2) == T_out;
    if (ok) {
        orc_int8_linear_ex(conv, c1, s1, z1, wq, sw, colsum, N, inner, bias,
                           output, T_out, work, 0, threads);
        if (residual)
            orc_int8_linear_ex(conv, c2, s2, z2, wq, sw, colsum, N, inner, NULL,
                               output, T_out, work, 1, threads);
        if (row_scale) memcpy(row_scale, s1, sizeof(float) * (size_t)T_out);
        if (row_zero) memcpy(row_zero, z1, sizeof(int32_t) * (size_t)T_out);
    }
    if (!cols) free(c1);
    free(c2); free(s1); free(z1); free(s2); free(z2); free(work);
    return ok ? T_out : -1;
}

/* ---- int8 ConvTranspose1d: dacvae.c:350-358, 696-795 -------------------- */

int orc_convtranspose1d_output_length(int T_in, int kernel, int stride,
                                      int padding, int output_padding) {
    if (T_in <= 0 || stride <= 0 || kernel <= 0) return -1;
    long long out = (long long)(T_in - 1) * stride - 2LL * padding + kernel +
                    output_padding;
    return out <= 0 || out > 0x7fffffffLL ? -1 : (int)out;
}

/* Without snake: every output row starts at the bias; the input rows are
   quantized (two-term with `residual`), one int8 linear gives the expanded
   rows [T_in, kernel*C_out] (plane 2 accumulated by a second linear), and
   the taps are scattered onto the output in ascending input row, tap and
   channel order, each add rounded on its own. */
int orc_convtranspose1d_int8(int conv, const float *input, int T_in, int C_in,
                             const int8_t *wq, const float *sw,
                             const int32_t *colsum, int C_out, int kernel,
                             int stride, int padding, int output_padding,
                             const float *bias, int residual, float *output,
                             int threads) {
    const int T_out = orc_convtranspose1d_output_length(T_in, kernel, stride,
                                                        padding, output_padding);
    if (T_out <= 0 || C_in <= 0 || C_out <= 0) return -1;
    const int N = kernel * C_out;
    for (int t = 0; t < T_out; t++)
        for (int c = 0; c < C_out; c++)
            output[(size_t)t * C_out + c] = bias ? bias[c] : 0.0f;
    uint8_t *q1 = malloc((size_t)T_in * C_in);
    uint8_t *q2 = residual ? malloc((size_t)T_in * C_in) : NULL;
    float *s1 = malloc(sizeof(float) * (size_t)T_in);
    float *s2 = malloc(sizeof(float) * (size_t)T_in);
    int32_t *z1 = malloc(sizeof(int32_t) * (size_t)T_in);
    int32_t *z2 = malloc(sizeof(int32_t) * (size_t)T_in);
    float *rem = residual ? malloc(sizeof(float) * (size_t)T_in * C_in) : NULL;
    float *expanded = malloc(sizeof(float) * (size_t)T_in * N);
    int32_t *work = malloc(sizeof(int32_t) * (size_t)T_in * N);
    int ok = q1 && s1 && s2 && z1 && z2 && expanded && work && (!residual || (q2 && rem));
    if (ok) {
        if (residual) {
            orc_quantize_rows_residual(conv, input, T_in, C_in, q1, s1, z1, rem, q2, s2, z2);
            orc_int8_linear_ex(conv, q1, s1, z1, wq, sw, colsum, N, C_in, NULL, expanded,
                               T_in, work, 0, threads);
            orc_int8_linear_ex(conv, q2, s2, z2, wq, sw, colsum, N, C_in, NULL, expanded,
                               T_in, work, 1, threads);
        } else {
            orc_quantize_rows(conv, input, T_in, C_in, q1, s1, z1);
            orc_int8_linear_ex(conv, q1, s1, z1, wq, sw, colsum, N, C_in, NULL, expanded,
                               T_in, work, 0, threads);
        }
        for (int row = 0; row < T_in; row++) {
            const int base = row * stride - padding;
            const float *src = expanded + (size_t)row * N;
            for (int tap = 0; tap < kernel; tap++) {
                const int t = base + tap;
                if (t < 0 || t >= T_out) continue;
                float *dst = output + (size_t)t * C_out;
                const float *k = src + (size_t)tap * C_out;
                for (int c = 0; c < C_out; c++) dst[c] += k[c];
            }
        }
    }
    free(q1); free(q2); free(s1); free(s2); free(z1); free(z2);
    free(rem); free(expanded); free(work);
    return ok ? T_out : -1;
}

/* ---- int8 1x1 projection onto the skip: dacvae.c:974-1012 --------------- */

/* output = skip, then the reference's two accumulating linears:
   output += lin(q1) + bias; with residual, output += lin(q2). */
int orc_conv1x1_skip_int8(int conv, const float *hidden, const float *skip,
                          int T, const int8_t *wq, const float *sw,
                          const int32_t *colsum, int C_out, int C_in,
                          const float *bias, int residual, float *output,
                          int threads) {
    if (T <= 0 || C_in <= 0 || C_out <= 0) return -1;
    memmove(output, skip, sizeof(float) * (size_t)T * C_out);
    uint8_t *q1 = malloc((size_t)T * C_in);
    uint8_t *q2 = residual ? malloc((size_t)T * C_in) : NULL;
    float *s1 = malloc(sizeof(float) * (size_t)T), *s2 = malloc(sizeof(float) * (size_t)T);
    int32_t *z1 = malloc(sizeof(int32_t) * (size_t)T), *z2 = malloc(sizeof(int32_t) * (size_t)T);
    float *rem = residual ? malloc(sizeof(float) * (size_t)T * C_in) : NULL;
    int32_t *work = malloc(sizeof(int32_t) * (size_t)T * C_out);
    int ok = q1 && s1 && s2 && z1 && z2 && work && (!residual || (q2 && rem));
    if (ok) {
        if (residual) {
            orc_quantize_rows_residual(conv, hidden, T, C_in, q1, s1, z1, rem, q2, s2, z2);
            orc_int8_linear_ex(conv, q1, s1, z1, wq, sw, colsum, C_out, C_in, bias, output,
                               T, work, 1, threads);
            orc_int8_linear_ex(conv, q2, s2, z2, wq, sw, colsum, C_out, C_in, NULL, output,
                               T, work, 1, threads);
        } else {
            orc_quantize_rows(conv, hidden, T, C_in, q1, s1, z1);
            orc_int8_linear_ex(conv, q1, s1, z1, wq, sw, colsum, C_out, C_in, bias, output,
                               T, work, 1, threads);
        }
    }
    free(q1); free(q2); free(s1); free(s2); free(z1); free(z2); free(rem); free(work);
    return ok ? 0 : -1;
}

/* sampler.c:281-297 (see iro_oracle.h). */
void orc_euler_update(int conv, float *state, const float *velocity, size_t n, int use_cfg,
                      int text_row, int speaker_row, int caption_row, float scale_text,
                      float scale_speaker, float scale_caption, float dt) {
    const int rows[3] = {text_row, speaker_row, caption_row};
    const float scales[3] = {scale_text, scale_speaker, scale_caption};
    int act_row[3];
    float act_scale[3];
    int terms = 0;
    for (int k = 0; k < 3; k++)
        if (use_cfg && rows[k] >= 0) {
            act_row[terms] = rows[k];
            act_scale[terms] = scales[k];
            terms++;
        }
    for (size_t i = 0; i < n; i++) {
        const float v = velocity[i];
        float d[3];
        for (int k = 0; k < terms; k++) d[k] = v - velocity[(size_t)act_row[k] * n + i];
        if (conv != ORC_GCC_FASTMATH) {
            float guided = v;
            for (int k = 0; k < terms; k++) guided += act_scale[k] * d[k];
            state[i] += guided * dt;
            continue;
        }
        float guided = v;
        if (terms == 1)
            guided = fmaf(act_scale[0], d[0], v);
        else if (terms == 2)
            guided = v + fmaf(act_scale[1], d[1], act_scale[0] * d[0]);
        else if (terms == 3)
            guided = fmaf(act_scale[2], d[2], v) + fmaf(act_scale[1], d[1], act_scale[0] * d[0]);
        state[i] = fmaf(guided, dt, state[i]);
    }
}
