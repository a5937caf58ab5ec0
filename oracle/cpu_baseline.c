/* cpu_baseline.c -- the reference's oneMKL int8 CPU path, re-expressed as a
 * timing harness for bench.py's cpu_baseline leg.  TEST/BENCH
 * INFRASTRUCTURE ONLY: never part of the HIP product path.
 *
 * What it times is what ops.c does in its oneMKL release build:
 *   quantize   ops.c:321-348, one thread, as the reference's serial loop;
 *   GEMM       ops.c:458-461 cblas_gemm_s8u8s32(RowMajor, NoTrans, Trans,
 *              FixOffset, alpha=1, ao=0, bo=0, beta=0, co=0) on MKL threads;
 *   epilogue   ops.c:468-490, one thread.
 * oneMKL is opened at run time (dlopen of libmkl_rt) with the CBWR branch
 * forced to AVX512_E1 as ops.c:400-425 does, and refused unless the
 * int16-saturation known answer (ops.c:375-398) sums exactly.  Without
 * oneMKL the GEMM falls back to the oracle's OpenMP loop (reported as such).
 */
#define _GNU_SOURCE
#include <dlfcn.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "iro_oracle.h"

typedef void (*gemm_s8u8s32_fn)(int layout, int transa, int transb, int offsetc,
                                int m, int n, int k, float alpha, const void *a,
                                int lda, signed char ao, const void *b, int ldb,
                                signed char bo, float beta, int32_t *c, int ldc,
                                const int32_t *co);
typedef int (*cbwr_set_fn)(int);
typedef int (*cbwr_get_fn)(int);
typedef int (*cbwr_auto_fn)(void);
typedef void (*set_threads_fn)(int);

enum {
    CBLAS_ROW_MAJOR = 101, CBLAS_NO_TRANS = 111, CBLAS_TRANS = 112,
    CBLAS_FIX_OFFSET = 173,
    MKL_CBWR_BRANCH = 1, MKL_CBWR_AVX512_E1 = 14, MKL_CBWR_SUCCESS = 0,
};

static void *mkl_handle;
static gemm_s8u8s32_fn mkl_gemm;
static set_threads_fn mkl_set_threads;
static int n_threads = 1;
static char backend_desc[320] = "oracle-openmp";

/* MKL_CBWR_* branch codes (mkl_cbwr.h) by name. */
static const char *cbwr_name(int code) {
    switch (code) {
        case 0: return "OFF";
        case 1: return "BRANCH_OFF";
        case 2: return "AUTO";
        case 3: return "COMPATIBLE";
        case 4: return "SSE2";
        case 6: return "SSSE3";
        case 7: return "SSE4_1";
        case 8: return "SSE4_2";
        case 9: return "AVX";
        case 10: return "AVX2";
        case 11: return "AVX512_MIC";
        case 12: return "AVX512";
        case 13: return "AVX512_MIC_E1";
        case 14: return "AVX512_E1";
        default: return code < 0 ? "unavailable" : "unknown";
    }
}

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

static void gemm(const uint8_t *a, const int8_t *b, int32_t *c, int M, int N, int K) {
    if (mkl_gemm) {
        const int32_t co = 0;
        mkl_gemm(CBLAS_ROW_MAJOR, CBLAS_NO_TRANS, CBLAS_TRANS, CBLAS_FIX_OFFSET,
                 M, N, K, 1.0f, a, K, 0, b, K, 0, 0.0f, c, N, &co);
    } else {
        orc_gemm_u8s8(a, b, c, M, N, K, n_threads);
    }
}

/* Returns 1 when oneMKL is in use, 0 for the OpenMP fallback.  desc gets a
   one-line description of the backend actually in effect. */
int cpub_init(const char *mkl_path, int threads, char *desc, size_t desc_len) {
    n_threads = threads > 0 ? threads : 1;
    if (!mkl_handle) {
        /* One OpenMP runtime per process: let MKL thread on libgomp. */
        setenv("MKL_THREADING_LAYER", "GNU", 0);
        if (!getenv("MKL_CBWR")) setenv("MKL_CBWR", "AVX512_E1", 0);
        const char *cands[] = {mkl_path, "libmkl_rt.so.3", "libmkl_rt.so.2",
                               "libmkl_rt.so.1", "/opt/conda/lib/libmkl_rt.so.1",
                               "/opt/conda/lib/libmkl_rt.so"};
        for (size_t i = 0; i < sizeof(cands) / sizeof(cands[0]) && !mkl_handle; i++)
            if (cands[i] && *cands[i]) mkl_handle = dlopen(cands[i], RTLD_NOW | RTLD_LOCAL);
        if (mkl_handle) {
            gemm_s8u8s32_fn g = (gemm_s8u8s32_fn)dlsym(mkl_handle, "cblas_gemm_s8u8s32");
            cbwr_set_fn cs = (cbwr_set_fn)dlsym(mkl_handle, "MKL_CBWR_Set");
            cbwr_get_fn cg = (cbwr_get_fn)dlsym(mkl_handle, "MKL_CBWR_Get");
            mkl_set_threads = (set_threads_fn)dlsym(mkl_handle, "MKL_Set_Num_Threads");
            cbwr_auto_fn ca = (cbwr_auto_fn)dlsym(mkl_handle, "MKL_CBWR_Get_Auto_Branch");
            int branch = -1, set_rc = -100, auto_branch = -1;
            if (cs) set_rc = cs(MKL_CBWR_AVX512_E1);
            if (cg) branch = cg(MKL_CBWR_BRANCH);
            if (ca) auto_branch = ca();
            if (g) {
                mkl_gemm = g;
                if (mkl_set_threads) mkl_set_threads(n_threads);
                uint8_t a[3 * 64];
                int8_t b[5 * 64];
                int32_t want[15], got[15];
                orc_selfcheck_kat(a, b, want);
                gemm(a, b, got, 3, 5, 64);
                if (memcmp(want, got, sizeof(got)) != 0) {
                    mkl_gemm = NULL; /* int16-saturating branch: refuse */
                    snprintf(backend_desc, sizeof backend_desc,
                             "oracle-openmp (oneMKL refused: selfcheck failed; CBWR setting %s)",
                             cbwr_name(branch));
                } else {
                    snprintf(backend_desc, sizeof backend_desc,
                             "oneMKL cblas_gemm_s8u8s32; CBWR AVX512_E1 requested "
                             "(MKL_CBWR_Set rc %d), setting in effect %s, AUTO would pick %s",
                             set_rc, cbwr_name(branch), cbwr_name(auto_branch));
                }
            }
        }
    }
    if (mkl_set_threads) mkl_set_threads(n_threads);
    if (desc && desc_len) snprintf(desc, desc_len, "%s", backend_desc);
    return mkl_gemm != NULL;
}

/* One reference int8 linear (ops.c:321-348 + 450-491) on host memory.
   x [M,K] fp32 -> y [M,N]; q/sx/zx/work are caller scratch.  Adds the
   seconds spent in each part to t[0] quantize, t[1] GEMM, t[2] epilogue. */
void cpub_linear(int conv, const float *x, int M, int K, const int8_t *wq,
                 const float *sw, const int32_t *colsum, int N,
                 const float *bias, float *y, uint8_t *q, float *sx,
                 int32_t *zx, int32_t *work, int accumulate, double *t) {
    double t0 = now_s();
    orc_quantize_rows(conv, x, M, K, q, sx, zx);
    double t1 = now_s();
    gemm(q, wq, work, M, N, K);
    double t2 = now_s();
    orc_epilogue(conv, work, sx, zx, sw, colsum, bias, y, M, N, accumulate);
    double t3 = now_s();
    t[0] += t1 - t0;
    t[1] += t2 - t1;
    t[2] += t3 - t2;
}

typedef struct {
    const int8_t *q;
    const float *s;
    const int32_t *cs;
    int N, K;
} CpubWeight;

/* One int8 projection of an activation already quantized (one or two
   planes), as int8_scratch_linear (dit.c:477-485): y = lin(q1); y += lin(q2). */
static void cpub_project(int conv, const uint8_t *q1, const float *s1, const int32_t *z1,
                         const uint8_t *q2, const float *s2, const int32_t *z2,
                         const CpubWeight *w, float *y, int M, int32_t *work, double *t) {
    double t0 = now_s();
    gemm(q1, w->q, work, M, w->N, w->K);
    double t1 = now_s();
    orc_epilogue(conv, work, s1, z1, w->s, w->cs, NULL, y, M, w->N, 0);
    double t2 = now_s();
    t[1] += t1 - t0;
    t[2] += t2 - t1;
    if (q2) {
        t0 = now_s();
        gemm(q2, w->q, work, M, w->N, w->K);
        t1 = now_s();
        orc_epilogue(conv, work, s2, z2, w->s, w->cs, NULL, y, M, w->N, 1);
        t2 = now_s();
        t[1] += t1 - t0;
        t[2] += t2 - t1;
    }
}

static void cpub_quantize(int conv, const float *x, int M, int K, int two, uint8_t *q1,
                          float *s1, int32_t *z1, float *r, uint8_t *q2, float *s2, int32_t *z2,
                          double *t) {
    double t0 = now_s();
    if (two)
        orc_quantize_rows_residual(conv, x, M, K, q1, s1, z1, r, q2, s2, z2);
    else
        orc_quantize_rows(conv, x, M, K, q1, s1, z1);
    t[0] += now_s() - t0;
}

/* One DiT block's int8 linears on host memory, in the order and with the
   activation sharing of dit.c: the modulation linear on cond, QKVG on one
   quantization of x (dit.c:780-798), Wo on V with x += gate_a * out
   (dit.c:876-884, 1013-1020), W1/W3 on one quantization of x, the SwiGLU
   gate (ops.c:781-784), W2 on the (two-term) hidden state with
   x += gate_m * out (dit.c:939-972, 1032-1039).  gate_a = mod[:, 2D:3D],
   gate_m = mod[:, 5D:6D].  w = {ada, wq, wk, wv, wgate, wo, w1, w3, w2}.
   residual_mask: 1 QKVG, 2 Wo, 4 W1/W3, 8 W2 (dit.c:278-291).  Adds
   quantize / GEMM / epilogue-and-elementwise seconds to t[0..2].
   Returns 0, or -1 when out of memory. */
int cpub_dit_block(int conv, const CpubWeight *w, float *x, const float *cond, int B, int S,
                   int D, int H, int residual_mask, double *t) {
    const size_t M = (size_t)B * S;
    const size_t KM = (size_t)(H > D ? H : D);
    const size_t NM = (size_t)(6 * D > H ? 6 * D : H);
    uint8_t *q1 = malloc(M * KM), *q2 = malloc(M * KM);
    float *s1 = malloc(4 * M), *s2 = malloc(4 * M), *r = malloc(4 * M * KM);
    int32_t *z1 = malloc(4 * M), *z2 = malloc(4 * M), *work = malloc(4 * M * NM);
    float *mod = malloc(4 * (size_t)B * 6 * D), *gate = malloc(4 * (size_t)B * D);
    float *qkvg = malloc(4 * 4 * M * D), *branch = malloc(4 * M * D);
    float *a = malloc(4 * M * H), *b = malloc(4 * M * H);
    int ok = q1 && q2 && s1 && s2 && r && z1 && z2 && work && mod && gate && qkvg && branch &&
             a && b;
    if (ok) {
        /* modulation rows */
        cpub_quantize(conv, cond, B, D, 0, q1, s1, z1, r, q2, s2, z2, t);
        cpub_project(conv, q1, s1, z1, NULL, NULL, NULL, &w[0], mod, B, work, t);
        /* QKVG */
        int two = (residual_mask & 1) != 0;
        cpub_quantize(conv, x, (int)M, D, two, q1, s1, z1, r, q2, s2, z2, t);
        for (int i = 0; i < 4; i++)
            cpub_project(conv, q1, s1, z1, two ? q2 : NULL, s2, z2, &w[1 + i], qkvg + i * M * D,
                         (int)M, work, t);
        /* Wo on V, attention gated residual */
        two = (residual_mask & 2) != 0;
        cpub_quantize(conv, qkvg + 2 * M * D, (int)M, D, two, q1, s1, z1, r, q2, s2, z2, t);
        cpub_project(conv, q1, s1, z1, two ? q2 : NULL, s2, z2, &w[5], branch, (int)M, work, t);
        double t0 = now_s();
        for (int bb = 0; bb < B; bb++)
            memcpy(gate + (size_t)bb * D, mod + (size_t)bb * 6 * D + 2 * D, 4 * (size_t)D);
        orc_gated_residual(conv, x, gate, branch, B, S, D);
        t[2] += now_s() - t0;
        /* SwiGLU */
        two = (residual_mask & 4) != 0;
        cpub_quantize(conv, x, (int)M, D, two, q1, s1, z1, r, q2, s2, z2, t);
        cpub_project(conv, q1, s1, z1, two ? q2 : NULL, s2, z2, &w[6], a, (int)M, work, t);
        cpub_project(conv, q1, s1, z1, two ? q2 : NULL, s2, z2, &w[7], b, (int)M, work, t);
        t0 = now_s();
        orc_silu_mul(a, b, M * H);
        t[2] += now_s() - t0;
        two = (residual_mask & 8) != 0;
        cpub_quantize(conv, a, (int)M, H, two, q1, s1, z1, r, q2, s2, z2, t);
        cpub_project(conv, q1, s1, z1, two ? q2 : NULL, s2, z2, &w[8], branch, (int)M, work, t);
        t0 = now_s();
        for (int bb = 0; bb < B; bb++)
            memcpy(gate + (size_t)bb * D, mod + (size_t)bb * 6 * D + 5 * D, 4 * (size_t)D);
        orc_gated_residual(conv, x, gate, branch, B, S, D);
        t[2] += now_s() - t0;
    }
    free(q1); free(q2); free(s1); free(s2); free(r); free(z1); free(z2); free(work);
    free(mod); free(gate); free(qkvg); free(branch); free(a); free(b);
    return ok ? 0 : -1;
}

/* Raw GEMM only (for the int32 cross-check against the oracle). */
void cpub_gemm(const uint8_t *a, const int8_t *b, int32_t *c, int M, int N, int K) {
    gemm(a, b, c, M, N, K);
}

/* The reference's int8 Conv1d (dacvae.c:543-688) on the host: the quantized
   im2col rows on one thread (the reference's serial loop), the GEMM on MKL
   threads (ops.c:458-461), the epilogue with bias on one thread
   (ops.c:468-490), and, with residual, the second plane accumulated.
   Returns T_out or -1; t[0..2] as cpub_linear. */
int cpub_conv1d(int conv, const float *x, int T, int C, const int8_t *wq, const float *sw,
                const int32_t *colsum, int N, int kernel, int stride, int dilation,
                int padding, const float *bias, int residual, float *y, double *t) {
    const int T_out = orc_conv1d_output_length(T, kernel, stride, dilation, padding);
    if (T_out <= 0) return -1;
    const size_t inner = (size_t)kernel * C;
    uint8_t *c1 = malloc((size_t)T_out * inner);
    uint8_t *c2 = residual ? malloc((size_t)T_out * inner) : NULL;
    float *s1 = malloc(sizeof(float) * T_out), *s2 = malloc(sizeof(float) * T_out);
    int32_t *z1 = malloc(sizeof(int32_t) * T_out), *z2 = malloc(sizeof(int32_t) * T_out);
    int32_t *work = malloc(sizeof(int32_t) * (size_t)T_out * N);
    int ok = c1 && s1 && s2 && z1 && z2 && work && (!residual || c2);
    if (ok) {
        double t0 = now_s();
        ok = orc_conv1d_quantize(conv, x, T, C, kernel, stride, dilation, padding, c1, s1, z1,
                                 c2, s2, z2) == T_out;
        double t1 = now_s();
        t[0] += t1 - t0;
        for (int plane = 0; ok && plane < (residual ? 2 : 1); plane++) {
            double a = now_s();
            gemm(plane ? c2 : c1, wq, work, T_out, N, (int)inner);
            double b = now_s();
            orc_epilogue(conv, work, plane ? s2 : s1, plane ? z2 : z1, sw, colsum,
                         plane ? NULL : bias, y, T_out, N, plane);
            double c = now_s();
            t[1] += b - a;
            t[2] += c - b;
        }
    }
    free(c1); free(c2); free(s1); free(s2); free(z1); free(z2); free(work);
    return ok ? T_out : -1;
}
