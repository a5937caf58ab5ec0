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
static char backend_desc[256] = "oracle-openmp";

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
            int branch = -1;
            if (cs) (void)cs(MKL_CBWR_AVX512_E1);
            if (cg) branch = cg(MKL_CBWR_BRANCH);
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
                             "oracle-openmp (oneMKL refused: selfcheck failed, cbwr %d)", branch);
                } else {
                    snprintf(backend_desc, sizeof backend_desc,
                             "oneMKL cblas_gemm_s8u8s32 (cbwr branch %d)", branch);
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

/* Raw GEMM only (for the int32 cross-check against the oracle). */
void cpub_gemm(const uint8_t *a, const int8_t *b, int32_t *c, int M, int N, int K) {
    gemm(a, b, c, M, N, K);
}
