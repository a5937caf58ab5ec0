/* iro_int8_ops.h -- drop-in for the int8 W8A8 section of the reference's
 * ops.h (ops.h:18-78), served by the MI355X library.
 *
 * Same names, signatures, struct layout, ownership and semantics as the
 * reference, so dit.c/dacvae.c/generate.c and tests/test_int8_ops.c link
 * unchanged once ops.c's int8 section (ops.c:257-491) is left out of the
 * build.  Inputs and outputs stay host memory: each call stages them through
 * a process-wide default context (device 0, convention from the environment
 * variable IRO_HIP_CONVENTION = "strict" (default) or "fastmath").  This
 * layer exists for compatibility and testing; resident activations use the
 * device API in iro_hip.h.
 *
 * Compute calls return void like the reference's; a HIP failure is kept in
 * a sticky flag readable with iro_int8_last_error().
 */
#ifndef IRO_INT8_OPS_H
#define IRO_INT8_OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ops.h:23-28 */
typedef struct {
    int8_t *data;    /* [N,K] row-major */
    float *scale;    /* [N] dequantization scale */
    int32_t *colsum; /* [N] sum over K of data[n][k], for zero-point removal */
    int N, K;
} IroInt8Weight;

/* ops.h:30 (ops.c:259-293).  Quantizes on the GPU; the host arrays are
   malloc'ed and filled as the reference does, and a pre-packed device copy
   is kept until iro_int8_weight_free. */
int iro_int8_weight_quantize(IroInt8Weight *dst, const float *w, int N, int K);
/* ops.h:33-34 (ops.c:295-306) */
int iro_int8_weight_quantize_transposed(IroInt8Weight *dst, const float *w, int N, int K);
/* ops.h:35 (ops.c:308-314): NULL-safe, zeroes the struct, drops the device copy. */
void iro_int8_weight_free(IroInt8Weight *w);
/* ops.h:36 (ops.c:316-319) */
size_t iro_int8_weight_bytes(const IroInt8Weight *w);

/* ops.h:39-40 (ops.c:321-348) */
void iro_int8_quantize_rows(const float *x, int M, int K, uint8_t *q, float *scale,
                            int32_t *zero);

/* ops.h:45-51 (ops.c:444-491).  work must hold M*N int32 and receives the
   raw u8 x s8 sums, as with cblas_gemm_s8u8s32. */
void iro_int8_linear(const uint8_t *q, const float *scale, const int32_t *zero,
                     const IroInt8Weight *w, const float *bias, float *y, int M,
                     int32_t *work);
void iro_int8_linear_ex(const uint8_t *q, const float *scale, const int32_t *zero,
                        const IroInt8Weight *w, const float *bias, float *y, int M,
                        int32_t *work, int accumulate);

/* ops.h:57-61 (ops.c:427-442) */
void iro_int8_quantize_rows_residual(const float *x, int M, int K, uint8_t *q1,
                                     float *scale1, int32_t *zero1, float *residual,
                                     uint8_t *q2, float *scale2, int32_t *zero2);

/* ops.h:65 (ops.c:367-373): 1, the GEMM runs on MFMA. */
int iro_int8_fast_available(void);
/* ops.h:74 (ops.c:400-425): names the GPU backend ("gfx950 MFMA i8 ..."),
   or NULL when no device is usable. */
const char *iro_int8_prepare_backend(void);
/* ops.h:78 (ops.c:375-398): 0 when the MFMA GEMM sums the known answer
   exactly, -1 otherwise (engines must then refuse int8). */
int iro_int8_selfcheck(void);

/* Not in the reference: the sticky error of the drop-in layer (0 none). */
int iro_int8_last_error(void);

#ifdef __cplusplus
}
#endif

#endif
