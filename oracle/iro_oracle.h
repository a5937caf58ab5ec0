/* iro_oracle.h -- CPU restatement of irodori-c's int8 W8A8 path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: the HIP product
 * path never links, loads or calls it.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may use it.
 *
 * Two rounding conventions are restated, because the reference's results
 * depend on how it was compiled (Makefile:4-7):
 *   ORC_STRICT        ops.c built with -O2 (the default `make irodori`,
 *                     `make test-int8-ops`): every float op rounds
 *                     separately, divisions are true divisions.
 *   ORC_GCC_FASTMATH  ops.c/dit.c/dacvae.c built with FAST_CFLAGS
 *                     (-O3 -march=native -ffast-math, the oneMKL release
 *                     build): GCC 11 folds the divisions by 255/127 into
 *                     reciprocal constants and contracts mul+add into FMA.
 * Integer results (codes, int32 sums) are convention-independent only
 * through the scales that produce them.
 */
#ifndef IRO_ORACLE_H
#define IRO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_STRICT = 0, ORC_GCC_FASTMATH = 1 };

/* ops.c:259-293 (iro_int8_weight_quantize). q [N,K] s8, scale[N], colsum[N]. */
int orc_weight_quantize(int conv, const float *w, int N, int K,
                        int8_t *q, float *scale, int32_t *colsum);
/* ops.c:295-306: source stored [K,N]; result as orc_weight_quantize. */
int orc_weight_quantize_transposed(int conv, const float *w, int N, int K,
                                   int8_t *q, float *scale, int32_t *colsum);

/* ops.c:321-348 (iro_int8_quantize_rows). */
void orc_quantize_rows(int conv, const float *x, int M, int K,
                       uint8_t *q, float *scale, int32_t *zero);

/* ops.c:427-442 (iro_int8_quantize_rows_residual). residual may be NULL. */
void orc_quantize_rows_residual(int conv, const float *x, int M, int K,
                                uint8_t *q1, float *scale1, int32_t *zero1,
                                float *residual,
                                uint8_t *q2, float *scale2, int32_t *zero2);

/* ops.c:351-364 (int8_gemm_reference): exact c = a[M,K]u8 . b[N,K]s8^T.
   threads > 1 splits rows across OpenMP threads (integer, order-free). */
void orc_gemm_u8s8(const uint8_t *a, const int8_t *b, int32_t *c,
                   int M, int N, int K, int threads);

/* ops.c:468-490: the four epilogue branches on a precomputed accumulator. */
void orc_epilogue(int conv, const int32_t *acc, const float *sx,
                  const int32_t *zx, const float *sw, const int32_t *colsum,
                  const float *bias, float *y, int M, int N, int accumulate);

/* ops.c:450-491 (iro_int8_linear_ex): gemm then epilogue. work [M,N]. */
void orc_int8_linear_ex(int conv, const uint8_t *q, const float *sx,
                        const int32_t *zx, const int8_t *wq, const float *sw,
                        const int32_t *colsum, int N, int K,
                        const float *bias, float *y, int M, int32_t *work,
                        int accumulate, int threads);

/* ops.c:375-398 (iro_int8_selfcheck): fills the known-answer arrays
   a[3*64], b[5*64] and the exact sums want[3*5]. */
void orc_selfcheck_kat(uint8_t *a, int8_t *b, int32_t *want);

/* ops.c:781-784 (iro_silu_mul_inplace), strict build: x = x/(1+expf(-x))*g
   with glibc's scalar expf. The fast-math build vectorises this with libmvec
   expf and an rcpps Newton step, whose results depend on the host CPU; it
   has no portable restatement. */
void orc_silu_mul(float *x, const float *g, size_t n);

/* glibc's expf restated (the function orc_silu_mul calls through libm):
   glibc >= 2.28 sysdeps/ieee754/flt-32/e_expf.c, the exp2f table method of
   ARM optimized-routines (N = 32 table, cubic in r), as GCC builds glibc's
   x86-64 __expf_fma variant (both uses of InvLn2N*x contracted to FMA). */
float orc_expf_restated(float x);
/* Count the float inputs (all 2^32 bit patterns) where orc_expf_restated
   and this process's libm expf differ (NaN == NaN). */
long long orc_expf_mismatches(int threads);
/* Sum over every float x (mod 2^64) of (bits(x) * 0x9E3779B97F4A7C15) ^
   (bits(orc_expf_restated(x)) * 0xC2B2AE3D27D4EB4F), NaN results counted as
   0x7FC00000: the digest a device restatement must reproduce. */
unsigned long long orc_expf_digest(int threads);
/* dit.c:593-606 (strict build): the adaLN RMSNorm modulate of x [B*S, D]
   with branch rows shift/scale [B, D]; the sum of squares runs in index
   order, as the strict build accumulates it. */
/* Digests of the host's sqrtf and 1.0f / x over every float input, in the
   form of orc_expf_digest. */
void orc_fp32_digests(int threads, unsigned long long *sqrt_digest,
                      unsigned long long *recip_digest);
void orc_adaln_apply(const float *x, const float *shift, const float *scale, int B, int S, int D,
                     float eps, float *h);
void orc_linear_f32(const float *x, int M, int K, const float *w, int N, const float *bias,
                    float *y);
void orc_rmsnorm(const float *x, int M, int D, const float *w, float eps, float *y);
float orc_expm1f(float x);
float orc_tanhf(float x);
long long orc_tanhf_mismatches(int threads);
float orc_sinf(float x);
float orc_cosf(float x);
long long orc_sincosf_mismatches(int which, int threads);
unsigned long long orc_sincosf_digest(int which, int threads);
void orc_snake(int conv, const float *x, int T, int C, const float *bias, const float *alpha,
               int inv_form, float *y);
unsigned long long orc_tanhf_digest(int threads);
void orc_adaln_params(const float *cond, int B, int D, int R, const float *const *down,
                      const float *const *up, const float *const *bias, float *out);
void orc_rope_table(int S, float *cos_t, float *sin_t);
int orc_head_norm_rope(float *q, const float *qw, float *k, const float *kw, int B, int S,
                       int heads, float eps, int rope);
int orc_attention_core(const float *q, const float *k, const float *v, const float *gate, int B,
                       int S, int D, const float *ck, const float *cv, const uint8_t *mask, int C,
                       int context_batch, float *mix, int threads);

/* dit.c:1013-1020 / 1032-1039: x[b,s,:] += gate[b,:] * branch[b,s,:].
   Strict: two roundings.  Fast-math: one FMA (vfmadd132ps). */
void orc_gated_residual(int conv, float *x, const float *gate,
                        const float *branch, int B, int S, int D);

/* dacvae.c:543-688 (conv1d_int8_forward) without snake: input [T, C]
   time-major, weight [N, kernel*C] (tap-major K).  cols (nullable) receives
   the u8 im2col [T_out, kernel*C]; scale/zero (nullable) the per-output-row
   quantization.  residual adds the fixed-scale second plane
   (s/255, zero point 128).  Returns T_out, or -1 on bad shape. */
int orc_conv1d_int8(int conv, const float *input, int T, int C,
                    const int8_t *wq, const float *sw, const int32_t *colsum,
                    int N, int kernel, int stride, int dilation, int padding,
                    const float *bias, int residual, float *output,
                    uint8_t *cols, float *row_scale, int32_t *row_zero,
                    int threads);

/* The quantized im2col rows of the conv alone (dacvae.c:607-673): c1 (and,
   with c2 != NULL, the second plane) [T_out, kernel*C], per-row s, zp. */
int orc_conv1d_quantize(int conv, const float *input, int T, int C, int kernel,
                        int stride, int dilation, int padding, uint8_t *c1,
                        float *s1, int32_t *z1, uint8_t *c2, float *s2,
                        int32_t *z2);

/* dacvae.c:350-358 (iro_convtranspose1d_output_length). */
int orc_convtranspose1d_output_length(int T_in, int kernel, int stride,
                                      int padding, int output_padding);

/* dacvae.c:696-795 (convtranspose1d_forward_impl) with an int8 weight and
   no snake: input [T_in, C_in], weight codes [kernel*C_out, C_in] (the
   transposed quantization of the [C_in, kernel, C_out] export layout),
   output [T_out, C_out].  Returns T_out, or -1. */
int orc_convtranspose1d_int8(int conv, const float *input, int T_in, int C_in,
                             const int8_t *wq, const float *sw,
                             const int32_t *colsum, int C_out, int kernel,
                             int stride, int padding, int output_padding,
                             const float *bias, int residual, float *output,
                             int threads);

/* dacvae.c:974-1012 (the int8 1x1 projection of run_residual_int8):
   output = skip + lin(q1) + bias (+ lin(q2) with residual), hidden [T, C_in]
   quantized per row, weight codes [C_out, C_in]; output may equal skip. */
int orc_conv1x1_skip_int8(int conv, const float *hidden, const float *skip,
                          int T, const int8_t *wq, const float *sw,
                          const int32_t *colsum, int C_out, int C_in,
                          const float *bias, int residual, float *output,
                          int threads);

/* sampler.c:281-297: the CFG combine and Euler update of one sampler step.
   velocity holds the step's CFG rows of n values each (row 0 conditional);
   text_row / speaker_row / caption_row are the unconditional rows (-1 when
   that branch has no CFG row) and apply only when use_cfg.  Strict: every
   op rounds in source order.  Fast: the CFG terms p_k = s_k * (v - v_k)
   (active terms in text, speaker, caption order) are combined as GCC 11
   reassociates them under -ffast-math (pinned against the fast build's
   traces): 1 term fma(s0, d0, v); 2 terms v + fma(s1, d1, p0); 3 terms
   fma(s2, d2, v) + fma(s1, d1, p0); then state = fma(guided, dt, state). */
void orc_euler_update(int conv, float *state, const float *velocity, size_t n, int use_cfg,
                      int text_row, int speaker_row, int caption_row, float scale_text,
                      float scale_speaker, float scale_caption, float dt);

/* dacvae.c:340-348 (iro_conv1d_output_length). */
int orc_conv1d_output_length(int T, int kernel, int stride, int dilation,
                             int padding);

#ifdef __cplusplus
}
#endif

#endif
