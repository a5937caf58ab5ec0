/* ref_driver.c -- exposes the reference's file-static int8 convolution to
 * the oracle's pin tests.  Compiled only by oracle/Makefile's `ref` target,
 * from the reference sources where they lie; the output goes to oracle/_ref/
 * (never committed).  TEST INFRASTRUCTURE ONLY.
 *
 * The wrapper builds the two structs conv1d_int8_forward expects
 * (dacvae.h:11-20 IroConv1d, ops.h:23-28 IroInt8Weight) and calls it without
 * snake, exactly as dacvae.c:1221-1233 does for the initial convolution. */
#include "dacvae.c"

int ref_conv1d_int8(const float *input, int T, int C, int N, int kernel,
                    int stride, int dilation, int padding, int8_t *wq,
                    float *sw, int32_t *colsum, const float *bias,
                    int residual, float *output) {
    IroConv1d conv = {0};
    conv.in_channels = C;
    conv.out_channels = N;
    conv.kernel = kernel;
    conv.stride = stride;
    conv.dilation = dilation;
    conv.padding = padding;
    IroInt8Weight w = {0};
    w.data = wq;
    w.scale = sw;
    w.colsum = colsum;
    w.N = N;
    w.K = kernel * C;
    return conv1d_int8_forward(&conv, &w, input, T, output, bias, NULL,
                               residual, NULL, NULL, NULL);
}

/* The int8 ConvTranspose1d without snake (dacvae.c:696-795); its two-term
   choice follows the reference's own policy (dacvae.c:27-73: off for the
   upsample group unless IRO_CODEC_INT8_RESIDUAL says otherwise). */
int ref_convtranspose1d_int8(const float *input, int T_in, int C_in, int C_out,
                             int kernel, int stride, int padding,
                             int output_padding, int8_t *wq, float *sw,
                             int32_t *colsum, const float *bias,
                             float *output) {
    IroConvTranspose1d conv = {0};
    conv.bias = bias;
    conv.in_channels = C_in;
    conv.out_channels = C_out;
    conv.kernel = kernel;
    conv.stride = stride;
    conv.padding = padding;
    conv.output_padding = output_padding;
    IroInt8Weight w = {0};
    w.data = wq;
    w.scale = sw;
    w.colsum = colsum;
    w.N = kernel * C_out;
    w.K = C_in;
    return convtranspose1d_forward_impl(&conv, &w, input, T_in, output, NULL,
                                        NULL, 0);
}

/* The adaLN of a DiT block (dit.c:561-617, iro_dit_adaln) with its low-rank
   linears zeroed: each branch then outputs its bias plus its slice of cond
   (dit.c:543-558), so shift = fl(shift_bias + cond[:, 0:D]) and scale =
   fl(scale_bias + cond[:, D:2D]) exactly, and h is the reference's RMSNorm
   modulate (dit.c:593-606) on those rows.  x and h are [B*S, D], cond is
   [B, 3D], D = the reference's model dimension. */
#include "dit.h"
int ref_dit_adaln_zero_rank(float eps, const float *x, const float *cond,
                            const float *shift_bias, const float *scale_bias,
                            const float *gate_bias, int B, int S, float *h, float *gate,
                            int *dim) {
    const size_t n = (size_t)IRO_DIT_MODEL_DIM * 192;
    float *z = calloc(n, sizeof(float));
    if (!z) return -1;
    IroAdaLN a = {z, z, shift_bias, z, z, scale_bias, z, z, gate_bias};
    const int rc = iro_dit_adaln(&a, eps, x, cond, B, S, h, gate);
    free(z);
    *dim = IRO_DIT_MODEL_DIM;
    return rc;
}
