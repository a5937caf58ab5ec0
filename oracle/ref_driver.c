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
