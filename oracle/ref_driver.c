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

/* The snake activations (dacvae.c:830-931): iro_snake_forward is public,
   snake_bias_forward file-static. */
void ref_snake(const float *input, float *output, int T, int C, const float *alpha) {
    iro_snake_forward(input, output, T, C, alpha);
}

void ref_snake_bias(const float *input, float *output, int T, int C, const float *bias,
                    const float *alpha) {
    snake_bias_forward(input, output, T, C, bias, alpha);
}

/* run_residual_int8 (dacvae.c:934-1018) on one residual unit built from fp32
   export-layout weights (conv0 [C, 7, C], conv1 [C, 1, C]), quantized as
   iro_dacvae_int8_quantize does (dacvae.c:247-255).  `stage` is the decoder
   stage the unit belongs to: with the default policy (dacvae.c:51-69) the
   second activation plane runs only in stage 3. */
int ref_dacvae_residual_int8(const float *input, int T, int C, const float *alpha0,
                             const float *w0, const float *b0, const float *alpha1,
                             const float *w1, const float *b1, int dilation, int stage,
                             float *output) {
    IroDACVAEResidual unit;
    memset(&unit, 0, sizeof(unit));
    unit.alpha0 = alpha0;
    unit.alpha1 = alpha1;
    IroConv1d c0 = {w0, b0, C, C, 7, 1, dilation, 3 * dilation};
    IroConv1d c1 = {w1, b1, C, C, 1, 1, 1, 0};
    unit.conv0 = c0;
    unit.conv1 = c1;
    IroDACVAEInt8Residual q;
    memset(&q, 0, sizeof(q));
    if (iro_int8_weight_quantize(&q.conv0, w0, C, 7 * C) != 0 ||
        iro_int8_weight_quantize(&q.conv1, w1, C, C) != 0) {
        iro_int8_weight_free(&q.conv0);
        iro_int8_weight_free(&q.conv1);
        return -1;
    }
    float *out = run_residual_int8(&unit, &q, input, T, C, NULL, stage, 0);
    iro_int8_weight_free(&q.conv0);
    iro_int8_weight_free(&q.conv1);
    if (!out) return -1;
    memcpy(output, out, sizeof(float) * (size_t)T * C);
    free(out);
    return 0;
}

/* iro_dacvae_decode (dacvae.c:1213-1300) with the int8 weights of
   iro_dacvae_int8_quantize, its trace observer keeping the quantizer_out
   state [frames, 1024] and the state after decoder stage 3 [T, 96].
   params holds 91 device-free host pointers in this order:
   quantizer_out weight [1024, 1, 32], bias; initial weight [1536, 7, 1024],
   bias; per stage: alpha, upsample weight [c_in, 2 rate, c_out], bias, then
   per residual unit alpha0, conv0 weight, bias, alpha1, conv1 weight, bias;
   final alpha [96], final weight [1, 7, 96], bias [1]. */
typedef struct {
    float *state, *core;
    int state_frames, core_frames;
} RefDecodeTrace;

static int ref_decode_observe(void *user, const char *name, const float *data, int frames,
                              int channels) {
    RefDecodeTrace *t = user;
    if (!strcmp(name, "codec_quantizer_out") && t->state) {
        memcpy(t->state, data, sizeof(float) * (size_t)frames * channels);
        t->state_frames = frames;
    } else if (!strcmp(name, "codec_decoder_stage3") && t->core) {
        memcpy(t->core, data, sizeof(float) * (size_t)frames * channels);
        t->core_frames = frames;
    }
    return 0;
}

int ref_dacvae_decode_trace(const float *const *params, const float *latent, int latent_frames,
                            float *state, float *core, float *waveform) {
    IroDACVAEDecoder dec;
    memset(&dec, 0, sizeof(dec));
    int i = 0;
    IroConv1d qo = {params[i], params[i + 1], CODEBOOK_DIM, LATENT_DIM, 1, 1, 1, 0};
    i += 2;
    IroConv1d ini = {params[i], params[i + 1], LATENT_DIM, DECODER_DIM, 7, 1, 1, 3};
    i += 2;
    dec.quantizer_out = qo;
    dec.initial = ini;
    const int cin[IRO_DACVAE_STAGES] = {1536, 768, 384, 192};
    const int cout[IRO_DACVAE_STAGES] = {768, 384, 192, 96};
    const int rates[IRO_DACVAE_STAGES] = {12, 10, 8, 2};
    const int dil[IRO_DACVAE_RESIDUALS] = {1, 3, 9};
    for (int s = 0; s < IRO_DACVAE_STAGES; s++) {
        IroDACVAEStage *st = &dec.stage[s];
        st->alpha = params[i++];
        IroConvTranspose1d up = {params[i], params[i + 1], cin[s], cout[s], 2 * rates[s],
                                 rates[s], (rates[s] + 1) / 2, rates[s] & 1};
        i += 2;
        st->upsample = up;
        for (int r = 0; r < IRO_DACVAE_RESIDUALS; r++) {
            IroDACVAEResidual *u = &st->residual[r];
            u->alpha0 = params[i++];
            IroConv1d c0 = {params[i], params[i + 1], cout[s], cout[s], 7, 1, dil[r], 3 * dil[r]};
            i += 2;
            u->alpha1 = params[i++];
            IroConv1d c1 = {params[i], params[i + 1], cout[s], cout[s], 1, 1, 1, 0};
            i += 2;
            u->conv0 = c0;
            u->conv1 = c1;
        }
    }
    dec.final_alpha = params[i++];
    IroConv1d fin = {params[i], params[i + 1], FINAL_CHANNELS, 1, 7, 1, 1, 3};
    dec.final = fin;
    IroDACVAEInt8 q;
    if (iro_dacvae_int8_quantize(&q, &dec) != 0) return -1;
    dec.int8 = &q;
    RefDecodeTrace t = {state, core, 0, 0};
    const int rc = iro_dacvae_decode(&dec, latent, latent_frames, waveform, ref_decode_observe, &t);
    iro_dacvae_int8_free(&q);
    return rc ? rc : t.core_frames;
}
