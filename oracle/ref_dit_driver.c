/* ref_dit_driver.c -- exposes the reference's file-static DiT helpers to the
 * oracle's pin tests.  Compiled only by oracle/Makefile's `ref` target in
 * place of dit.c itself (it includes dit.c, so every public symbol of dit.c
 * comes with it), from the reference sources where they lie; the output goes
 * to oracle/_ref/ (never committed).  TEST INFRASTRUCTURE ONLY. */
#include "dit.c"

/* dit.c:638-706 head_rmsnorm_rope_pair on q, k [B*S, MODEL_DIM] in place. */
void ref_head_rmsnorm_rope_pair(float *q, const float *q_weight, float *k, const float *k_weight,
                                int B, int S, float eps, int *dim, int *heads) {
    head_rmsnorm_rope_pair(q, q_weight, k, k_weight, B, S, eps);
    *dim = MODEL_DIM;
    *heads = IRO_DIT_HEADS;
}

/* dit.c:619-636 head_rmsnorm on x [B*S, MODEL_DIM] in place. */
void ref_head_rmsnorm(float *x, const float *weight, int B, int S, float eps) {
    head_rmsnorm(x, weight, B, S, eps);
}

/* iro_dit_attention (dit.c:895-901, context per batch) or
   iro_dit_attention_shared_context (dit.c:903-911) with every projection the
   identity matrix: the scalar linear then copies its input exactly, so
   q = k = v = gate = x before the head norms, and the output is the
   attention core of dit.c:808-870 on (norm-rope(x), norm-rope(x), x, gate x). */
int ref_dit_attention_identity(const float *x, const float *q_norm, const float *k_norm,
                               const float *ck, const float *cv, const uint8_t *mask, int B,
                               int S, int C, int shared, float eps, float *out) {
    const size_t n = (size_t)MODEL_DIM * MODEL_DIM;
    float *eye = calloc(n, sizeof(float));
    if (!eye) return -1;
    for (int i = 0; i < MODEL_DIM; i++) eye[(size_t)i * MODEL_DIM + i] = 1.0f;
    IroJointAttention a = {0};
    a.wq = a.wk = a.wv = a.wo = a.gate = eye;
    a.q_norm = q_norm;
    a.k_norm = k_norm;
    const int rc = shared ? iro_dit_attention_shared_context(&a, eps, x, ck, cv, mask, B, S, C, out)
                          : iro_dit_attention(&a, eps, x, ck, cv, mask, B, S, C, out);
    free(eye);
    return rc;
}

/* Layer 0 of a DiT with the given adaLN weights (ada: 18 arrays, the
   attention then the MLP IroAdaLN in dit.h:11-23 order) and attention / MLP
   weights, quantized to int8 as iro_dit_int8_quantize does (dit.c:235-259)
   into q8 when use_int8 != 0. */
static int setup_layer0(IroDiT *d, IroDiTInt8 *q8, const float *const *ada, const float *wq,
                        const float *wk, const float *wv, const float *wgate, const float *wo,
                        const float *q_norm, const float *k_norm, const float *w1,
                        const float *w3, const float *w2, float eps, int use_int8) {
    IroAdaLN att = {ada[0], ada[1], ada[2], ada[3], ada[4], ada[5], ada[6], ada[7], ada[8]};
    IroAdaLN mlp = {ada[9], ada[10], ada[11], ada[12], ada[13], ada[14], ada[15], ada[16],
                    ada[17]};
    d->attention_adaln[0] = att;
    d->mlp_adaln[0] = mlp;
    IroJointAttention a = {0};
    a.wq = wq;
    a.wk = wk;
    a.wv = wv;
    a.wo = wo;
    a.gate = wgate;
    a.q_norm = q_norm;
    a.k_norm = k_norm;
    d->attention[0] = a;
    IroSwiGLU m = {w1, w2, w3};
    d->mlp[0] = m;
    d->norm_eps = eps;
    if (use_int8) {
        IroDiTInt8Layer *l = &q8->layer[0];
        if (iro_int8_weight_quantize(&l->wq, wq, MODEL_DIM, MODEL_DIM) ||
            iro_int8_weight_quantize(&l->wk, wk, MODEL_DIM, MODEL_DIM) ||
            iro_int8_weight_quantize(&l->wv, wv, MODEL_DIM, MODEL_DIM) ||
            iro_int8_weight_quantize(&l->gate, wgate, MODEL_DIM, MODEL_DIM) ||
            iro_int8_weight_quantize(&l->wo, wo, MODEL_DIM, MODEL_DIM) ||
            iro_int8_weight_quantize(&l->w1, w1, MLP_DIM, MODEL_DIM) ||
            iro_int8_weight_quantize(&l->w3, w3, MLP_DIM, MODEL_DIM) ||
            iro_int8_weight_quantize(&l->w2, w2, MODEL_DIM, MLP_DIM))
            return -1;
        d->int8 = q8;
    }
    return 0;
}

/* iro_dit_block (dit.c:1042-1047) of layer 0 set up as setup_layer0 does.
   x [B*S, MODEL_DIM] is updated in place. */
int ref_dit_block(float *x, const float *cond, const float *const *ada, const float *wq,
                  const float *wk, const float *wv, const float *wgate, const float *wo,
                  const float *q_norm, const float *k_norm, const float *w1, const float *w3,
                  const float *w2, const float *ck, const float *cv, const uint8_t *mask, int B,
                  int S, int C, float eps, int use_int8, int *dims) {
    IroDiT *d = calloc(1, sizeof(IroDiT));
    IroDiTInt8 *q8 = calloc(1, sizeof(IroDiTInt8));
    int rc = -1;
    if (!d || !q8) goto out;
    if (setup_layer0(d, q8, ada, wq, wk, wv, wgate, wo, q_norm, k_norm, w1, w3, w2, eps,
                     use_int8))
        goto out;
    rc = iro_dit_block(d, 0, x, cond, ck, cv, mask, B, S, C);
    dims[0] = MODEL_DIM;
    dims[1] = MLP_DIM;
    dims[2] = ADALN_RANK;
out:
    if (q8) iro_dit_int8_free(q8);
    free(q8);
    free(d);
    return rc;
}

/* The two operands of the attention half's gated residual inside
   iro_dit_block (dit.c:1004-1020), computed by the functions dit_block
   itself calls, on the same layer: dit_adaln of the attention adaLN (its
   gate [B, MODEL_DIM]) and dit_attention with the per-batch context
   (branch [B*S, MODEL_DIM]).  x is not modified. */
int ref_dit_attn_parts(const float *x, const float *cond, const float *const *ada,
                       const float *wq, const float *wk, const float *wv, const float *wgate,
                       const float *wo, const float *q_norm, const float *k_norm,
                       const float *w1, const float *w3, const float *w2, const float *ck,
                       const float *cv, const uint8_t *mask, int B, int S, int C, float eps,
                       int use_int8, float *gate, float *branch) {
    IroDiT *d = calloc(1, sizeof(IroDiT));
    IroDiTInt8 *q8 = calloc(1, sizeof(IroDiTInt8));
    float *h = malloc(sizeof(float) * (size_t)B * S * MODEL_DIM);
    int rc = -1;
    if (!d || !q8 || !h) goto out;
    if (setup_layer0(d, q8, ada, wq, wk, wv, wgate, wo, q_norm, k_norm, w1, w3, w2, eps,
                     use_int8))
        goto out;
    if (dit_adaln(&d->attention_adaln[0], eps, x, cond, B, S, h, gate, 0)) goto out;
    rc = dit_attention(&d->attention[0], eps, h, ck, cv, mask, B, B, S, C, branch, 0,
                       d->int8 ? &d->int8->layer[0] : NULL);
out:
    if (q8) iro_dit_int8_free(q8);
    free(q8);
    free(d);
    free(h);
    return rc;
}

/* iro_dit_adaln (dit.c:614-617) with the given low-rank weights: w holds
   shift_down, shift_up, shift_bias, scale_down, scale_up, scale_bias,
   gate_down, gate_up, gate_bias (dit.h:11-23 order).  h [B*S, MODEL_DIM],
   gate [B, MODEL_DIM]. */
int ref_dit_adaln_full(float eps, const float *x, const float *cond, const float *const *w,
                       int B, int S, float *h, float *gate) {
    IroAdaLN a = {w[0], w[1], w[2], w[3], w[4], w[5], w[6], w[7], w[8]};
    return iro_dit_adaln(&a, eps, x, cond, B, S, h, gate);
}

/* The DiT evaluation of one sampler step (sampler.c:259-278) over `layers`
   layers with the shared context: iro_dit_input on one latent row set
   x [S, LATENT_DIM] (dit.c:532-540), broadcast to B rows, then
   iro_dit_block_shared_context per layer (dit.c:1063-1068), then
   iro_dit_output (dit.c:1070-1089) into velocity [B*S, LATENT_DIM].  head:
   in_w, in_b, out_norm, out_w, out_b; per layer l: ada[18 l ...] (attention
   then MLP IroAdaLN arrays) and blk[10 l ...] (wq, wk, wv, wgate, wo,
   q_norm, k_norm, w1, w3, w2), int8-quantized as iro_dit_int8_quantize does. */
int ref_dit_step(const float *x, const float *cond, const float *const *head,
                 const float *const *ada, const float *const *blk, int layers, const float *ck,
                 const float *cv, const uint8_t *mask, int B, int S, int C, float eps,
                 float *velocity) {
    if (layers < 1 || layers > IRO_DIT_LAYERS) return -1;
    IroDiT *d = calloc(1, sizeof(IroDiT));
    IroDiTInt8 *q8 = calloc(1, sizeof(IroDiTInt8));
    float *proj = malloc(sizeof(float) * (size_t)B * S * MODEL_DIM);
    int rc = -1;
    if (!d || !q8 || !proj) goto out;
    d->in_w = head[0];
    d->in_b = head[1];
    d->out_norm = head[2];
    d->out_w = head[3];
    d->out_b = head[4];
    d->norm_eps = eps;
    for (int l = 0; l < layers; l++) {
        const float *const *a = ada + 18 * l;
        const float *const *w = blk + 10 * l;
        IroAdaLN att = {a[0], a[1], a[2], a[3], a[4], a[5], a[6], a[7], a[8]};
        IroAdaLN mlp = {a[9], a[10], a[11], a[12], a[13], a[14], a[15], a[16], a[17]};
        d->attention_adaln[l] = att;
        d->mlp_adaln[l] = mlp;
        IroJointAttention at = {0};
        at.wq = w[0];
        at.wk = w[1];
        at.wv = w[2];
        at.gate = w[3];
        at.wo = w[4];
        at.q_norm = w[5];
        at.k_norm = w[6];
        d->attention[l] = at;
        IroSwiGLU m = {w[7], w[9], w[8]};
        d->mlp[l] = m;
        IroDiTInt8Layer *q = &q8->layer[l];
        if (iro_int8_weight_quantize(&q->wq, w[0], MODEL_DIM, MODEL_DIM) ||
            iro_int8_weight_quantize(&q->wk, w[1], MODEL_DIM, MODEL_DIM) ||
            iro_int8_weight_quantize(&q->wv, w[2], MODEL_DIM, MODEL_DIM) ||
            iro_int8_weight_quantize(&q->gate, w[3], MODEL_DIM, MODEL_DIM) ||
            iro_int8_weight_quantize(&q->wo, w[4], MODEL_DIM, MODEL_DIM) ||
            iro_int8_weight_quantize(&q->w1, w[7], MLP_DIM, MODEL_DIM) ||
            iro_int8_weight_quantize(&q->w3, w[8], MLP_DIM, MODEL_DIM) ||
            iro_int8_weight_quantize(&q->w2, w[9], MODEL_DIM, MLP_DIM))
            goto out;
    }
    d->int8 = q8;
    if (iro_dit_input(d, x, 1, S, proj)) goto out;
    for (int b = 1; b < B; b++)
        memcpy(proj + (size_t)b * S * MODEL_DIM, proj, sizeof(float) * (size_t)S * MODEL_DIM);
    for (int l = 0; l < layers; l++)
        if (iro_dit_block_shared_context(d, l, proj, cond, ck, cv, mask, B, S, C)) goto out;
    rc = iro_dit_output(d, proj, B, S, velocity);
out:
    if (q8) iro_dit_int8_free(q8);
    free(q8);
    free(d);
    free(proj);
    return rc;
}

/* iro_dit_text_kv / iro_dit_speaker_kv (dit.c:708-726): kind 0 = text
   (TEXT_DIM inputs), 1 = speaker (SPEAKER_DIM). */
int ref_dit_context_kv(int kind, const float *in, const float *wk, const float *wv,
                       const float *k_norm, int B, int T, float eps, float *k, float *v,
                       int *in_dim) {
    IroJointAttention a = {0};
    a.k_norm = k_norm;
    if (kind == 0) {
        a.wk_text = wk;
        a.wv_text = wv;
        *in_dim = TEXT_DIM;
        return iro_dit_text_kv(&a, eps, in, B, T, k, v);
    }
    a.wk_speaker = wk;
    a.wv_speaker = wv;
    *in_dim = SPEAKER_DIM;
    return iro_dit_speaker_kv(&a, eps, in, B, T, k, v);
}

/* iro_dit_condition (dit.c:501-530) with only the conditioner weights set:
   w0 [MODEL_DIM, TIMESTEP_DIM], w1 [MODEL_DIM, MODEL_DIM], w2 [COND_DIM,
   MODEL_DIM]; cond [B, COND_DIM].  dims: TIMESTEP_DIM, MODEL_DIM, COND_DIM. */
int ref_dit_condition(const float *w0, const float *w1, const float *w2, const float *t, int B,
                      float *cond, int *dims) {
    IroDiT *d = calloc(1, sizeof(IroDiT));
    if (!d) return -1;
    d->cond_w0 = w0;
    d->cond_w1 = w1;
    d->cond_w2 = w2;
    const int rc = iro_dit_condition(d, t, B, cond);
    free(d);
    dims[0] = TIMESTEP_DIM;
    dims[1] = MODEL_DIM;
    dims[2] = COND_DIM;
    return rc;
}
