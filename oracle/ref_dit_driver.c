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
