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
