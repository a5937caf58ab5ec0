/* ref_sampler_driver.c -- runs the reference's own Euler sampler
 * (sampler.c, public entry iro_sample_euler_conditions) on a random-weight
 * DiT and records what its trace callback sees, so the CFG combine and
 * Euler update of sampler.c:281-297 can be pinned step by step: the trace of
 * step s gives x_t (row 0 is the state entering step s) and the velocity
 * rows; the state entering step s+1 is row 0 of the next trace, and the last
 * state is the sampler's output.  Every weight array of the DiT aliases one
 * caller-filled pool (each weight reads a prefix of it), so no checkpoint
 * and no stand-in code is needed.  Compiled only by oracle/Makefile's `ref`
 * target from the reference sources where they lie; outputs stay in
 * oracle/_ref/.  TEST INFRASTRUCTURE ONLY. */
#include <stdlib.h>
#include <string.h>

#include "sampler.h"

enum { REF_LATENT_DIM = 32, REF_MAX_BATCH = 4 };

typedef struct {
    int max_steps, n;
    float *x_t, *vel, *timestep;
    int *batch;
} RefTrace;

static int ref_trace(void *user, int step, float timestep, int batch, const float *x_t,
                     const float *velocity) {
    RefTrace *r = user;
    if (step < 0 || step >= r->max_steps || batch < 1 || batch > REF_MAX_BATCH) return 1;
    const size_t row = (size_t)REF_MAX_BATCH * r->n;
    memcpy(r->x_t + (size_t)step * row, x_t, sizeof(float) * (size_t)batch * r->n);
    memcpy(r->vel + (size_t)step * row, velocity, sizeof(float) * (size_t)batch * r->n);
    r->batch[step] = batch;
    r->timestep[step] = timestep;
    return 0;
}

/* cfg: steps, init_scale, cfg_scale_text, cfg_scale_speaker,
   cfg_scale_caption, cfg_min_t, cfg_max_t (sampler.h IroEulerConfig).
   x_t and vel hold [steps][4][S*32], batch and timestep [steps].
   pool must hold at least 3 * 1280 * 1280 floats (the largest weight,
   cond_module.4 [COND_DIM, MODEL_DIM]). */
int ref_sample_euler(const float *pool, float eps, const float *text, const uint8_t *text_mask,
                     int text_tokens, const float *speaker, int speaker_tokens,
                     const float *caption, int caption_tokens, const float *noise, int S,
                     const float *cfg, float *output, float *x_t, float *vel, int *batch,
                     float *timestep) {
    IroDiT *d = calloc(1, sizeof(IroDiT));
    if (!d) return -1;
    d->cond_w0 = d->cond_w1 = d->cond_w2 = pool;
    d->in_w = d->in_b = d->out_norm = d->out_w = d->out_b = pool;
    for (int l = 0; l < IRO_DIT_LAYERS; l++) {
        IroAdaLN a = {pool, pool, pool, pool, pool, pool, pool, pool, pool};
        d->attention_adaln[l] = a;
        d->mlp_adaln[l] = a;
        IroJointAttention j = {pool, pool, pool, pool, pool, pool, pool,
                               pool, pool, pool, pool, pool, pool};
        d->attention[l] = j;
        IroSwiGLU m = {pool, pool, pool};
        d->mlp[l] = m;
    }
    d->norm_eps = eps;
    IroEulerConfig c = {(int)cfg[0], cfg[1], cfg[2], cfg[3], cfg[4], cfg[5], cfg[6]};
    RefTrace r = {c.steps, S * REF_LATENT_DIM, x_t, vel, timestep, batch};
    const int rc = iro_sample_euler_conditions(d, text, text_mask, text_tokens, speaker,
                                               speaker_tokens, caption, caption_tokens, noise, S,
                                               &c, output, ref_trace, &r, NULL);
    free(d);
    return rc;
}
