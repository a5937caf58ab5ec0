/* iro_hip.h -- C ABI of the MI355X (gfx950) int8 W8A8 path of irodori-c.
 *
 * Two layers, both plain C (pointers and sizes, no HIP or torch types):
 *
 *  1. The device API (`iro_hip_*`).  Every pointer argument marked "device"
 *     is HIP device memory; work is queued on the context's stream and the
 *     call returns once it is queued (call iro_hip_sync to wait).  Calls
 *     return 0 on success and -1 on error; the error text is sticky in the
 *     context (iro_hip_error) until iro_hip_clear_error.
 *
 *  2. The ops.h drop-in (`iro_int8_*`, declared in iro_int8_ops.h): the
 *     reference's host-pointer int8 API with identical names, signatures and
 *     semantics, routed through a process-wide default context.
 *
 * Rounding follows one of the reference's two builds, chosen per context:
 *   IRO_HIP_STRICT        ops.c compiled with -O2 (Makefile:4, the default
 *                         `make irodori` / `make test-int8-ops` build);
 *   IRO_HIP_GCC_FASTMATH  ops.c/dit.c/dacvae.c compiled with FAST_CFLAGS
 *                         (Makefile:7, the oneMKL release build).
 * int8 codes, scales, zero points and int32 sums are bit-exact against the
 * chosen build; fp32 outputs too, except the SwiGLU gate's expf (see
 * iro_hip_dit_swiglu).
 *
 * Contexts are not re-entrant: calls on one context must be serialized,
 * as the reference engine's contract requires (generate.h:49-51).
 */
#ifndef IRO_HIP_H
#define IRO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { IRO_HIP_STRICT = 0, IRO_HIP_GCC_FASTMATH = 1 };

typedef struct IroHipContext IroHipContext;
typedef struct IroHipWeight IroHipWeight;

/* ---- context, stream, memory ------------------------------------------ */

/* Create a context on `device` with its own HIP stream.  Runs the int32
   known-answer test (ops.c:375-398) through the MFMA GEMM and fails if it
   does not sum exactly, as iro_engine_init refuses an inexact backend
   (generate.c:527-536). */
int iro_hip_create(int device, int convention, IroHipContext **out);
void iro_hip_destroy(IroHipContext *ctx);
int iro_hip_get_convention(const IroHipContext *ctx);
const char *iro_hip_error(const IroHipContext *ctx);
void iro_hip_clear_error(IroHipContext *ctx);
int iro_hip_sync(IroHipContext *ctx);
/* The context's hipStream_t, for callers that share it. */
void *iro_hip_stream(IroHipContext *ctx);
/* GEMM tile shape of the context's M > 32 launches: 32*ti rows by 128*tj
   columns (ti in {1,2,4}, tj in {1,2}; ti = 1 implies tj = 2); ti = tj = 0 restores the per-GEMM
   choice.  Negative ti selects another schedule knob with value tj:
   -1 tile order (-1 per GEMM, 0 column slabs first, 1 row tiles first),
   -2 weight ring depth of the whole-tile kernel (0 default, 4, 8),
   -3 column slabs per whole-tile block (0 chosen per GEMM, else 1..64),
   -4 the LDS-pipelined kernel of signed-code GEMMs (0 shape chosen per GEMM,
      -1 off, 1 192x256, 2 96x128, 3 128x256, 4 96x256, 5 64x128 rows x
      columns per workgroup; shapes a GEMM cannot take fall back),
   -5 rows per whole-tile block (0 chosen per GEMM, 64, 128),
   -6 kernel-7 convolution codes (2, the default: the GEMM codes the input
      rows itself from their ranges where that is measured faster -- 64..256
      channels in multiples of 32, 384 on inputs of 16384 rows or more, up
      to 1024 on inputs of 65536 rows or more -- else as 1; 3 the same wherever the kernel takes the shape; 1
      window ranges and im2col codes in one pass; 0 two passes),
   -7 SwiGLU hidden state (0, the default: stored in fp32 and quantized by
      a row quantization launch; 1: the W1/W3 kernel quantizes it for W2
      itself, its blocks exchanging row ranges through device memory, when
      the GEMM's grid fits the GPU at once and the caller does not ask for
      the fp32 hidden state -- measured slower at the DiT shapes),
   -8 output channels per block of the kernel-7 GEMM that codes its rows
      (0 chosen per conv, 128, 256).
   Tuning knobs only: results are identical for every setting.  No
   counterpart in the reference (oneMKL picks its own blocking). */
int iro_hip_set_gemm_tile(IroHipContext *ctx, int ti, int tj);

int iro_hip_alloc(IroHipContext *ctx, size_t bytes, void **dptr);
int iro_hip_free(IroHipContext *ctx, void *dptr);
/* Synchronous copies between host and device memory. */
int iro_hip_upload(IroHipContext *ctx, void *dst_device, const void *src_host, size_t bytes);
int iro_hip_download(IroHipContext *ctx, void *dst_host, const void *src_device, size_t bytes);
/* Byte fill with a kernel on the context stream (capture-safe). */
int iro_hip_fill(IroHipContext *ctx, void *dst_device, int value, size_t bytes);
/* Device-to-device copy queued on the context stream. */
int iro_hip_copy(IroHipContext *ctx, void *dst_device, const void *src_device, size_t bytes);

/* Stream-ordered timing on the context stream. */
int iro_hip_event_create(void **event);
void iro_hip_event_destroy(void *event);
int iro_hip_event_record(IroHipContext *ctx, void *event);
int iro_hip_event_elapsed_ms(void *start, void *stop, float *ms);

/* ---- weights: ops.h:23-28 IroInt8Weight, device resident -------------- */

/* Quantize an fp32 [N,K] row-major device matrix per output row exactly as
   iro_int8_weight_quantize (ops.c:259-293) and pre-pack it once into the
   MFMA fragment layout the GEMM streams (32 rows x 32 k per 1 KiB tile). */
int iro_hip_weight_create(IroHipContext *ctx, const float *w_device, int N, int K,
                          IroHipWeight **out);
/* Same for a [K,N] row-major source (ops.c:295-306, ConvTranspose). */
int iro_hip_weight_create_transposed(IroHipContext *ctx, const float *w_device,
                                     int N, int K, IroHipWeight **out);
/* Fused projection: `parts` fp32 [N_i,K] device matrices quantized row by
   row as above and packed into one weight.  layout 0 concatenates them
   (QKVG: [Wq;Wk;Wv;Wgate], dit.c:786-792 run as one GEMM); layout 1
   interleaves two equal parts in 32-row blocks so each output tile holds
   matching W1 and W3 columns (dit.c:944-956, SwiGLU).  Quantization is per
   row, so codes, scales and sums are identical to separate weights. */
int iro_hip_weight_create_fused(IroHipContext *ctx, const float *const *parts_device,
                                const int *parts_N, int nparts, int K, int layout,
                                IroHipWeight **out);
/* Adopt an already quantized host weight (codes [N,K], scale[N], colsum[N]). */
int iro_hip_weight_from_host(IroHipContext *ctx, const int8_t *data, const float *scale,
                             const int32_t *colsum, int N, int K, IroHipWeight **out);
/* Copy a weight back to host arrays in its logical row order. */
int iro_hip_weight_export(IroHipContext *ctx, const IroHipWeight *w, int8_t *data,
                          float *scale, int32_t *colsum);
void iro_hip_weight_destroy(IroHipWeight *w);
/* Logical N (all parts) and K. */
int iro_hip_weight_dims(const IroHipWeight *w, int *N, int *K);
/* Same accounting as iro_int8_weight_bytes (ops.c:316-319). */
size_t iro_hip_weight_bytes(const IroHipWeight *w);

/* ---- activations ------------------------------------------------------ */

/* iro_int8_quantize_rows (ops.c:321-348) on device memory.  x [M,K] fp32,
   q [M,K] u8, scale[M], zero[M]. */
int iro_hip_quantize_rows(IroHipContext *ctx, const float *x, int M, int K, uint8_t *q,
                          float *scale, int32_t *zero);
/* iro_int8_quantize_rows_residual (ops.c:427-442); residual may be NULL. */
int iro_hip_quantize_rows_residual(IroHipContext *ctx, const float *x, int M, int K,
                                   uint8_t *q1, float *scale1, int32_t *zero1,
                                   float *residual, uint8_t *q2, float *scale2,
                                   int32_t *zero2);

/* ---- linear ----------------------------------------------------------- */

/* iro_int8_linear_ex (ops.c:450-491): int32 work[M,N] = q . W^T (u8 x s8,
   raw, as cblas_gemm_s8u8s32 with zero offsets) and
   y = float(work - zero*colsum) * (scale*w.scale) [+ bias], or y += ... when
   accumulate.  work may be NULL (then it is not written).  q rows are
   K bytes apart. */
int iro_hip_int8_linear_ex(IroHipContext *ctx, const uint8_t *q, const float *scale,
                           const int32_t *zero, const IroHipWeight *w, const float *bias,
                           float *y, int M, int32_t *work, int accumulate);

/* Two quantized planes of one activation against the same weight in one
   pass (dit.c:477-485 int8_scratch_linear with residual):
   y = lin(q1) [+bias]; y += lin(q2). */
int iro_hip_int8_linear_two_term(IroHipContext *ctx, const uint8_t *q1, const float *scale1,
                                 const int32_t *zero1, const uint8_t *q2,
                                 const float *scale2, const int32_t *zero2,
                                 const IroHipWeight *w, const float *bias, float *y, int M,
                                 int accumulate);

/* ---- fused DiT projections (device memory, rows m = b*S + s) ---------- */

/* dit.c:780-798: quantize x [M,D] once, one GEMM against the fused QKVG
   weight ([4D,D], layout 0), split store into q,k,v,gate [M,D].
   residual != 0 runs the two-term activation (IRO_INT8_RESIDUAL bit 1). */
int iro_hip_dit_qkvg(IroHipContext *ctx, const float *x, int M, const IroHipWeight *w_qkvg,
                     float *q, float *k, float *v, float *gate, int residual);

/* dit.c:876-884 then dit.c:1013-1020: quantize mix [M,D], GEMM with w
   ([D,D]) and, when x_res is not NULL, x_res[b,s,:] += gate[b,:] * out
   fused in the epilogue (out then may be NULL); otherwise out = result. */
int iro_hip_dit_linear_gated(IroHipContext *ctx, const float *mix, int M,
                             const IroHipWeight *w, int residual, float *out, float *x_res,
                             const float *gate, int S);

/* iro_hip_dit_linear_gated without any device allocation, for callers that
   cannot allocate (code under HIP graph capture, tight serving loops,
   harnesses that forbid hipMalloc).  No counterpart in the reference.  The
   quantized activation is staged in a fixed per-GPU scratch of 16 MiB held
   from library load to process end instead of the context's growable
   workspace: M rows of K codes (two planes when residual) plus their
   scales and zero points must fit, else the call fails with an error (at
   K = 1024 that is up to about 8000 rows, 4000 with two planes).  Every
   call on one GPU shares that scratch, so calls that overlap on one GPU
   (other streams, other threads, other contexts) race.  Results are
   identical to iro_hip_dit_linear_gated. */
int iro_hip_dit_linear_gated_noalloc(IroHipContext *ctx, const float *mix, int M,
                                     const IroHipWeight *w, int residual, float *out,
                                     float *x_res, const float *gate, int S);

/* dit.c:939-972 then dit.c:1032-1039: SwiGLU MLP.  h [M,D] quantized once;
   fused W1/W3 GEMM (layout 1 weight, [2H,D]) whose epilogue writes
   hidden = silu(w1)*w3 [M,H]; hidden quantized with the two-term residual
   when residual_w2 (the reference default, dit.c:422-436); W2 ([D,H]) GEMM
   over both planes; x_res += gate * out fused when x_res is not NULL,
   else out = result.  hidden may be NULL (context scratch is used).
   The gate's expf is evaluated in double precision and rounded once, which
   matches glibc's scalar expf except where glibc itself misrounds. */
int iro_hip_dit_swiglu(IroHipContext *ctx, const float *h, int M, const IroHipWeight *w13,
                       const IroHipWeight *w2, int residual_w13, int residual_w2,
                       float *hidden, float *out, float *x_res, const float *gate, int S);

/* ---- weight source: safetensors checkpoints, packed weight files ------- */

/* A safetensors checkpoint opened read-only through mmap, its header parsed
   and checked as iro_st_load checks it (safetensors.c:302-497): header
   length inside the file, every tensor with a known dtype (IroDType order:
   0 F32, 1 F16, 2 BF16, 3 I64, 4 I32, 5 I16, 6 I8, 7 U8, 8 BOOL), at most 8
   dimensions, data_offsets inside the data section and numel x item size
   equal to its byte length; "__metadata__" an object of strings.  Needs no
   device.  Returns 0, or -1 with iro_hip_st_last_error() set. */
typedef struct IroHipSafetensors IroHipSafetensors;
int iro_hip_st_open(const char *path, IroHipSafetensors **out);
void iro_hip_st_close(IroHipSafetensors *st);
const char *iro_hip_st_last_error(void);
/* Number of tensors and the i-th name (header order). */
int iro_hip_st_count(const IroHipSafetensors *st);
const char *iro_hip_st_name(const IroHipSafetensors *st, int i);
/* safetensors.c:520-524 iro_st_get: dtype, ndims, shape[8], a pointer into
   the mapping and the byte length of the named tensor; -1 if absent. */
int iro_hip_st_tensor(const IroHipSafetensors *st, const char *name, int *dtype, int *ndims,
                      uint64_t *shape, const void **data, uint64_t *nbytes);
/* safetensors.c:526-530 iro_st_meta: the metadata value, NULL if absent. */
const char *iro_hip_st_meta(const IroHipSafetensors *st, const char *key);
/* The int8 weight of a 2-D F32 / F16 / BF16 tensor ([N, K] rows = output
   rows, or [K, N] with transposed = 1), 16-bit formats widened exactly:
   uploaded, quantized and packed as iro_hip_weight_create does, the step
   the reference takes at engine init from its mmapped tensors
   (generate.c:526-544, iro_dit_int8_quantize).  The fp32 copy is not kept. */
int iro_hip_weight_from_st(IroHipContext *ctx, const IroHipSafetensors *st, const char *name,
                           int transposed, IroHipWeight **out);
/* The packed int8 weight (fragments, scales, sums, shape, layout, parts and
   the rounding convention its codes were made under) as a file, and back
   without re-quantizing: no counterpart in the reference, which quantizes
   at every engine init; for callers that start often.  Loading checks the
   header, the size, a 64-bit checksum of the payload and that the
   convention matches the context's. */
int iro_hip_weight_save(IroHipContext *ctx, const IroHipWeight *w, const char *path);
int iro_hip_weight_load(IroHipContext *ctx, const char *path, IroHipWeight **out);

/* ---- fp32 neighbours ------------------------------------------------------ */

/* dit.c:543-588, the parameters of n_adaln (1 or 2) adaLNs from cond [B, 3D]:
   for adaLN a and branch br (shift, scale, gate), act = silu(cond[:, br*D:
   (br+1)*D]) as x / (1 + expf(-x)); low = act @ down^T (down [R, D]) summed
   in index order; out = (low @ up^T (up [D, R]) in index order + bias) +
   the cond slice; the gate branch then through glibc's tanhf.  weights: a
   host array of 9 * n_adaln device pointers, per adaLN in dit.h's IroAdaLN
   order (shift_down, shift_up, shift_bias, scale_down, ..., gate_bias).
   out [n_adaln][3][B][D] device memory -- the shift, scale and gate that
   iro_hip_dit_adaln_apply and the gated residuals take.  Bit-identical to the
   scalar build. */
int iro_hip_dit_adaln_params(IroHipContext *ctx, const float *cond, int B, int D, int R,
                             const float *const *weights, int n_adaln, float *out);

/* The device tanhf on all 2^32 float inputs as one digest, to compare with
   the same digest of libm's tanhf computed on the host (equal exactly when
   every result agrees, barring a hash collision); takes a few seconds. */
int iro_hip_selfcheck_tanhf(IroHipContext *ctx, unsigned long long *digest);

/* ops.c:221-234, iro_linear of the scalar build: y [M, N] = x [M, K] @ w
   [N, K]^T with each output a K-order chain of rounded products, then +
   bias[n] (bias may be NULL: + 0).  Device memory.  Bit-identical to the
   scalar build (the DiT's input / output projections, dit.c:532-540 and
   1070-1089, and the context K/V projections, dit.c:708-735). */
int iro_hip_linear_f32(IroHipContext *ctx, const float *x, int M, int K, const float *w, int N,
                       const float *bias, float *y);

/* sampler.c:281-297, the CFG combine and Euler update of one sampler step,
   on device memory: state [len] += guided * dt with guided = v + sum over
   the unconditional rows k of scale_k * (v - v_k), where velocity holds
   `batch` rows of len values (row 0 conditional; batch 1..4) and
   text_row / speaker_row / caption_row are the unconditional rows (1 ..
   batch-1, or -1 when that branch has no CFG row; sampler.c:133-139).  With
   use_cfg == 0 (sampler.c:247-249) guided = v, batch may be 1 and the rows
   (1..3 or -1) are not read.  dt = timestep_next -
   timestep as sampler.c:243-246, 281 computes it.  Bit-identical to the
   strict build, and to the fast-math build's reassociated form under
   IRO_HIP_GCC_FASTMATH.  Replaces the host loop between iro_dit_output and
   the next step of sample_euler, so the state stays on the device. */
int iro_hip_euler_update(IroHipContext *ctx, float *state, const float *velocity, int len,
                         int batch, int use_cfg, int text_row, int speaker_row, int caption_row,
                         float scale_text, float scale_speaker, float scale_caption, float dt);

/* ops.c:738-747, iro_rmsnorm: y = (x * inv) * w[d], inv = 1 / sqrtf(mean of
   x^2 in index order + eps), rows of D (D % 4 == 0, D <= 2048, 16-byte
   aligned).  Bit-identical to the scalar build (the DiT's output norm,
   dit.c:1082). */
int iro_hip_rmsnorm_f32(IroHipContext *ctx, const float *x, int M, int D, const float *w,
                        float eps, float *y);

/* dit.c:593-606, the apply step of dit_adaln: h = x * inv * (1 + scale[b])
   + shift[b] for row r of x [B*S, D] (b = r / S, shift/scale [B, D]) with
   inv = 1 / sqrtf(mean(x^2) + eps), the sum of squares taken in index order
   as the strict build does, so h is bit-identical to it.  (The fast-math
   build vectorizes that sum in a host-dependent order.)  shift and scale
   come from the caller (dit.c:580-588 computes them with fp32 low-rank
   linears on the host). */
int iro_hip_dit_adaln_apply(IroHipContext *ctx, const float *x, int B, int S, int D,
                            const float *shift, const float *scale, float eps, float *h);

/* dit.c:638-706 head_rmsnorm_rope_pair, in place on q and k [B*S, D]
   (D = heads * 64, 16-byte aligned): per 64-wide head row, inv = 1 /
   sqrtf(mean(x^2) + eps) with the squares summed in index order, x = x *
   (inv * weight[h*64 + d]); heads h < heads/2 then rotate pair p by position
   s = row % S of the reference's table (double recurrence of the step 1 /
   10000^(2p/64), dit.c:641-657, 697-703).  Bit-identical to the strict build.
   The context keeps the table; a call with more positions than any before it
   allocates and uploads a longer one (so the first call per length is not
   capturable). */
int iro_hip_dit_qk_norm_rope(IroHipContext *ctx, float *q, const float *q_weight, float *k,
                             const float *k_weight, int B, int S, int D, float eps);

/* dit.c:619-636 head_rmsnorm (the text and speaker keys, no rotation), in
   place on x [B*S, D]; same arithmetic as above. */
int iro_hip_dit_head_rmsnorm(IroHipContext *ctx, float *x, const float *weight, int B, int S,
                             int D, float eps);

/* The joined-key layout of one utterance's attention context
   (dit.c:815-843): per batch b, the context rows ci < C whose
   mask[b*C + ci] (host memory) is set, in order -- row ci of the shared
   context when context_batch == 1 (iro_dit_attention_shared_context,
   dit.c:903-911), row b*C + ci when context_batch == B (iro_dit_attention,
   dit.c:895-901).  Made once per utterance (the mask does not change across
   layers and sampler steps); it allocates and uploads.  Destroy it before
   its context. */
typedef struct IroHipAttnContext IroHipAttnContext;
int iro_hip_dit_attn_context_create(IroHipContext *ctx, const uint8_t *mask, int B, int C,
                                    int context_batch, IroHipAttnContext **out);
void iro_hip_dit_attn_context_destroy(IroHipAttnContext *actx);

/* dit.c:808-870, the attention core between head_rmsnorm_rope_pair and Wo,
   as the reference's scalar build computes it (ops.c:577-600 scores, 754-766
   softmax, 681-703 P@V, 786-789 gate): per batch b and head h, the joined
   keys are the S tokens of b (rows of k, v) then the kept context rows (of
   context_k, context_v, [(context_batch == 1 ? 1 : B) * C, D]);
   mix[b*S + s, h*64 + n] = sum_j softmax(q.k_j / 8)_j v_j[n], every sum in
   the scalar build's order, times 1 / (1 + expf(-gate)).  q, k, v, gate, mix
   [B*S, D], D = heads * 64, all 16-byte aligned device memory.  B may be below
   actx's batch (rows 0 .. B-1 of its mask are used).  Bit-identical
   to the scalar build.  Workspace: 4 * B * heads * S * (S + kept rows,
   rounded up to 128) bytes of scores. */
int iro_hip_dit_attention(IroHipContext *ctx, const IroHipAttnContext *actx, const float *q,
                          const float *k, const float *v, const float *gate, int B, int S, int D,
                          const float *context_k, const float *context_v, float *mix);

/* ---- the int8 linear stack of one Euler step --------------------------- */

/* The int8 projections of `blocks` DiT blocks (dit.h:51-58 IroDiTInt8,
   built once as iro_dit_int8_quantize does, dit.c:235-259), device
   resident.  residual_mask has IRO_INT8_RESIDUAL's meaning (dit.c:278-291:
   1 QKVG, 2 Wo, 4 W1/W3, 8 W2; the reference default is 8). */
typedef struct IroHipDiTStack IroHipDiTStack;
int iro_hip_dit_stack_create(IroHipContext *ctx, int blocks, int D, int H, int residual_mask,
                             IroHipDiTStack **out);
/* Device fp32 weights of one block: ada [6D,D] (modulation linear),
   wq/wk/wv/wgate/wo [D,D], w1/w3 [H,D], w2 [D,H].  ada may be NULL: only
   iro_hip_dit_stack_step reads the modulation weight (the block forward and
   the sampler step take fp32 adaLN parameters, dit.c:543-588). */
int iro_hip_dit_stack_set_block(IroHipDiTStack *s, int block, const float *ada, const float *wq,
                                const float *wk, const float *wv, const float *wgate,
                                const float *wo, const float *w1, const float *w3,
                                const float *w2);
/* One step of every block's int8 linears (the dit_block sequence,
   dit.c:983-1040): mod = ada . cond [B,6D]; QKVG on x; Wo on V with
   x += mod[:,2D:3D] * out; SwiGLU on x with x += mod[:,5D:6D] * out.
   x [B*S, D] is updated in place, cond is [B, D].  The fp32 attention core
   and RMSNorm-modulate between the projections are not part of this path
   (Wo reads V; QKVG and W1/W3 read x). */
int iro_hip_dit_stack_step(IroHipDiTStack *s, float *x, const float *cond, int B, int S);
/* Resident int8 bytes, iro_int8_weight_bytes summed (generate.h:43-46). */
size_t iro_hip_dit_stack_bytes(const IroHipDiTStack *s);
/* Device pointers of the step's activation buffers: the last block's q, k,
   v, gate [M,D] and hidden [M,H], and the modulation rows of every block
   [B, blocks*P] with block b at column b*P, P = 6D rounded up to 256. */
int iro_hip_dit_stack_buffers(IroHipDiTStack *s, float **q, float **k, float **v, float **gate,
                              float **hidden, float **mod);
void iro_hip_dit_stack_destroy(IroHipDiTStack *s);
/* Steps with the same x, cond, B and S as the previous step replay a HIP
   graph of the whole step (default on); off runs every launch directly.
   The profiler (iro_hip_profile_enable) always runs steps directly. */
int iro_hip_dit_stack_use_graph(IroHipDiTStack *s, int on);
/* Steps run as one persistent kernel after the modulation GEMM (default
   off; where supported: D a multiple of 256 up to 1024, H a multiple of 256
   up to 3072, residual_mask 0 or 8, int8 mask 15): workgroups take
   quantization and GEMM items of their own XCD's rows from a queue, so the
   hand-offs stay in one L2.  Off runs one kernel per quantization and GEMM.
   Results are identical either way; no counterpart in the reference. */
int iro_hip_dit_stack_use_persistent(IroHipDiTStack *s, int on);
/* IRO_INT8_MASK (dit.c:273-291): the projection groups that run in int8
   (1 Q/K/V/gate, 2 Wo, 4 W1/W3, 8 W2; default 15).  A group whose bit is
   clear runs through iro_hip_linear_f32 (the reference's iro_linear) on a
   device copy of its fp32 weights that set_block keeps, with the SiLU gate
   and gated residual as separate fp32 passes (ops.c:781-784,
   dit.c:1013-1039); the int8 weights are built regardless, as
   iro_dit_int8_quantize builds all of them, so iro_hip_dit_stack_bytes is
   unchanged.  Must be set before the first set_block. */
int iro_hip_dit_stack_set_int8_mask(IroHipDiTStack *s, int mask);
int iro_hip_dit_stack_get_int8_mask(const IroHipDiTStack *s);
/* Concurrent row runs of iro_hip_dit_stack_step (no counterpart in the
   reference; a scheduling choice): with runs > 1 the step forks after the
   modulation GEMM into one stream per CFG branch (B > 1) or per slice of
   whole 32-row blocks of S (B = 1, up to `runs` slices), each taking its
   rows through every block, and joins them before returning.  Rows are
   independent through the linear stack, so the results are identical; the
   runs' kernels overlap on the GPU.  0 or 1: one stream (default). */
int iro_hip_dit_stack_set_runs(IroHipDiTStack *s, int runs);

/* One DiT block forward (dit.c:984-1040 dit_block) on the device, in place on
   x [B*S, D], with this stack's int8 weights of `block`: adaLN apply, fused
   QKVG, QK-norm + half-RoPE, the attention core with the context of actx,
   Wo with x += gate * branch, adaLN apply, W1/W3 + SiLU gate, W2 with
   x += gate * branch -- the reference's order and arithmetic at every step,
   so x is bit-identical to iro_dit_block of the scalar build given the same
   adaLN parameters.  ada_attn and ada_mlp are [3, B, D] device arrays:
   shift, scale and the tanhf'd gate of dit_adaln (dit.c:580-588) for each
   half; q_norm, k_norm [D].  Uses the stack's activation buffers; not
   capturable (the attention workspace may grow). */
int iro_hip_dit_stack_block_forward(IroHipDiTStack *s, int block, float *x, int B, int S,
                                    const float *ada_attn, const float *ada_mlp,
                                    const float *q_norm, const float *k_norm, float eps,
                                    const IroHipAttnContext *actx, const float *context_k,
                                    const float *context_v);

/* The fp32 parameters of one DiT layer that a sampler step reads besides the
   stack's int8 weights (dit.h:11-35): the attention then the MLP IroAdaLN
   (shift_down, shift_up, shift_bias, scale_down, scale_up, scale_bias,
   gate_down, gate_up, gate_bias each), the head norms [D], and the layer's
   cached context keys and values ([C, D] shared by the CFG rows, or
   [B*C, D] per row, as the attention context says; sampler.c:215-236 fills
   them once per utterance).  Device arrays, borrowed until the layer is set
   again or the stack is destroyed. */
typedef struct {
    const float *adaln[18];
    const float *q_norm, *k_norm;
    const float *context_k, *context_v;
} IroHipDiTLayerF32;

/* The DiT's input and output heads (dit.c:146-150: in_proj [D, latent] and
   bias [D], out_norm [D], out_proj [latent, D] and bias [latent]), the adaLN
   rank (ADALN_RANK, dit.c:16) and the norm epsilon; device arrays, borrowed. */
typedef struct {
    const float *in_w, *in_b, *out_norm, *out_w, *out_b;
    int latent;
    int rank;
    float eps;
} IroHipDiTHead;

int iro_hip_dit_stack_set_layer_f32(IroHipDiTStack *s, int layer, const IroHipDiTLayerF32 *p);
int iro_hip_dit_stack_set_head(IroHipDiTStack *s, const IroHipDiTHead *head);

/* One Euler step of sample_euler (sampler.c:259-297) on the device, with
   every layer's weights set: the input projection of state [S, latent]
   (iro_dit_input), broadcast to the `batch` CFG rows, every layer's adaLN
   parameters from cond [batch, 3D] (the caller uploads iro_dit_condition's
   row, broadcast, as sampler.c:262-266 does) and block forward with the
   context of actx (iro_dit_block_shared_context), the output RMSNorm and
   projection into velocity [batch*S, latent] (iro_dit_output; the trace
   callback's velocity), then the CFG combine and Euler update of state in
   place (iro_hip_euler_update's arguments).  Each part is bit-identical to
   the reference's scalar build, so the step is too; only cond crosses PCIe
   per step.  batch may be below actx's batch: a plain step (use_cfg 0,
   batch 1, sampler.c:247-249) reads mask row 0 of the CFG context, as the
   reference does.  Every argument is checked before the first launch.
   Steps with the same state, cond, batch, S, actx and velocity as the
   previous one (and use_graph on) replay a HIP graph of the network
   forward (input projection to velocity), captured on the second such
   step; the CFG / Euler update, whose scalars change per step, is launched
   after it. */
int iro_hip_dit_sampler_step(IroHipDiTStack *s, float *state, const float *cond, int batch,
                             int S, const IroHipAttnContext *actx, int use_cfg, int text_row,
                             int speaker_row, int caption_row, float scale_text,
                             float scale_speaker, float scale_caption, float dt,
                             float *velocity);

/* iro_dit_condition (dit.c:488-530) on the device: the timestep embedding
   of t [B] (cos then sin of t * 1000 expf(-log(10000) i / half), half =
   tdim / 2, with glibc's expf, cosf and sinf), then linear w0 [D, tdim],
   SiLU, linear w1 [D, D], SiLU, linear w2 [cond_dim, D], no biases, into
   cond [B, cond_dim].  Bit-identical to the strict build; the fast build
   vectorises the embedding with libmvec, which is not restated. */
int iro_hip_dit_condition(IroHipContext *ctx, const float *t, int B, const float *w0,
                          const float *w1, const float *w2, int tdim, int D, int cond_dim,
                          float *cond);
/* ops.c:776-784 in place on n device floats: x = x / (1 + expf(-x)), times
   gate[i] when gate is not NULL (iro_silu_inplace / iro_silu_mul_inplace,
   glibc's expf, the strict build's rounding). */
int iro_hip_silu(IroHipContext *ctx, float *x, const float *gate, long long n);
/* dit.c:1013-1020: x[m][d] += gate[(m / S) * ldg + d] * branch[m][d] for M
   rows of D (two roundings; one fma under IRO_HIP_GCC_FASTMATH). */
int iro_hip_gated_residual(IroHipContext *ctx, float *x, const float *gate, int ldg,
                           const float *branch, int M, int D, int S);

/* ---- DACVAE int8 Conv1d (dacvae.c:543-688, no snake) ------------------- */

/* input [T, C] fp32 time-major, weight [N, kernel*C] (tap-major K as
   iro_dacvae_int8_quantize lays it out, dacvae.c:228-240), bias [N] or
   NULL; residual adds the fixed-scale second plane (dacvae.c:637-663).
   output [T_out, N].  Each output row is quantized over its whole
   kernel*C window with one scale and zero point; padding taps hold the zero
   point.  Returns T_out through *t_out when not NULL. */
int iro_hip_conv1d_int8(IroHipContext *ctx, const float *input, int T, int C,
                        const IroHipWeight *w, int kernel, int stride, int dilation,
                        int padding, const float *bias, int residual, float *output,
                        int *t_out);

/* dacvae.c:696-795 (convtranspose1d_forward_impl, int8 weight, no snake):
   input [T_in, C_in] fp32 time-major; w from iro_hip_weight_create_transposed
   of the [C_in, kernel, C_out] export layout (N = kernel*C_out, K = C_in,
   dacvae.c:239-243); output [T_out, C_out] with T_out =
   (T_in-1)*stride - 2*padding + kernel + output_padding (dacvae.c:350-358).
   The input rows are quantized per row (two-term when residual, the
   IRO_CODEC_GROUP_UPSAMPLE policy bit), one int8 GEMM forms the expanded
   [T_in, kernel*C_out] rows, and each output row is bias plus the taps that
   land on it, added in ascending input row as the reference's scatter
   loop does.  *t_out (nullable) receives T_out. */
int iro_hip_convtranspose1d_int8(IroHipContext *ctx, const float *input, int T_in, int C_in,
                                 const IroHipWeight *w, int C_out, int kernel, int stride,
                                 int padding, int output_padding, const float *bias,
                                 int residual, float *output, int *t_out);

/* dacvae.c:974-1012, the int8 1x1 projection of a decoder residual unit:
   output = skip + conv1(hidden) + bias, with hidden [T, C_in] quantized per
   row (two-term when residual: the IRO_CODEC_GROUP_CONV1 policy bit and
   stage mask of dacvae.c:27-73), w the [C_out, C_in] 1x1 weight, skip and
   output [T, C_out] (output may be skip: it is then updated in place;
   otherwise the two must not overlap).  The snake activations around it
   are fp32 neighbours, not part of this call. */
int iro_hip_conv1x1_skip_int8(IroHipContext *ctx, const float *hidden, const float *skip, int T,
                              const IroHipWeight *w, const float *bias, int residual,
                              float *output);

/* ---- DACVAE decoder: snake, residual unit, int8 core ------------------- */

/* iro_snake_forward (dacvae.c:830-857): y = x + sin(a x)^2 / a per element
   of the time-major [T, C] rows (alpha [C]); up to 1536 channels with the
   hoisted reciprocal 1 / (a + 1e-9), wider rows with the quotient.  sinf
   is glibc's, bit for bit.  y may be x.  C % 4 == 0, 16-byte aligned rows.
   Bit-exact against the strict build; the fast build's vectorised libmvec
   sinf is not restated (its results are compared within a tolerance). */
int iro_hip_snake(IroHipContext *ctx, const float *x, int T, int C, const float *alpha,
                  float *y);
/* snake_bias_forward (dacvae.c:910-931): v = x + bias, y = snake(v); the
   hoisted reciprocal only in place (y == x) up to 1536 channels. */
int iro_hip_snake_bias(IroHipContext *ctx, const float *x, int T, int C, const float *bias,
                       const float *alpha, float *y);
/* Digests (the iro_hip_selfcheck_silu form) of the device sinf and cosf
   over all 2^32 float inputs, to be compared with glibc's (no counterpart
   in the reference; a test hook). */
int iro_hip_selfcheck_sincosf(IroHipContext *ctx, unsigned long long *sin_digest,
                              unsigned long long *cos_digest);

/* run_residual_int8 (dacvae.c:934-1018) with the int8 group mask 15:
   hidden = Conv7(snake(input, alpha0)) (dilation d, padding 3d, no bias,
   second activation plane when residual_conv7), snake_bias in place with
   conv0_bias and alpha1, output = input + conv1(hidden) + conv1_bias
   (second plane when residual_conv1).  conv0 from iro_hip_weight_create of
   the [C, 7, C] export ([C, 7C]), conv1 [C, C].  input and output [T, C],
   distinct.  The reference's residual flags are the policy of
   dacvae.c:27-73: (IRO_CODEC_INT8_RESIDUAL & group) and bit `stage` of
   IRO_CODEC_INT8_RESIDUAL_STAGES. */
int iro_hip_dacvae_residual_int8(IroHipContext *ctx, const float *input, int T, int C,
                                 const IroHipWeight *conv0, const float *alpha0,
                                 const float *conv0_bias, const float *alpha1, int dilation,
                                 const IroHipWeight *conv1, const float *conv1_bias,
                                 int residual_conv7, int residual_conv1, float *output);

#define IRO_HIP_DACVAE_STAGES 4
#define IRO_HIP_DACVAE_RESIDUALS 3

/* The decoder's fp32 parameters (IroDACVAEDecoder, dacvae.h:36-76) as
   device pointers in the export layouts, borrowed: they must outlive the
   IroHipDACVAE made from them. */
typedef struct {
    const float *alpha0, *conv0_weight, *conv0_bias; /* [C], [C, 7, C], [C] */
    const float *alpha1, *conv1_weight, *conv1_bias; /* [C], [C, 1, C], [C] */
    int dilation;                                    /* 1, 3, 9 (dacvae.c:187) */
} IroHipDACVAEResidualF32;
typedef struct {
    const float *alpha;     /* [c_in], the snake before the upsample */
    const float *up_weight; /* [c_in, kernel, c_out] */
    const float *up_bias;   /* [c_out] */
    int c_in, c_out, kernel, stride, padding, output_padding;
    IroHipDACVAEResidualF32 residual[IRO_HIP_DACVAE_RESIDUALS];
} IroHipDACVAEStageF32;
typedef struct {
    const float *initial_weight; /* [channels, 7, latent_channels] */
    const float *initial_bias;   /* [channels] */
    int latent_channels, channels; /* 1024, 1536 */
    IroHipDACVAEStageF32 stage[IRO_HIP_DACVAE_STAGES];
} IroHipDACVAEDecoderF32;
typedef struct IroHipDACVAE IroHipDACVAE;

/* iro_dacvae_int8_quantize (dacvae.c:228-262): the initial conv as
   [channels, 7 latent], each upsample transposed to [kernel c_out, c_in],
   each residual unit's conv0 [C, 7C] and conv1 [C, C], quantized and packed
   on the device.  Refuses stages whose channels do not chain. */
int iro_hip_dacvae_create(IroHipContext *ctx, const IroHipDACVAEDecoderF32 *params,
                          IroHipDACVAE **out);
/* IroDACVAEInt8.bytes: iro_int8_weight_bytes summed over the 26 weights. */
size_t iro_hip_dacvae_int8_bytes(const IroHipDACVAE *d);
void iro_hip_dacvae_destroy(IroHipDACVAE *d);
/* Frames after the four upsamples (iro_convtranspose1d_output_length
   chained, dacvae.c:350-358), or -1. */
int iro_hip_dacvae_output_frames(const IroHipDACVAE *d, int frames);
/* The int8 core of iro_dacvae_decode (dacvae.c:1221-1277) with all four
   groups in int8 (IRO_CODEC_INT8_MASK 15): state [frames, latent] (the
   quantizer_out result) -> initial conv (second plane when residual_mask
   & 1) -> per stage snake + upsample (& 2) and three residual units (& 4,
   & 8, each only in the stages of residual_stages) -> out
   [output_frames, last c_out].  The fp32 quantizer_out before it and the
   final snake + 96->1 tap + tanh after it stay with the caller, as the
   reference keeps them in fp32.  The defaults are residual_mask 12,
   residual_stages 8 (dacvae.c:51-69). */
int iro_hip_dacvae_decode_int8(IroHipDACVAE *d, const float *state, int frames,
                               int residual_mask, int residual_stages, float *out);

/* ---- per-kernel event profiler ----------------------------------------- */

/* While enabled, every kernel launch on the context is bracketed by HIP
   events on its stream and accumulated per kernel kind (the role of the
   reference's IRO_GEMM_PROFILE / IRO_DIT_PROFILE, ops.c:14-110,
   dit.c:22-120).  Reading collects pending events (synchronizes). */
int iro_hip_profile_enable(IroHipContext *ctx, int on);
int iro_hip_profile_reset(IroHipContext *ctx);
int iro_hip_profile_kinds(void);
/* Totals for `kind` in [0, iro_hip_profile_kinds()): launches, summed
   milliseconds, algorithmic ops (2*M*N*K per plane) and HBM bytes. */
int iro_hip_profile_read(IroHipContext *ctx, int kind, const char **name, long long *launches,
                         double *ms, double *ops, double *bytes);

/* ---- backend queries: ops.h:55-78 ------------------------------------- */

/* Runs the ops.c:375-398 known answer through the MFMA GEMM: 0 exact. */
int iro_hip_selfcheck(IroHipContext *ctx);
/* Test hook (the counterpart of the reference refusing an inexact backend
   at init, generate.c:527-536): while on, the known answer's input is
   altered after its expected sums are computed, so iro_hip_selfcheck and
   iro_hip_create must refuse.  Process-wide. */
int iro_hip_selfcheck_inject_fault(int on);
/* Exhaustive check of the SiLU gate's device pieces over all 2^32 float
   inputs (no counterpart in the reference; a test hook): exp_digest = sum
   mod 2^64 of (bits(x) * 0x9E3779B97F4A7C15) ^ (bits(expf(x)) *
   0xC2B2AE3D27D4EB4F) for the device's glibc-exact expf (NaN results as
   0x7FC00000), to be compared with the same sum over glibc's expf;
   div_mismatches = inputs a whose fast quotient a / (1 + expf(-a)) differs
   from the IEEE division (0 expected).  Takes well under a second. */
int iro_hip_selfcheck_silu(IroHipContext *ctx, unsigned long long *exp_digest,
                           unsigned long long *div_mismatches);
/* Exhaustive check of the code packing every activation quantizer uses
   (no counterpart in the reference; a test hook): the number of float
   inputs v whose packed u8 code differs from the reference's
   clamp(nearbyintf(v), 0, 255) (NaN: 0).  0 expected. */
int iro_hip_selfcheck_codes(IroHipContext *ctx, unsigned long long *mismatches);
/* Exhaustive digests (same form) of the device's sqrtf(x) and 1 / x over all
   2^32 float inputs, to be compared with the host's IEEE results: the
   correctly rounded operations the adaLN apply relies on (no counterpart in
   the reference; a test hook). */
int iro_hip_selfcheck_fp32(IroHipContext *ctx, unsigned long long *sqrt_digest,
                           unsigned long long *recip_digest);
/* "gfx950 MFMA i8" plus device name; never NULL. */
const char *iro_hip_backend_name(IroHipContext *ctx);

#ifdef __cplusplus
}
#endif

#endif
