// iro_codec.hip -- the DACVAE decoder's int8 path around the convolutions:
// the snake activations (dacvae.c:803-925), the residual unit
// (run_residual_int8, dacvae.c:934-1018), the decoder's int8 weight set
// (IroDACVAEInt8, dacvae.h:53-67, built as iro_dacvae_int8_quantize does,
// dacvae.c:228-262) and the int8 part of iro_dacvae_decode
// (dacvae.c:1221-1290: initial conv, then per stage snake + upsample and
// three residual units).
//
// Snake: y = x + sin(a x)^2 / a with the reference's scalar arithmetic:
// channels <= 1536 take the hoisted reciprocal inv = 1 / (a + 1e-9),
// y = x + (s * s) * inv; wider rows the quotient y = x + (s * s) / (a + 1e-9)
// (dacvae.c:827-857); sinf is glibc's (iro_sincosf.h).  Bound by HBM: 8
// bytes per element in and out.
#include <cmath>
#include <cstring>
#include <new>
#include <algorithm>

#include "iro_internal.h"
#include "iro_round.h"
#include "iro_snake.h"

namespace iro {
namespace {

// One thread per four consecutive elements of a row (C % 4 == 0, rows
// 16-byte aligned).  BIAS: v = x + bias (snake_bias_forward).  INV: the
// hoisted-reciprocal form.  FMA: the fast build's contraction of the final
// add into one fma.
// With INV (C <= 1536) the block first stages alpha and inv = 1 / (alpha +
// 1e-9) per channel in LDS, as the reference hoists its reciprocal
// (dacvae.c:827-828).
template <bool BIAS, bool INV, bool FMA>
__global__ __launch_bounds__(256) void snake_kernel(const float *__restrict__ x, int C,
                                                    long long n4, const float *__restrict__ bias,
                                                    const float *__restrict__ alpha, float *y) {
    __shared__ float s_alpha[INV ? kSnakeMaxChannels : 1], s_inv[INV ? kSnakeMaxChannels : 1];
    __shared__ uint32_t s_pio4[24];
    stage_invpio4(s_pio4, threadIdx.x);
    if (INV) {
        for (int c = threadIdx.x; c < C; c += 256) {
            const float a = alpha[c];
            s_alpha[c] = a;
            s_inv[c] = snake_inv(a);
        }
    }
    __syncthreads();
    for (long long i = blockIdx.x * 256ll + threadIdx.x; i < n4; i += (long long)gridDim.x * 256) {
        const long long e = 4 * i;
        const int c = (int)(e % C);
        float4 v = *reinterpret_cast<const float4 *>(x + e);
        if (BIAS) {
            v.x = v.x + bias[c];
            v.y = v.y + bias[c + 1];
            v.z = v.z + bias[c + 2];
            v.w = v.w + bias[c + 3];
        }
        const float *ap = INV ? s_alpha : alpha;
        const float4 a = make_float4(ap[c], ap[c + 1], ap[c + 2], ap[c + 3]);
        const float4 inv = INV ? make_float4(s_inv[c], s_inv[c + 1], s_inv[c + 2], s_inv[c + 3])
                               : make_float4(0.f, 0.f, 0.f, 0.f);
        *reinterpret_cast<float4 *>(y + e) = snake_value4<INV, FMA>(v, a, inv, s_pio4);
    }
}

// Exhaustive digests of the device sinf and cosf over the 2^28 inputs from
// base: the sum mod 2^64 of (bits(x) * 0x9E3779B97F4A7C15) ^ (bits(f(x)) *
// 0xC2B2AE3D27D4EB4F), NaN results counted as 0x7FC00000.
__global__ __launch_bounds__(256) void sincosf_selfcheck_kernel(unsigned long long *out,
                                                                unsigned base) {
    __shared__ unsigned long long part[2][4];
    const unsigned u = base + blockIdx.x * 256u + threadIdx.x;
    const float x = __uint_as_float(u);
    unsigned long long h[2];
#pragma unroll
    for (int w = 0; w < 2; ++w) {
        const float t = sincosf_glibc(x, w);
        const unsigned ut = t != t ? 0x7FC00000u : __float_as_uint(t);
        h[w] = ((unsigned long long)u * 0x9E3779B97F4A7C15ull) ^
               ((unsigned long long)ut * 0xC2B2AE3D27D4EB4Full);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        h[0] += __shfl_xor(h[0], off, 64);
        h[1] += __shfl_xor(h[1], off, 64);
    }
    if ((threadIdx.x & 63) == 0) {
        part[0][threadIdx.x >> 6] = h[0];
        part[1][threadIdx.x >> 6] = h[1];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        atomicAdd(&out[0], part[0][0] + part[0][1] + part[0][2] + part[0][3]);
        atomicAdd(&out[1], part[1][0] + part[1][1] + part[1][2] + part[1][3]);
    }
}

int launch_snake(IroHipContext *ctx, const float *x, int T, int C, const float *bias,
                 const float *alpha, float *y, bool inv_form) {
    const long long n4 = (long long)T * C / 4;
    if (n4 == 0) return 0;
    long long blocks = (n4 + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    const dim3 g((unsigned)blocks), b(256);
    const bool fma = ctx->convention == IRO_HIP_GCC_FASTMATH;
    prof_begin(ctx);
#define IRO_SNAKE(B, I, F)                                                                       \
    hipLaunchKernelGGL((snake_kernel<B, I, F>), g, b, 0, ctx->stream, x, C, n4, bias, alpha, y)
    if (bias) {
        if (inv_form) {
            if (fma) IRO_SNAKE(true, true, true);
            else IRO_SNAKE(true, true, false);
        } else {
            IRO_SNAKE(true, false, false);
        }
    } else {
        if (inv_form) {
            if (fma) IRO_SNAKE(false, true, true);
            else IRO_SNAKE(false, true, false);
        } else {
            IRO_SNAKE(false, false, false);
        }
    }
#undef IRO_SNAKE
    IRO_HIP_CHECK_LAUNCH(ctx);
    // Algorithmic HBM bytes: the rows in and out.
    prof_end(ctx, PK_SNAKE, 0, 8.0 * T * C);
    return 0;
}

// iro_snake_forward (reciprocal form, C <= 1536) out of place, and each
// output row's lo/hi over its channels as conv_rows computes them
// (dacvae.c:607-616, lo and hi from 0): the snake a Conv7 applies to its
// input rows (dacvae.c:599-603) with the row ranges its quantization needs,
// in one pass.  A block takes R rows (R C <= 4096): phase 1 snakes them as
// flat float4 chunks (every lane busy) into y and an LDS tile, phase 2
// reduces each row of the tile with eight lanes (fmin/fmax: any order).
template <bool FMA>
__global__ __launch_bounds__(256) void snake_rows_kernel(const float *__restrict__ x, int T, int C,
                                                         int R, unsigned k4_magic,
                                                         const float *__restrict__ alpha,
                                                         float *__restrict__ y,
                                                         float *__restrict__ row_lo,
                                                         float *__restrict__ row_hi) {
    extern __shared__ __attribute__((aligned(16))) float snake_rows_lds[];
    __shared__ uint32_t s_pio4[24];
    float *s_a = snake_rows_lds, *s_i = s_a + C, *tile = s_i + C;
    stage_invpio4(s_pio4, threadIdx.x);
    for (int c = threadIdx.x; c < C; c += 256) {
        const float a = alpha[c];
        s_a[c] = a;
        s_i[c] = snake_inv(a);
    }
    const int row0 = blockIdx.x * R;
    const int rows = min(R, T - row0);
    const int k4 = C >> 2, chunks = rows * k4;
    float4 v4[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int f = threadIdx.x + 256 * j;
        if (f < chunks) v4[j] = *reinterpret_cast<const float4 *>(x + (size_t)row0 * C + 4 * f);
    }
    __syncthreads();  // the staged parameters
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int f = threadIdx.x + 256 * j;
        if (f < chunks) {
            const int c4 = f - (int)__umulhi(2u * f, k4_magic) * k4;
            const float4 a = *reinterpret_cast<const float4 *>(s_a + 4 * c4);
            const float4 i = *reinterpret_cast<const float4 *>(s_i + 4 * c4);
            const float4 o = snake_value4<true, FMA>(v4[j], a, i, s_pio4);
            *reinterpret_cast<float4 *>(y + (size_t)row0 * C + 4 * f) = o;
            *reinterpret_cast<float4 *>(tile + 4 * f) = o;
        }
    }
    __syncthreads();
    // eight lanes per row, 32 rows per pass: every lane of an aligned group
    // of eight shares the row, so the group exchange reads active lanes only
    const int sub = threadIdx.x & 7;
    for (int r = threadIdx.x >> 3; r < rows; r += 32) {
        float lo = 0.0f, hi = 0.0f;
        for (int c4 = sub; c4 < k4; c4 += 8) {
            const float4 v = *reinterpret_cast<const float4 *>(tile + r * C + 4 * c4);
            lo = sel_min(lo, v.x); lo = sel_min(lo, v.y); lo = sel_min(lo, v.z); lo = sel_min(lo, v.w);
            hi = sel_max(hi, v.x); hi = sel_max(hi, v.y); hi = sel_max(hi, v.z); hi = sel_max(hi, v.w);
        }
        lo = group8_range<false>(lo);
        hi = group8_range<true>(hi);
        if (sub == 0) {
            row_lo[row0 + r] = lo;
            row_hi[row0 + r] = hi;
        }
    }
}

bool snake_args_ok(const float *x, int T, int C, const float *alpha, const float *y) {
    return x && alpha && y && T >= 0 && C > 0 && C % 4 == 0 &&
           ((((uintptr_t)x) | ((uintptr_t)y)) & 15) == 0;
}

// dacvae.c:974-1012 (the int8 1x1 projection of run_residual_int8): the skip
// connection first (output = skip), then output += lin(q1) + bias and, with
// `residual` (the IRO_CODEC_GROUP_CONV1 policy bit for this stage),
// output += lin(q2), the rows of `hidden` quantized once per row.  Both
// planes run in one GEMM pass with the reference's rounding order; the
// epilogue reads the skip rows where the reference reads its copy of them,
// so no copy is made (output and skip are the same buffer or disjoint).
// With `snake` the rows are snaked (bias + alpha, reciprocal form) as they
// are quantized; returns 1, launching nothing, when that path declines.
int conv1x1_skip(IroHipContext *ctx, const float *hidden, const float *skip, int T,
                 const IroHipWeight *w, const float *bias, int residual, float *output,
                 const SnakePre *snake) {
    if (!ctx || !hidden || !skip || !w || !output || T <= 0)
        return set_error(ctx, "conv1x1_skip_int8: invalid arguments");
    const int C_in = w->K, C_out = w->N;
    const size_t rows_bytes = sizeof(float) * (size_t)T * C_out;
    const uintptr_t o = (uintptr_t)output, s = (uintptr_t)skip;
    if (o != s && o < s + rows_bytes && s < o + rows_bytes)
        return set_error(ctx, "conv1x1_skip_int8: output partly overlaps skip");
    Workspace ws{ctx};
    size_t off[6];
    act_reserve(ws, T, C_in, residual != 0, off);
    if (ws.commit()) return -1;
    const ActBufs b = act_at(ws, C_in, residual != 0, off);
    const int rc = launch_quant_rows(ctx, hidden, T, C_in, C_in, b.q1, b.ld, b.s1, b.z1, nullptr,
                                     b.q2, b.s2, b.z2, true, snake);
    if (rc) return rc;
    GemmArgs a = gemm_args(b, T, C_in);
    a.bias = bias;
    a.y = output;
    a.yin = skip;
    a.ldy = C_out;
    a.accumulate = 1;
    return launch_gemm(ctx, w, a, EPI_LINEAR);
}

}  // namespace

bool snake_rows_ok(const float *x, int C, const float *y) {
    return C % 4 == 0 && C <= kSnakeMaxChannels && ((((uintptr_t)x) | ((uintptr_t)y)) & 15) == 0;
}

int launch_snake_rows(IroHipContext *ctx, const float *x, int T, int C, const float *alpha,
                      float *y, float *row_lo, float *row_hi) {
    if (T <= 0) return 0;
    if (!snake_rows_ok(x, C, y)) return set_error(ctx, "snake_rows: unsupported shape");
    const int R = 4096 / C;
    const unsigned k4 = (unsigned)C / 4;
    // floor(f / k4) == umulhi(2 f, ceil(2^31 / k4)) for the chunk indices
    // f < 1024 used: the rounding adds less than 2^11 / 2^32 < 1 / k4.
    const unsigned magic = (unsigned)((0x80000000ull + k4 - 1) / k4);
    const size_t lds = sizeof(float) * ((size_t)2 * C + (size_t)R * C);
    const dim3 grid((unsigned)((T + R - 1) / R)), block(256);
    prof_begin(ctx);
    if (ctx->convention == IRO_HIP_GCC_FASTMATH)
        hipLaunchKernelGGL((snake_rows_kernel<true>), grid, block, lds, ctx->stream, x, T, C, R,
                           magic, alpha, y, row_lo, row_hi);
    else
        hipLaunchKernelGGL((snake_rows_kernel<false>), grid, block, lds, ctx->stream, x, T, C, R,
                           magic, alpha, y, row_lo, row_hi);
    IRO_HIP_CHECK_LAUNCH(ctx);
    // Algorithmic HBM bytes: the rows in and out, two floats per row.
    prof_end(ctx, PK_SNAKE, 0, 8.0 * T * C + 8.0 * T);
    return 0;
}

namespace {

// The groups of the codec's int8 policy (dacvae.c:38-43).
enum { GROUP_INITIAL = 1, GROUP_UPSAMPLE = 2, GROUP_CONV7 = 4, GROUP_CONV1 = 8 };

// run_residual_int8 (dacvae.c:934-1018) with caller-provided [T, C] scratch
// `act` and `hidden`: the convolutions use the context's inner workspace.
int residual_unit(IroHipContext *ctx, const float *input, int T, int C, const IroHipWeight *conv0,
                  const float *alpha0, const float *conv0_bias, const float *alpha1, int dilation,
                  const IroHipWeight *conv1, const float *conv1_bias, bool two7, bool two1,
                  float *act, float *hidden, float *output) {
    // dacvae.c:954-961 (conv1d_int8_forward with the snake of alpha0 on its
    // input rows, not in place, dacvae.c:599-603): Conv7, dilation d,
    // padding 3d, no bias.
    int t_out = 0;
    if (conv1d_int8(ctx, input, T, C, conv0, 7, 1, dilation, 3 * dilation, nullptr, two7, hidden,
                    &t_out, alpha0, act))
        return -1;
    if (t_out != T) return set_error(ctx, "dacvae residual: Conv7 changed the length");
    // dacvae.c:967-968: snake with conv0's bias and alpha1, in place, then
    // dacvae.c:983-1012: output = input, then += conv1(hidden) + bias.  Up to
    // 256 channels one kernel does all of it; else the in-place snake is the
    // 1x1 quantizer's pre-op where it takes the shape (its reciprocal form,
    // C <= 1536), else its own pass.
    if (conv0_bias && alpha1 && ctx->conv_mode == 2) {
        const int rc = launch_conv1x1_snake(ctx, conv1, hidden, T, conv0_bias, alpha1, two1,
                                            conv1_bias, input, output);
        if (rc <= 0) return rc;
    }
    if (conv0_bias && alpha1 && C <= kSnakeMaxChannels) {
        const SnakePre sp{conv0_bias, alpha1};
        const int rc = conv1x1_skip(ctx, hidden, input, T, conv1, conv1_bias, two1, output, &sp);
        if (rc <= 0) return rc;
    }
    if (iro_hip_snake_bias(ctx, hidden, T, C, conv0_bias, alpha1, hidden)) return -1;
    return conv1x1_skip(ctx, hidden, input, T, conv1, conv1_bias, two1, output, nullptr);
}

bool weight_is(const IroHipWeight *w, int N, int K) {
    int n = 0, k = 0;
    return w && iro_hip_weight_dims(w, &n, &k) == 0 && n == N && k == K;
}

}  // namespace
}  // namespace iro

using namespace iro;

// The decoder's int8 weights and the fp32 parameters its int8 core reads
// (IroDACVAEInt8, dacvae.h:53-67, beside the borrowed IroDACVAEDecoder).
struct IroHipDACVAE {
    IroHipContext *ctx = nullptr;
    IroHipDACVAEDecoderF32 f32{};
    IroHipWeight *initial = nullptr;
    IroHipWeight *upsample[IRO_HIP_DACVAE_STAGES] = {};
    IroHipWeight *conv0[IRO_HIP_DACVAE_STAGES][IRO_HIP_DACVAE_RESIDUALS] = {};
    IroHipWeight *conv1[IRO_HIP_DACVAE_STAGES][IRO_HIP_DACVAE_RESIDUALS] = {};
    size_t bytes = 0;
};

extern "C" {

int iro_hip_snake(IroHipContext *ctx, const float *x, int T, int C, const float *alpha,
                  float *y) {
    if (!ctx) return -1;
    if (!snake_args_ok(x, T, C, alpha, y))
        return set_error(ctx, "snake: invalid arguments (C %% 4 == 0, 16-byte aligned rows)");
    // iro_snake_forward (dacvae.c:830-857): the reciprocal form up to 1536
    // channels, in place or not.
    return launch_snake(ctx, x, T, C, nullptr, alpha, y, C <= kSnakeMaxChannels);
}

int iro_hip_conv1x1_skip_int8(IroHipContext *ctx, const float *hidden, const float *skip, int T,
                              const IroHipWeight *w, const float *bias, int residual,
                              float *output) {
    return conv1x1_skip(ctx, hidden, skip, T, w, bias, residual, output, nullptr);
}

int iro_hip_snake_bias(IroHipContext *ctx, const float *x, int T, int C, const float *bias,
                       const float *alpha, float *y) {
    if (!ctx) return -1;
    if (!bias || !snake_args_ok(x, T, C, alpha, y))
        return set_error(ctx, "snake_bias: invalid arguments (C %% 4 == 0, 16-byte aligned rows)");
    // snake_bias_forward (dacvae.c:910-931): the reciprocal form only in
    // place up to 1536 channels.
    return launch_snake(ctx, x, T, C, bias, alpha, y, C <= kSnakeMaxChannels && x == y);
}

int iro_hip_selfcheck_sincosf(IroHipContext *ctx, unsigned long long *sin_digest,
                              unsigned long long *cos_digest) {
    if (!ctx || !sin_digest || !cos_digest) return -1;
    Workspace ws{ctx};
    const size_t od = ws.reserve(2 * sizeof(unsigned long long));
    if (ws.commit()) return -1;
    unsigned long long *d = ws.at<unsigned long long>(od);
    if (launch_fill(ctx, d, 0, 2 * sizeof(unsigned long long))) return -1;
    for (unsigned long long base = 0; base < (1ull << 32); base += (1ull << 28)) {
        hipLaunchKernelGGL(sincosf_selfcheck_kernel, dim3(1u << 20), dim3(256), 0, ctx->stream, d,
                           (unsigned)base);
        IRO_HIP_CHECK_LAUNCH(ctx);
    }
    unsigned long long h[2] = {0, 0};
    IRO_HIP_TRY(ctx, hipMemcpyAsync(h, d, sizeof(h), hipMemcpyDeviceToHost, ctx->stream));
    IRO_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    *sin_digest = h[0];
    *cos_digest = h[1];
    return 0;
}

int iro_hip_dacvae_residual_int8(IroHipContext *ctx, const float *input, int T, int C,
                                 const IroHipWeight *conv0, const float *alpha0,
                                 const float *conv0_bias, const float *alpha1, int dilation,
                                 const IroHipWeight *conv1, const float *conv1_bias,
                                 int residual_conv7, int residual_conv1, float *output) {
    if (!ctx) return -1;
    if (!input || !alpha0 || !conv0_bias || !alpha1 || !conv1_bias || !output || T <= 0 ||
        C <= 0 || C % 4 || dilation <= 0 || output == input)
        return set_error(ctx, "dacvae_residual_int8: invalid arguments");
    if (!weight_is(conv0, C, 7 * C) || !weight_is(conv1, C, C))
        return set_error(ctx, "dacvae_residual_int8: weights must be [C, 7C] and [C, C]");
    // act and hidden live in the outer workspace: the convolutions grow
    // and use the inner one.
    Workspace ws{ctx, 1};
    const size_t n = (size_t)T * C;
    const size_t oa = ws.reserve(sizeof(float) * n), oh = ws.reserve(sizeof(float) * n);
    if (ws.commit()) return -1;
    return residual_unit(ctx, input, T, C, conv0, alpha0, conv0_bias, alpha1, dilation, conv1,
                         conv1_bias, residual_conv7 != 0, residual_conv1 != 0, ws.at<float>(oa),
                         ws.at<float>(oh), output);
}

void iro_hip_dacvae_destroy(IroHipDACVAE *d) {
    if (!d) return;
    iro_hip_weight_destroy(d->initial);
    for (int s = 0; s < IRO_HIP_DACVAE_STAGES; ++s) {
        iro_hip_weight_destroy(d->upsample[s]);
        for (int r = 0; r < IRO_HIP_DACVAE_RESIDUALS; ++r) {
            iro_hip_weight_destroy(d->conv0[s][r]);
            iro_hip_weight_destroy(d->conv1[s][r]);
        }
    }
    delete d;
}

int iro_hip_dacvae_create(IroHipContext *ctx, const IroHipDACVAEDecoderF32 *p,
                          IroHipDACVAE **out) {
    if (!ctx) return -1;
    if (!p || !out || !p->initial_weight || !p->initial_bias || p->latent_channels <= 0 ||
        p->channels <= 0 || p->channels % 4)
        return set_error(ctx, "dacvae_create: invalid arguments");
    *out = nullptr;
    int c_in = p->channels;
    for (int s = 0; s < IRO_HIP_DACVAE_STAGES; ++s) {
        const IroHipDACVAEStageF32 &st = p->stage[s];
        bool ok = st.alpha && st.up_weight && st.up_bias && st.c_in == c_in && st.c_out > 0 &&
                  st.c_out % 4 == 0 && st.kernel > 0 && st.stride > 0 && st.padding >= 0 &&
                  st.output_padding >= 0;
        for (int r = 0; ok && r < IRO_HIP_DACVAE_RESIDUALS; ++r) {
            const IroHipDACVAEResidualF32 &u = st.residual[r];
            ok = u.alpha0 && u.conv0_weight && u.conv0_bias && u.alpha1 && u.conv1_weight &&
                 u.conv1_bias && u.dilation > 0;
        }
        if (!ok)
            return set_error(ctx, "dacvae_create: stage %d is incomplete or its channels do not "
                                  "chain", s);
        c_in = st.c_out;
    }
    IroHipDACVAE *d = new (std::nothrow) IroHipDACVAE();
    if (!d) return set_error(ctx, "dacvae_create: out of host memory");
    d->ctx = ctx;
    d->f32 = *p;
    // dacvae.c:232-262: the initial conv [out, 7, in] read as [out, 7 in];
    // each upsample [in, kernel, out] read as the transpose of
    // [kernel out, in]; conv0 [C, 7, C] as [C, 7C]; conv1 [C, 1, C] as [C, C].
    int rc = iro_hip_weight_create(ctx, p->initial_weight, p->channels, 7 * p->latent_channels,
                                   &d->initial);
    for (int s = 0; !rc && s < IRO_HIP_DACVAE_STAGES; ++s) {
        const IroHipDACVAEStageF32 &st = p->stage[s];
        rc = iro_hip_weight_create_transposed(ctx, st.up_weight, st.kernel * st.c_out, st.c_in,
                                              &d->upsample[s]);
        for (int r = 0; !rc && r < IRO_HIP_DACVAE_RESIDUALS; ++r) {
            const IroHipDACVAEResidualF32 &u = st.residual[r];
            rc = iro_hip_weight_create(ctx, u.conv0_weight, st.c_out, 7 * st.c_out,
                                       &d->conv0[s][r]);
            if (!rc)
                rc = iro_hip_weight_create(ctx, u.conv1_weight, st.c_out, st.c_out,
                                           &d->conv1[s][r]);
        }
    }
    if (rc) {
        iro_hip_dacvae_destroy(d);
        return -1;
    }
    d->bytes = iro_hip_weight_bytes(d->initial);
    for (int s = 0; s < IRO_HIP_DACVAE_STAGES; ++s) {
        d->bytes += iro_hip_weight_bytes(d->upsample[s]);
        for (int r = 0; r < IRO_HIP_DACVAE_RESIDUALS; ++r)
            d->bytes += iro_hip_weight_bytes(d->conv0[s][r]) + iro_hip_weight_bytes(d->conv1[s][r]);
    }
    *out = d;
    return 0;
}

size_t iro_hip_dacvae_int8_bytes(const IroHipDACVAE *d) { return d ? d->bytes : 0; }

int iro_hip_dacvae_output_frames(const IroHipDACVAE *d, int frames) {
    if (!d || frames <= 0) return -1;
    long long t = frames;  // the initial conv keeps the length (kernel 7, padding 3)
    for (int s = 0; s < IRO_HIP_DACVAE_STAGES; ++s) {
        const IroHipDACVAEStageF32 &st = d->f32.stage[s];
        // dacvae.c:350-358
        t = (t - 1) * st.stride - 2ll * st.padding + st.kernel + st.output_padding;
        if (t <= 0 || t > 0x7fffffffll) return -1;
    }
    return (int)t;
}

int iro_hip_dacvae_decode_int8(IroHipDACVAE *d, const float *state, int frames,
                               int residual_mask, int residual_stages, float *out) {
    if (!d) return -1;
    IroHipContext *ctx = d->ctx;
    if (!state || !out || frames <= 0)
        return set_error(ctx, "dacvae_decode_int8: invalid arguments");
    if (iro_hip_dacvae_output_frames(d, frames) <= 0)
        return set_error(ctx, "dacvae_decode_int8: output length out of range");
    // Four [T, C] buffers of the largest state: two that alternate as the
    // state, and the residual unit's act and hidden (act also holds the
    // snake'd stage input).
    size_t most = (size_t)frames * d->f32.channels;
    long long t = frames;
    for (int s = 0; s < IRO_HIP_DACVAE_STAGES; ++s) {
        const IroHipDACVAEStageF32 &st = d->f32.stage[s];
        t = (t - 1) * st.stride - 2ll * st.padding + st.kernel + st.output_padding;
        most = std::max(most, (size_t)t * st.c_out);
    }
    Workspace ws{ctx, 1};
    size_t off[4];
    for (size_t &o : off) o = ws.reserve(sizeof(float) * most);
    if (ws.commit()) return -1;
    float *cur = ws.at<float>(off[0]), *spare = ws.at<float>(off[1]);
    float *act = ws.at<float>(off[2]), *hidden = ws.at<float>(off[3]);
    // dacvae.c:1228-1237: the initial Conv7 (padding 3) with its bias.
    int tt = 0;
    if (iro_hip_conv1d_int8(ctx, state, frames, d->f32.latent_channels, d->initial, 7, 1, 1, 3,
                            d->f32.initial_bias, (residual_mask & GROUP_INITIAL) != 0, cur, &tt))
        return -1;
    for (int s = 0; s < IRO_HIP_DACVAE_STAGES; ++s) {
        const IroHipDACVAEStageF32 &st = d->f32.stage[s];
        // dacvae.c:1255-1264 (convtranspose1d_forward_impl, dacvae.c:736-748):
        // snake(alpha) on the input rows (inside the upsample's row quantizer,
        // so the snaked rows never reach HBM), then the int8 upsample with its
        // bias.
        int t_up = 0;
        if (convtranspose1d_int8(ctx, cur, tt, st.c_in, d->upsample[s], st.c_out, st.kernel,
                                 st.stride, st.padding, st.output_padding, st.up_bias,
                                 (residual_mask & GROUP_UPSAMPLE) != 0, spare, &t_up, st.alpha,
                                 act))
            return -1;
        tt = t_up;
        std::swap(cur, spare);
        // dacvae.c:1268-1277: three residual units; the second activation
        // plane of Conv7 / Conv1 only in the stages of residual_stages.
        const bool stage_on = (residual_stages >> s & 1) != 0;
        const bool two7 = (residual_mask & GROUP_CONV7) && stage_on;
        const bool two1 = (residual_mask & GROUP_CONV1) && stage_on;
        for (int r = 0; r < IRO_HIP_DACVAE_RESIDUALS; ++r) {
            const IroHipDACVAEResidualF32 &u = st.residual[r];
            const bool final_unit = s == IRO_HIP_DACVAE_STAGES - 1 && r == IRO_HIP_DACVAE_RESIDUALS - 1;
            float *dst = final_unit ? out : spare;
            if (residual_unit(ctx, cur, tt, st.c_out, d->conv0[s][r], u.alpha0, u.conv0_bias,
                              u.alpha1, u.dilation, d->conv1[s][r], u.conv1_bias, two7, two1, act,
                              hidden, dst))
                return -1;
            if (!final_unit) std::swap(cur, spare);
        }
    }
    return ctx->has_err ? -1 : 0;
}

}  // extern "C"
