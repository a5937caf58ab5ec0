// iro_f32.hip -- the fp32 linear of the reference's scalar build on gfx950
// (ops.c:221-234 iro_linear_scalar): y[m][n] = (sum_k x[m][k] w[n][k] in
// index order, each product rounded) + bias[n] (+ 0 without bias).  Used by
// the DiT's input and output projections and the context key/value
// projections (dit.c:532-540, 708-735, 1070-1089).
//
// Block tile: 64 rows x 128 outputs; K passes through LDS 64 at a time; a
// thread owns 4 rows x 8 outputs (32 chains).  K is zero-padded to a multiple
// of 64: a chain starts at +0 and never holds -0 (a sum is -0 only when both
// terms are), so adding +0 * +0 leaves every chain's bits unchanged.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "iro_hip.h"
#include "iro_internal.h"

namespace iro {
namespace {

constexpr int kLM = 64, kLN = 128, kLK = 64, kLP = 68;

__global__ __launch_bounds__(256) void linear_f32_kernel(const float *__restrict__ x, int M,
                                                         int K, const float *__restrict__ w, int N,
                                                         const float *__restrict__ bias,
                                                         float *__restrict__ y) {
    __shared__ __attribute__((aligned(16))) float Xs[kLM * kLP];
    __shared__ __attribute__((aligned(16))) float Ws[kLN * kLP];
    const int tid = threadIdx.x;
    const int m0 = blockIdx.y * kLM, n0 = blockIdx.x * kLN;
    const int tm = tid >> 4, tn = tid & 15;  // rows 4 tm .. +3, outputs tn + 16 j
    float acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += kLK) {
        // Scalar staging (any K, any alignment): element (r, c) of the tile.
        for (int e = tid; e < kLM * kLK; e += 256) {
            const int r = e / kLK, c = e - r * kLK;
            const int m = m0 + r < M ? m0 + r : M - 1;
            Xs[r * kLP + c] = k0 + c < K ? x[(size_t)m * K + k0 + c] : 0.0f;
        }
        for (int e = tid; e < kLN * kLK; e += 256) {
            const int r = e / kLK, c = e - r * kLK;
            const int n = n0 + r < N ? n0 + r : N - 1;
            Ws[r * kLP + c] = k0 + c < K ? w[(size_t)n * K + k0 + c] : 0.0f;
        }
        __syncthreads();
#pragma unroll 4
        for (int c4 = 0; c4 < kLK / 4; ++c4) {
            float4 xv[4], wv[8];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                xv[i] = *reinterpret_cast<const float4 *>(&Xs[(tm * 4 + i) * kLP + c4 * 4]);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                wv[j] = *reinterpret_cast<const float4 *>(&Ws[(tn + 16 * j) * kLP + c4 * 4]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    acc[i][j] = acc[i][j] + xv[i].x * wv[j].x;
                    acc[i][j] = acc[i][j] + xv[i].y * wv[j].y;
                    acc[i][j] = acc[i][j] + xv[i].z * wv[j].z;
                    acc[i][j] = acc[i][j] + xv[i].w * wv[j].w;
                }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + tm * 4 + i;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int n = n0 + tn + 16 * j;
            if (n < N) y[(size_t)m * N + n] = acc[i][j] + (bias ? bias[n] : 0.0f);
        }
    }
}

// Narrow outputs (N <= 32: the output head's 1280 -> 32 projection): a
// block is 8 rows x 32 outputs, one K-order chain per thread, so the grid
// has a block per 8 rows instead of one 64 x 128 tile per 64 rows of which
// three quarters would be padding.  x and w pass through LDS in 64-k
// chunks, the next chunk's loads in flight while one is summed; only k < K
// enters a chain, as in the reference loop.
constexpr int kNR = 8, kNK = 64, kNP = 65;

__global__ __launch_bounds__(256) void linear_f32_narrow_kernel(const float *__restrict__ x,
                                                                int M, int K,
                                                                const float *__restrict__ w,
                                                                int N,
                                                                const float *__restrict__ bias,
                                                                float *__restrict__ y) {
    __shared__ float Xs[kNR * kNP];
    __shared__ float Ws[32 * kNP];
    const int tid = threadIdx.x, r = tid >> 5, n = tid & 31;
    const int m0 = blockIdx.x * kNR;
    // Staging: x element tid + 256 i (i < 2) and w element tid + 256 i
    // (i < 8) of a chunk, row e / 64, column e % 64.
    float xr[2], wr[8];
    auto load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int e = tid + 256 * i, rr = e >> 6, c = e & 63;
            const int m = m0 + rr < M ? m0 + rr : M - 1;
            xr[i] = k0 + c < K ? x[(size_t)m * K + k0 + c] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = tid + 256 * i, rr = e >> 6, c = e & 63;
            const int nn = rr < N ? rr : N - 1;
            wr[i] = k0 + c < K ? w[(size_t)nn * K + k0 + c] : 0.0f;
        }
    };
    float acc = 0.0f;
    load(0);
    for (int k0 = 0; k0 < K; k0 += kNK) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int e = tid + 256 * i;
            Xs[(e >> 6) * kNP + (e & 63)] = xr[i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = tid + 256 * i;
            Ws[(e >> 6) * kNP + (e & 63)] = wr[i];
        }
        __syncthreads();
        if (k0 + kNK < K) load(k0 + kNK);
        const float *xs = &Xs[r * kNP], *ws = &Ws[n * kNP];
        if (K - k0 >= kNK) {
#pragma unroll 16
            for (int c = 0; c < kNK; ++c) acc = acc + xs[c] * ws[c];
        } else {
            for (int c = 0; c < K - k0; ++c) acc = acc + xs[c] * ws[c];
        }
        __syncthreads();
    }
    const int m = m0 + r;
    if (m < M && n < N) y[(size_t)m * N + n] = acc + (bias ? bias[n] : 0.0f);
}

// sampler.c:281-297, the CFG combine and Euler update after the DiT
// velocity of a step: guided = v + sum_k s_k * (v - v_k) over the active
// unconditional rows k (text, speaker, caption order), state += guided * dt.
// The strict build rounds every op in source order (this file is compiled
// with -ffp-contract=off); the fast-math build's GCC reassociates the CFG
// sum and fuses the products (pinned against its traces): 1 term
// fma(s0, d0, v); 2 terms v + fma(s1, d1, s0 d0); 3 terms
// fma(s2, d2, v) + fma(s1, d1, s0 d0); then state = fma(guided, dt, state).
struct EulerTerms {
    int n;                // active terms, 0..3
    int off[3];           // element offset of each term's row: row * len
    float s[3];
};

template <int CONV>
__global__ __launch_bounds__(256) void euler_update_kernel(float *__restrict__ state,
                                                           const float *__restrict__ vel,
                                                           long long len, EulerTerms t, float dt) {
    const long long stride = (long long)gridDim.x * 256;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < len; i += stride) {
        const float v = vel[i];
        float d[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < 3; ++k)
            if (k < t.n) d[k] = v - vel[t.off[k] + i];
        float g = v;
        if (CONV == 0) {
#pragma unroll
            for (int k = 0; k < 3; ++k)
                if (k < t.n) g = g + t.s[k] * d[k];
            state[i] = state[i] + g * dt;
        } else {
            if (t.n == 1)
                g = __builtin_fmaf(t.s[0], d[0], v);
            else if (t.n == 2)
                g = v + __builtin_fmaf(t.s[1], d[1], t.s[0] * d[0]);
            else if (t.n == 3)
                g = __builtin_fmaf(t.s[2], d[2], v) + __builtin_fmaf(t.s[1], d[1], t.s[0] * d[0]);
            state[i] = __builtin_fmaf(g, dt, state[i]);
        }
    }
}

}  // namespace
}  // namespace iro

using namespace iro;

extern "C" {

int iro_hip_linear_f32(IroHipContext *ctx, const float *x, int M, int K, const float *w, int N,
                       const float *bias, float *y) {
    if (!ctx || M < 0 || K <= 0 || N <= 0 || (M && (!x || !w || !y)))
        return set_error(ctx, "linear_f32: invalid arguments");
    if (M == 0) return 0;
    if ((long long)M * K > INT64_MAX / 8 || (M + kLM - 1) / kLM > 65535)
        return set_error(ctx, "linear_f32: too many rows");
    if (N <= 32 && K >= 128) {
        if ((M + kNR - 1) / kNR > INT32_MAX / 2) return set_error(ctx, "linear_f32: too many rows");
        hipLaunchKernelGGL(linear_f32_narrow_kernel, dim3((M + kNR - 1) / kNR), dim3(256), 0,
                           ctx->stream, x, M, K, w, N, bias, y);
    } else {
        hipLaunchKernelGGL(linear_f32_kernel, dim3((N + kLN - 1) / kLN, (M + kLM - 1) / kLM),
                           dim3(256), 0, ctx->stream, x, M, K, w, N, bias, y);
    }
    IRO_HIP_CHECK_LAUNCH(ctx);
    return 0;
}

int iro_hip_euler_update(IroHipContext *ctx, float *state, const float *velocity, int len,
                         int batch, int use_cfg, int text_row, int speaker_row, int caption_row,
                         float scale_text, float scale_speaker, float scale_caption, float dt) {
    if (!ctx || len < 0 || batch < 1 || batch > 4 || (len && (!state || !velocity)))
        return set_error(ctx, "euler_update: invalid arguments");
    const int rows[3] = {text_row, speaker_row, caption_row};
    const float scales[3] = {scale_text, scale_speaker, scale_caption};
    EulerTerms t{};
    for (int k = 0; k < 3; ++k) {
        // Rows index the velocity only on CFG steps; a plain step (batch 1)
        // keeps the sampler's row numbers unused.
        if (rows[k] < -1 || rows[k] == 0 || rows[k] > 3 || (use_cfg && rows[k] >= batch))
            return set_error(ctx, "euler_update: CFG row %d outside 1..%d", rows[k],
                             use_cfg ? batch - 1 : 3);
        if (use_cfg && rows[k] > 0) {
            t.off[t.n] = rows[k] * len;
            t.s[t.n] = scales[k];
            ++t.n;
        }
    }
    if ((long long)batch * len > INT32_MAX) return set_error(ctx, "euler_update: too many values");
    if (len == 0) return 0;
    const unsigned grid = (unsigned)((len + 255) / 256 < 1024 ? (len + 255) / 256 : 1024);
    if (ctx->convention == IRO_HIP_GCC_FASTMATH)
        hipLaunchKernelGGL(euler_update_kernel<1>, dim3(grid), dim3(256), 0, ctx->stream, state,
                           velocity, (long long)len, t, dt);
    else
        hipLaunchKernelGGL(euler_update_kernel<0>, dim3(grid), dim3(256), 0, ctx->stream, state,
                           velocity, (long long)len, t, dt);
    IRO_HIP_CHECK_LAUNCH(ctx);
    return 0;
}

}  // extern "C"
