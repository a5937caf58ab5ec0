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
    hipLaunchKernelGGL(linear_f32_kernel, dim3((N + kLN - 1) / kLN, (M + kLM - 1) / kLM),
                       dim3(256), 0, ctx->stream, x, M, K, w, N, bias, y);
    IRO_HIP_CHECK_LAUNCH(ctx);
    return 0;
}

}  // extern "C"
