// iro_engine.hip -- the fp32 elementwise pieces around the int8 linears that
// let a whole step stay on the device: the timestep conditioner
// (iro_dit_condition, dit.c:488-530), the SiLU forms of ops.c:776-784 and
// the gated residual of a block (dit.c:1013-1020, 1032-1039), used where the
// int8 group mask (IRO_INT8_MASK, dit.c:273-291) runs a group in fp32.
// All are HBM-bound elementwise kernels: one pass over their rows.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "iro_hip.h"
#include "iro_internal.h"
#include "iro_gemm_core.h"
#include "iro_sincosf.h"

namespace iro {
namespace {

// ops.c:776-784 on the device with glibc's expf: x / (1 + expf(-x)), times
// g when G; silu_div gives the correctly rounded quotient.
template <bool G>
__global__ __launch_bounds__(256) void silu_kernel(float *__restrict__ x,
                                                   const float *__restrict__ g, long long n) {
    __shared__ uint64_t tab[32];
    if (threadIdx.x < 32) tab[threadIdx.x] = kExp2Tab[threadIdx.x];
    __syncthreads();
    for (long long i = blockIdx.x * 256ll + threadIdx.x; i < n; i += (long long)gridDim.x * 256) {
        const float a = x[i];
        const float s = silu_div(a, 1.0f + expf_glibc(-a, tab));
        x[i] = G ? s * g[i] : s;
    }
}

// x[m][d] += gate[m / S][d] * branch[m][d]: the strict build rounds the
// product and the sum, the fast build contracts them into one fma.
template <int CONV>
__global__ __launch_bounds__(256) void gated_residual_kernel(float *__restrict__ x,
                                                             const float *__restrict__ gate,
                                                             int ldg,
                                                             const float *__restrict__ branch,
                                                             long long n, int D, int S) {
    for (long long i = blockIdx.x * 256ll + threadIdx.x; i < n; i += (long long)gridDim.x * 256) {
        const long long m = i / D;
        const int d = (int)(i - m * D);
        const float gv = gate[(m / S) * ldg + d];
        const float y = branch[i];
        x[i] = CONV == 1 ? __builtin_fmaf(gv, y, x[i]) : x[i] + gv * y;
    }
}

// dit.c:488-499: row b of the embedding is cos(t_b f_i) for i < half, then
// sin(t_b f_i), f_i = 1000 expf(-log(10000) i / half).
__global__ __launch_bounds__(256) void timestep_embedding_kernel(const float *__restrict__ t,
                                                                 int B, int half,
                                                                 float log_theta,
                                                                 float *__restrict__ emb) {
    __shared__ uint64_t tab[32];
    if (threadIdx.x < 32) tab[threadIdx.x] = kExp2Tab[threadIdx.x];
    __syncthreads();
    const int n = B * half;
    for (int e = blockIdx.x * 256 + threadIdx.x; e < n; e += gridDim.x * 256) {
        const int b = e / half, i = e - b * half;
        const float freq = 1000.0f * expf_glibc(-log_theta * (float)i / (float)half, tab);
        const float arg = t[b] * freq;
        emb[(size_t)b * 2 * half + i] = cosf_glibc(arg);
        emb[(size_t)b * 2 * half + half + i] = sinf_glibc(arg);
    }
}

unsigned grid_for(long long n) {
    const long long g = (n + 255) / 256;
    return (unsigned)(g < 1 ? 1 : g > 4096 ? 4096 : g);
}

}  // namespace

int launch_silu(IroHipContext *ctx, float *x, const float *g, long long n) {
    if (n <= 0) return 0;
    if (g)
        hipLaunchKernelGGL(silu_kernel<true>, dim3(grid_for(n)), dim3(256), 0, ctx->stream, x, g, n);
    else
        hipLaunchKernelGGL(silu_kernel<false>, dim3(grid_for(n)), dim3(256), 0, ctx->stream, x,
                           nullptr, n);
    IRO_HIP_CHECK_LAUNCH(ctx);
    return 0;
}

int launch_gated_residual(IroHipContext *ctx, float *x, const float *gate, int ldg,
                          const float *branch, int M, int D, int S) {
    const long long n = (long long)M * D;
    if (n <= 0) return 0;
    if (ctx->convention == IRO_HIP_GCC_FASTMATH)
        hipLaunchKernelGGL(gated_residual_kernel<1>, dim3(grid_for(n)), dim3(256), 0, ctx->stream,
                           x, gate, ldg, branch, n, D, S);
    else
        hipLaunchKernelGGL(gated_residual_kernel<0>, dim3(grid_for(n)), dim3(256), 0, ctx->stream,
                           x, gate, ldg, branch, n, D, S);
    IRO_HIP_CHECK_LAUNCH(ctx);
    return 0;
}

}  // namespace iro

using namespace iro;

extern "C" {

int iro_hip_silu(IroHipContext *ctx, float *x, const float *gate, long long n) {
    if (!ctx) return -1;
    if (n < 0 || (n && !x)) return set_error(ctx, "silu: invalid arguments");
    return launch_silu(ctx, x, gate, n);
}

int iro_hip_gated_residual(IroHipContext *ctx, float *x, const float *gate, int ldg,
                           const float *branch, int M, int D, int S) {
    if (!ctx) return -1;
    if (M < 0 || D <= 0 || S <= 0 || ldg < D || (M && (!x || !gate || !branch)))
        return set_error(ctx, "gated_residual: invalid arguments");
    return launch_gated_residual(ctx, x, gate, ldg, branch, M, D, S);
}

int iro_hip_dit_condition(IroHipContext *ctx, const float *t, int B, const float *w0,
                          const float *w1, const float *w2, int tdim, int D, int cond_dim,
                          float *cond) {
    if (!ctx) return -1;
    if (!t || B <= 0 || !w0 || !w1 || !w2 || tdim <= 0 || tdim % 2 || D <= 0 || cond_dim <= 0 ||
        !cond)
        return set_error(ctx, "dit_condition: invalid arguments");
    Workspace ws{ctx};
    const size_t oe = ws.reserve(sizeof(float) * (size_t)B * tdim);
    const size_t o0 = ws.reserve(sizeof(float) * (size_t)B * D);
    const size_t o1 = ws.reserve(sizeof(float) * (size_t)B * D);
    if (ws.commit()) return -1;
    float *emb = ws.at<float>(oe), *h0 = ws.at<float>(o0), *h1 = ws.at<float>(o1);
    const int half = tdim / 2;
    // logf(10000.0f), which GCC folds to the correctly rounded constant.
    constexpr float kLogTheta = 0x1.26bb1cp+3f;
    hipLaunchKernelGGL(timestep_embedding_kernel, dim3(grid_for((long long)B * half)), dim3(256),
                       0, ctx->stream, t, B, half, kLogTheta, emb);
    IRO_HIP_CHECK_LAUNCH(ctx);
    // dit.c:519-524: three linears without bias, SiLU after the first two.
    if (iro_hip_linear_f32(ctx, emb, B, tdim, w0, D, nullptr, h0) ||
        launch_silu(ctx, h0, nullptr, (long long)B * D) ||
        iro_hip_linear_f32(ctx, h0, B, D, w1, D, nullptr, h1) ||
        launch_silu(ctx, h1, nullptr, (long long)B * D) ||
        iro_hip_linear_f32(ctx, h1, B, D, w2, cond_dim, nullptr, cond))
        return -1;
    return 0;
}

}  // extern "C"
