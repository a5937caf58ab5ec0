// iro_attn.hip -- the fp32 attention core of a DiT block on gfx950, as the
// reference's scalar build computes it (dit.c:808-870 with ops.c:577-600,
// 681-703, 754-766, 786-789).
//
// Every sum runs in the scalar build's order, so the result is bit-identical
// to it: a score is a 64-term dot product in index order, times 1/sqrtf(64);
// a softmax row takes its maximum by strict replacement from the first score,
// p = expf(score - max) (glibc's expf), the sum of p in key order, and p / sum;
// each output element is the sum over keys, in key order, of p * v; the mix
// is then scaled by 1 / (1 + expf(-gate)).  The joined keys of batch b are its
// S latent tokens, then the context rows its mask keeps, in order.
//
// Three kernels per call:
//   attn_scores   64 queries x 128 keys per block, 32 dot-product chains per
//                 thread from LDS tiles; scores to a workspace [B*H, S, Jp],
//                 and the maximum of each row's 128-key tile
//   attn_softmax  RW rows per wave: the row maximum from the tile maxima,
//                 p = expf(score - max) written in place, the key-order sum
//                 of p by one lane per row (through LDS)
//   attn_pv       64 (or, for small grids, 32) queries x 64 dims per block:
//                 p / sum staged per 64-key chunk, 16 (8) key-order chains
//                 per thread, the gate applied at the store
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <new>
#include <vector>

#include "iro_expf.h"
#include "iro_hip.h"
#include "iro_internal.h"


namespace iro {
namespace {

constexpr int kQT = 64;     // queries per score block
constexpr int kKT = 128;    // keys per score block
constexpr int kPitch = 68;  // LDS row pitch (floats) of 64-wide tiles
constexpr int kPVK = 64;    // keys per PV chunk

// The source of joined key j < S + nvalid[b] of batch b, head column h*64.
// Branch-free, so the callers' row loads are not split by a divergent branch
// (which made the compiler wait for and spill each one): both candidate
// rows are formed and one selected, and the context row index is read at a
// clamped position that is always inside rows[b*C .. b*C + C) (C >= 1 and
// j - S < nvalid[b] <= C).
__device__ __forceinline__ const float *key_row(const float *self, const float *ctxr,
                                                const int *rows, int b, int S, int C, int D,
                                                int j) {
    const int jc = j - S;
    const int r = rows[b * C + (jc > 0 ? jc : 0)];
    const float *ps = self + ((size_t)b * S + (j < S ? j : 0)) * D;
    const float *pc = ctxr + (size_t)r * D;
    return j < S ? ps : pc;
}

__global__ __launch_bounds__(256) void attn_scores_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ ck,
    const int *__restrict__ rows, const int *__restrict__ nvalid, int S, int D, int H, int C,
    int Jp, float *__restrict__ sc, float *__restrict__ pmax) {
    __shared__ __attribute__((aligned(16))) float Qs[kQT * kPitch];
    __shared__ __attribute__((aligned(16))) float Ks[kKT * kPitch];
    const int bh = blockIdx.z, b = bh / H, h = bh - b * H;
    const int J = S + nvalid[b];
    const int k0 = blockIdx.x * kKT;
    if (k0 >= J) return;
    const int q0 = blockIdx.y * kQT;
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int idx = tid + 256 * i, r = idx >> 4, c4 = (idx & 15) * 4;
        const int s = q0 + r < S ? q0 + r : S - 1;
        *reinterpret_cast<float4 *>(&Qs[r * kPitch + c4]) =
            *reinterpret_cast<const float4 *>(q + ((size_t)b * S + s) * D + h * 64 + c4);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int idx = tid + 256 * i, r = idx >> 4, c4 = (idx & 15) * 4;
        const int j = k0 + r < J ? k0 + r : J - 1;
        *reinterpret_cast<float4 *>(&Ks[r * kPitch + c4]) = *reinterpret_cast<const float4 *>(
            key_row(k, ck, rows, b, S, C, D, j) + h * 64 + c4);
    }
    __syncthreads();
    // Thread: queries 4 tq .. 4 tq + 3, keys tk + 16 jj (jj < 8).
    const int tq = tid >> 4, tk = tid & 15;
    float acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) acc[i][jj] = 0.0f;
#pragma unroll 4
    for (int d4 = 0; d4 < 16; ++d4) {
        float4 qv[4], kv[8];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            qv[i] = *reinterpret_cast<const float4 *>(&Qs[(tq * 4 + i) * kPitch + d4 * 4]);
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
            kv[jj] = *reinterpret_cast<const float4 *>(&Ks[(tk + 16 * jj) * kPitch + d4 * 4]);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                acc[i][jj] = acc[i][jj] + qv[i].x * kv[jj].x;
                acc[i][jj] = acc[i][jj] + qv[i].y * kv[jj].y;
                acc[i][jj] = acc[i][jj] + qv[i].z * kv[jj].z;
                acc[i][jj] = acc[i][jj] + qv[i].w * kv[jj].w;
            }
    }
    const int NKT = Jp / kKT;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int s = q0 + tq * 4 + i;
        float m = -__builtin_inff();
        float *dst = sc + ((size_t)bh * S + (s < S ? s : S - 1)) * Jp;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            const int j = k0 + tk + 16 * jj;
            const float v = acc[i][jj] * 0.125f;  // 1 / sqrtf(64)
            if (j < J) {
                m = __builtin_fmaxf(m, v);
                if (s < S) dst[j] = v;
            }
        }
        // Tile maximum over the 16 lanes of this query row (fmaxf ignores NaN;
        // the softmax kernel restores the first score's NaN rule).
        m = __builtin_fmaxf(m, __shfl_xor(m, 1));
        m = __builtin_fmaxf(m, __shfl_xor(m, 2));
        m = __builtin_fmaxf(m, __shfl_xor(m, 4));
        m = __builtin_fmaxf(m, __shfl_xor(m, 8));
        if (tk == 0 && s < S) pmax[((size_t)bh * S + s) * NKT + blockIdx.x] = m;
    }
}

// RW rows per wave, rows g = (b*H + h) * S + s.
template <int RW>
__global__ __launch_bounds__(64) void attn_softmax_kernel(float *__restrict__ sc,
                                                          const float *__restrict__ pmax,
                                                          const int *__restrict__ nvalid, int R,
                                                          int S, int H, int Jp,
                                                          float *__restrict__ sums) {
    __shared__ uint64_t exptab[32];
    __shared__ float tile[RW * 65];
    __shared__ float mx_s[RW];
    __shared__ int J_s[RW];
    const int lane = threadIdx.x;
    if (lane < 32) exptab[lane] = kExp2Tab[lane];
    const int g0 = blockIdx.x * RW;
    const int NKT = Jp / kKT;
    int Jl = 0;
    if (lane < RW) {
        const int g = g0 + lane < R ? g0 + lane : R - 1;
        Jl = S + nvalid[(g / S) / H];
        // The scalar loop's maximum: the first score if it is NaN, else the
        // largest score (the tile maxima skip NaN; a zero's sign does not
        // change x - max for any x).
        float m = -__builtin_inff();
        for (int t = 0; t < (Jl + kKT - 1) / kKT; ++t)
            m = __builtin_fmaxf(m, pmax[(size_t)g * NKT + t]);
        const float x0 = sc[(size_t)g * Jp];
        mx_s[lane] = x0 != x0 ? x0 : m;
        J_s[lane] = g0 + lane < R ? Jl : 0;
    }
    __syncthreads();
    int Jw = 0;
#pragma unroll
    for (int r = 0; r < RW; ++r) Jw = J_s[r] > Jw ? J_s[r] : Jw;
    float sum = 0.0f;
    // Chunk c0's scores are loaded while chunk c0 - 64 is computed.
    float xn[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) xn[r] = lane < J_s[r] ? sc[(size_t)(g0 + r) * Jp + lane] : 0.0f;
    for (int c0 = 0; c0 < Jw; c0 += 64) {
        const int col = c0 + lane;
        float x[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) x[r] = xn[r];
        if (c0 + 64 < Jw) {
#pragma unroll
            for (int r = 0; r < RW; ++r)
                xn[r] = col + 64 < J_s[r] ? sc[(size_t)(g0 + r) * Jp + col + 64] : 0.0f;
        }
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            if (col < J_s[r]) {
                const float p = expf_glibc(x[r] - mx_s[r], exptab);
                sc[(size_t)(g0 + r) * Jp + col] = p;
                tile[r * 65 + lane] = p;
            }
        }
        __syncthreads();
        if (lane < RW) {
            const int n = Jl - c0 < 64 ? Jl - c0 : 64;
            const float *tr = &tile[lane * 65];
            for (int i = 0; i < n; ++i) sum = sum + tr[i];
        }
        __syncthreads();
    }
    if (lane < RW && g0 + lane < R) sums[g0 + lane] = sum;
}

// QT queries x 64 dims per block; thread: QT/16 queries x 4 dims (QT 32,
// 64 or 128).
template <int QT>
__global__ __launch_bounds__(256) void attn_pv_kernel(
    const float *__restrict__ sc, const float *__restrict__ sums, const float *__restrict__ v,
    const float *__restrict__ cv, const int *__restrict__ rows, const int *__restrict__ nvalid,
    const float *__restrict__ gate, int S, int D, int H, int C, int Jp,
    float *__restrict__ mix) {
    constexpr int QPT = QT / 16, PP = QT + 4, NP = QT / 4;
    __shared__ uint64_t exptab[32];
    __shared__ __attribute__((aligned(16))) float Ps[kPVK * PP];      // [key][query]
    __shared__ __attribute__((aligned(16))) float Vs[kPVK * kPitch];  // [key][dim]
    __shared__ float sum_s[QT];
    const int bh = blockIdx.y, b = bh / H, h = bh - b * H;
    const int J = S + nvalid[b];
    const int q0 = blockIdx.x * QT;
    const int tid = threadIdx.x;
    if (tid < 32) exptab[tid] = kExp2Tab[tid];
    if (tid < QT) {
        const int s = q0 + tid < S ? q0 + tid : S - 1;
        sum_s[tid] = sums[(size_t)bh * S + s];
    }
    // Staging: P element (query (tid >> 6) + 4 i, key tid & 63); V float4s
    // tid + 256 i of the chunk's 64 x 64 tile.
    const int kj = tid & 63, qi0 = tid >> 6;
    // The staged V rows are four named registers, not an array: as an array
    // held across the chunk loop the compiler kept them in scratch and waited
    // for each prefetch at once to store it there.
    float pr[NP];
    float4 vr0, vr1, vr2, vr3;
    auto vload = [&](int kc, int i) {
        const int idx = tid + 256 * i, r = idx >> 4, c4 = (idx & 15) * 4;
        const int jv = kc + r < J ? kc + r : J - 1;
        return *reinterpret_cast<const float4 *>(key_row(v, cv, rows, b, S, C, D, jv) + h * 64 +
                                                 c4);
    };
    auto load = [&](int kc) {
        const int j = kc + kj < J ? kc + kj : J - 1;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int s = q0 + qi0 + 4 * i < S ? q0 + qi0 + 4 * i : S - 1;
            pr[i] = sc[((size_t)bh * S + s) * Jp + j];
        }
        vr0 = vload(kc, 0);
        vr1 = vload(kc, 1);
        vr2 = vload(kc, 2);
        vr3 = vload(kc, 3);
    };
    const int tq = tid >> 4, tn = tid & 15;
    float acc[QPT][4];
#pragma unroll
    for (int i = 0; i < QPT; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[i][e] = 0.0f;
    load(0);
    __syncthreads();  // sum_s
    for (int kc = 0; kc < J; kc += kPVK) {
#pragma unroll
        for (int i = 0; i < NP; ++i) Ps[kj * PP + qi0 + 4 * i] = pr[i] / sum_s[qi0 + 4 * i];
        auto vstore = [&](int i, const float4 &x) {
            const int idx = tid + 256 * i, r = idx >> 4, c4 = (idx & 15) * 4;
            *reinterpret_cast<float4 *>(&Vs[r * kPitch + c4]) = x;
        };
        vstore(0, vr0);
        vstore(1, vr1);
        vstore(2, vr2);
        vstore(3, vr3);
        __syncthreads();
        if (kc + kPVK < J) load(kc + kPVK);
        auto step = [&](int kk) {
            float p[QPT];
            if constexpr (QPT % 4 == 0) {
#pragma unroll
                for (int c = 0; c < QPT; c += 4) {
                    const float4 pv =
                        *reinterpret_cast<const float4 *>(&Ps[kk * PP + tq * QPT + c]);
                    p[c] = pv.x, p[c + 1] = pv.y, p[c + 2] = pv.z, p[c + 3] = pv.w;
                }
            } else {
                const float2 pv = *reinterpret_cast<const float2 *>(&Ps[kk * PP + tq * 2]);
                p[0] = pv.x, p[1] = pv.y;
            }
            const float4 vv = *reinterpret_cast<const float4 *>(&Vs[kk * kPitch + tn * 4]);
#pragma unroll
            for (int i = 0; i < QPT; ++i) {
                acc[i][0] = acc[i][0] + p[i] * vv.x;
                acc[i][1] = acc[i][1] + p[i] * vv.y;
                acc[i][2] = acc[i][2] + p[i] * vv.z;
                acc[i][3] = acc[i][3] + p[i] * vv.w;
            }
        };
        const int nk = J - kc < kPVK ? J - kc : kPVK;
        if (nk == kPVK) {
            // Full chunk: unrolled, so the LDS reads of later keys go out
            // ahead of the additions of earlier ones.
#pragma unroll 16
            for (int kk = 0; kk < kPVK; ++kk) step(kk);
        } else {
            for (int kk = 0; kk < nk; ++kk) step(kk);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
        const int s = q0 + tq * QPT + i;
        if (s >= S) continue;
        const size_t off = ((size_t)b * S + s) * D + h * 64 + tn * 4;
        const float4 g = *reinterpret_cast<const float4 *>(gate + off);
        const float g4[4] = {g.x, g.y, g.z, g.w};
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float r = 1.0f / (1.0f + expf_glibc(-g4[e], exptab));
            o[e] = acc[i][e] * r;
        }
        *reinterpret_cast<float4 *>(mix + off) = make_float4(o[0], o[1], o[2], o[3]);
    }
}

}  // namespace
}  // namespace iro

using namespace iro;

extern "C" {

int iro_hip_dit_attn_context_create(IroHipContext *ctx, const uint8_t *mask, int B, int C,
                                    int context_batch, IroHipAttnContext **out) {
    if (!ctx || !out || !mask || B <= 0 || C <= 0 || (context_batch != 1 && context_batch != B))
        return set_error(ctx, "dit_attn_context: invalid arguments");
    *out = nullptr;
    IroHipAttnContext *a = new (std::nothrow) IroHipAttnContext();
    if (!a) return set_error(ctx, "dit_attn_context: out of host memory");
    a->ctx = ctx;
    a->B = B;
    a->C = C;
    a->context_batch = context_batch;
    std::vector<int> rows((size_t)B * C, 0);
    a->nvalid_h.assign(B, 0);
    for (int b = 0; b < B; ++b) {
        const int crow = context_batch == 1 ? 0 : b * C;
        int n = 0;
        for (int ci = 0; ci < C; ++ci)
            if (mask[(size_t)b * C + ci]) rows[(size_t)b * C + n++] = crow + ci;
        a->nvalid_h[b] = n;
        a->max_valid = n > a->max_valid ? n : a->max_valid;
    }
    if (hipMalloc(&a->rows, rows.size() * sizeof(int)) != hipSuccess ||
        hipMalloc(&a->nvalid, (size_t)B * sizeof(int)) != hipSuccess ||
        hipMemcpyAsync(a->rows, rows.data(), rows.size() * sizeof(int), hipMemcpyHostToDevice,
                       ctx->stream) != hipSuccess ||
        hipMemcpyAsync(a->nvalid, a->nvalid_h.data(), (size_t)B * sizeof(int),
                       hipMemcpyHostToDevice, ctx->stream) != hipSuccess ||
        hipStreamSynchronize(ctx->stream) != hipSuccess) {
        iro_hip_dit_attn_context_destroy(a);
        return set_error(ctx, "dit_attn_context: device allocation or upload failed");
    }
    *out = a;
    return 0;
}

void iro_hip_dit_attn_context_destroy(IroHipAttnContext *a) {
    if (!a) return;
    if (a->ctx && a->ctx->stream) (void)hipStreamSynchronize(a->ctx->stream);
    if (a->rows) (void)hipFree(a->rows);
    if (a->nvalid) (void)hipFree(a->nvalid);
    delete a;
}

int iro_hip_dit_attention(IroHipContext *ctx, const IroHipAttnContext *a, const float *q,
                          const float *k, const float *v, const float *gate, int B, int S, int D,
                          const float *context_k, const float *context_v, float *mix) {
    // B may be below the context's batch: rows 0 .. B-1 of its mask are used,
    // as the sampler's plain steps (batch 1, sampler.c:247-249) read row 0
    // of the CFG mask.
    if (!ctx || !a || a->ctx != ctx || B < 1 || B > a->B || S <= 0 || D <= 0 || D % 64 || !q ||
        !k || !v || !gate || !mix || !context_k || !context_v)
        return set_error(ctx, "dit_attention: invalid arguments (D a multiple of 64, B at most "
                              "the batch of an attention context made on this context)");
    if (((((uintptr_t)q) | ((uintptr_t)k) | ((uintptr_t)v) | ((uintptr_t)gate) |
          ((uintptr_t)mix) | ((uintptr_t)context_k) | ((uintptr_t)context_v)) & 15) != 0)
        return set_error(ctx, "dit_attention: every tensor must be 16-byte aligned");
    const int H = D / 64;
    const long long Jmax = (long long)S + a->max_valid;
    const long long Jp = (Jmax + kKT - 1) / kKT * kKT;
    const long long R = (long long)B * H * S;
    if (R > INT32_MAX / 2 || Jp > INT32_MAX / 2 || (long long)S > 65535LL * 32 ||
        (long long)B * H > 65535)
        return set_error(ctx, "dit_attention: shape too large");
    Workspace ws{ctx};
    const size_t o_sc = ws.reserve((size_t)R * Jp * sizeof(float));
    const size_t o_pm = ws.reserve((size_t)R * (Jp / kKT) * sizeof(float));
    const size_t o_sum = ws.reserve((size_t)R * sizeof(float));
    if (ws.commit()) return -1;
    float *sc = ws.at<float>(o_sc), *pm = ws.at<float>(o_pm), *sums = ws.at<float>(o_sum);
    const int C = a->C;
    hipLaunchKernelGGL(attn_scores_kernel, dim3((unsigned)(Jp / kKT), (S + kQT - 1) / kQT, B * H),
                       dim3(256), 0, ctx->stream, q, k, context_k, a->rows, a->nvalid, S, D, H, C,
                       (int)Jp, sc, pm);
    IRO_HIP_CHECK_LAUNCH(ctx);
    constexpr int RW = 8;  // rows per softmax wave (measured: 8 < 16 < 32 in time)
    hipLaunchKernelGGL((attn_softmax_kernel<RW>), dim3((unsigned)((R + RW - 1) / RW)), dim3(64), 0,
                       ctx->stream, sc, pm, a->nvalid, (int)R, S, H, (int)Jp, sums);
    IRO_HIP_CHECK_LAUNCH(ctx);
    // 64 queries per block (16 chains per thread) where that gives at least
    // 2.5 blocks per CU, else 32 (measured on one box at 3 x 750 queries:
    // 20 heads, 2.8 blocks per CU at 64: the call 0.469 ms at 64, 0.516 at 32,
    // 0.500 at 128; 16 heads, 2.25 per CU: 0.407 at 64, 0.397 at 32).
    const int cus = ctx->cus > 0 ? ctx->cus : 256;
    if ((long long)((S + 63) / 64) * B * H * 2 >= 5LL * cus)
        hipLaunchKernelGGL((attn_pv_kernel<64>), dim3((S + 63) / 64, B * H), dim3(256), 0,
                           ctx->stream, sc, sums, v, context_v, a->rows, a->nvalid, gate, S, D, H,
                           C, (int)Jp, mix);
    else
        hipLaunchKernelGGL((attn_pv_kernel<32>), dim3((S + 31) / 32, B * H), dim3(256), 0,
                           ctx->stream, sc, sums, v, context_v, a->rows, a->nvalid, gate, S, D, H,
                           C, (int)Jp, mix);
    IRO_HIP_CHECK_LAUNCH(ctx);
    return 0;
}

}  // extern "C"
