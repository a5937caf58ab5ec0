// iro_gemm.hip -- int8 x int8 -> int32 GEMM on gfx950 MFMA with the
// reference's dequantization epilogue fused in.
//
// C[m,n] = sum_k A[m,k] * W[n,k], A = u8 activation codes (row-major),
// W = s8 weight codes pre-packed in 1 KiB MFMA fragments (IroHipWeight).
// gfx950 int8 MFMA is signed-only, so A is fed as (a ^ 0x80) = a - 128 and
// the raw u8 x s8 sum is recovered exactly in int32 as
// acc + 128 * rowsum[n], rowsum = sum over k of W[n,k]  (|acc| < 2^31 for
// K < 66k).
//
// Tiling: 256 threads = 4 wavefronts in 2x2, block tile 128x128x64, wave
// tile 64x64 = 2x2 v_mfma_i32_32x32x32_i8.  Both operands are staged in LDS
// in fragment order (lane L reads 16 bytes at L*16), so every ds_read_b128
// is conflict-free; LDS is double-buffered with one barrier per k-step.
// The two-term activation (ops.c:427-442 + dit.c:477-485) runs both planes
// against the same W fragment, two accumulators, one pass over W.
//
// Epilogues (all per element, identical op order to the reference):
//   EPI_LINEAR  ops.c:468-490 four branches (+ optional raw int32 `work`)
//   EPI_QKVG    dit.c:786-792 four projections, split store
//   EPI_SWIGLU  dit.c:945-956 W1,W3 then silu(w1)*w3 (ops.c:781-784)
//   EPI_GATED   dit.c:1013-1020 / 1032-1039 x += gate[b] * y
#include "iro_internal.h"
#include "iro_round.h"

namespace iro {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int TILE_A = BM * BK;  // bytes per A plane per stage
constexpr int TILE_B = BN * BK;

struct KParams {
    const uint8_t *a1, *a2;
    int lda;
    const int8_t *bp;
    int kb_count;  // Kp / 32
    int M, N, K;
    const float *sx1, *sx2;
    const int32_t *zx1, *zx2;
    const float *sw;
    const int32_t *colsum;
    const int32_t *rowsum;
    const float *bias;
    float *y;
    int ldy;
    int32_t *work;
    int ldw;
    int accumulate;
    float *seg0, *seg1, *seg2, *seg3;
    int seg_n;
    float *hidden;
    int ldh;
    int hidden_n;
    float *xres;
    const float *gate;
    int ldg;
    int ldx;
    int rows_per_branch;
};

// ops.c:468-490: y = t*c [+ b] or y += t*c [+ b] with the build's rounding.
template <int CONV>
__device__ __forceinline__ float lin_out(float t, float c, float b, bool has_bias, bool acc,
                                         float yold) {
    if (CONV == 1) {
        if (acc && has_bias) return __builtin_fmaf(t, c, yold + b);
        if (acc) return __builtin_fmaf(t, c, yold);
        if (has_bias) return __builtin_fmaf(t, c, b);
        return t * c;
    }
    if (acc && has_bias) return yold + (t * c + b);
    if (acc) return yold + t * c;
    if (has_bias) return t * c + b;
    return t * c;
}

// Second plane accumulated without bias (accumulate = 1 branch).
template <int CONV>
__device__ __forceinline__ float add_term(float y, float t, float c) {
    return CONV == 1 ? __builtin_fmaf(t, c, y) : y + t * c;
}

// expf as glibc >= 2.28 computes it on x86-64 with FMA (the __expf_fma
// ifunc variant the reference's libm call resolves to): the published
// exp2f table method of ARM optimized-routines, N = 32:
//   x*N/ln2 = k + r,  exp(x) = 2^(k/N) * (1 + C2 r + C1 r^2 + C0 r^3),
// in double, with GCC's contraction of both uses of InvLn2N*x into FMAs.
// Bit-identical to glibc's expf for every float input.
__constant__ uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

__device__ __forceinline__ float expf_glibc(float x) {
    if (x != x) return x + x;
    if (x > 0x1.62e42ep6f) return __builtin_inff();  // overflow
    if (x < -0x1.9fe368p6f) return 0.0f;             // underflow (and -inf)
    const double invln2n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    double kd = __builtin_fma(invln2n, xd, shift);
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= shift;
    const double r = __builtin_fma(invln2n, xd, -kd);
    const uint64_t t = kExp2Tab[ki % 32] + (ki << 47);
    const double s = __longlong_as_double((long long)t);
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    return (float)(y * s);
}

// ops.c:781-784 as the strict build computes it: x / (1 + expf(-x)) * g.
__device__ __forceinline__ float silu_mul(float a, float g) {
    const float e = expf_glibc(-a);
    return (a / (1.0f + e)) * g;
}

template <int CONV, int EPI, bool TWO>
__global__ __launch_bounds__(256) void gemm_i8_kernel(KParams p) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[2][(TWO ? 2 : 1) * TILE_A + TILE_B];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * BN;

    // Global sources of this thread's two 16-byte chunks per operand.
    const uint8_t *pa1[2];
    const uint8_t *pa2[2];
    const int8_t *pb[2];
    int kk_of[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = tid + 256 * i;
        const int f = c >> 6, ln = c & 63;
        const int row = (f & 3) * 32 + (ln & 31);
        const int kk = (f >> 2) * 32 + (ln >> 5) * 16;
        int gr = m0 + row;
        gr = gr < p.M ? gr : p.M - 1;
        kk_of[i] = kk;
        pa1[i] = p.a1 + (size_t)gr * p.lda + kk;
        pa2[i] = TWO ? p.a2 + (size_t)gr * p.lda + kk : nullptr;
        pb[i] = p.bp + ((size_t)((n0 >> 5) + (f >> 1)) * p.kb_count + (f & 1)) * 1024 + ln * 16;
    }

    v16i acc[2][2], acc2[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                acc[i][j][r] = 0;
                acc2[i][j][r] = 0;
            }
        }

    v4i ra1[2], ra2[2], rb[2];
    const v4i flip = {(int)0x80808080, (int)0x80808080, (int)0x80808080, (int)0x80808080};
    const v4i zero4 = {0, 0, 0, 0};

    auto gload = [&](int kt) {
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const bool ok = k0 + kk_of[i] < p.K;
            ra1[i] = (ok ? *reinterpret_cast<const v4i *>(pa1[i] + k0) : zero4) ^ flip;
            if (TWO) ra2[i] = (ok ? *reinterpret_cast<const v4i *>(pa2[i] + k0) : zero4) ^ flip;
            rb[i] = *reinterpret_cast<const v4i *>(pb[i] + (size_t)kt * 2048);
        }
    };
    auto sstore = [&](int buf) {
        uint8_t *base = lds[buf];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int off = (tid + 256 * i) * 16;
            *reinterpret_cast<v4i *>(base + off) = ra1[i];
            if (TWO) *reinterpret_cast<v4i *>(base + TILE_A + off) = ra2[i];
            *reinterpret_cast<v4i *>(base + (TWO ? 2 : 1) * TILE_A + off) = rb[i];
        }
    };

    const int nk = (p.K + BK - 1) / BK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);
        const uint8_t *A1 = lds[cur];
        const uint8_t *A2 = A1 + TILE_A;
        const uint8_t *B = A1 + (TWO ? 2 : 1) * TILE_A;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            v4i a[2], a2[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int off = ((s * 4 + wm * 2 + i) * 64 + lane) * 16;
                a[i] = *reinterpret_cast<const v4i *>(A1 + off);
                if (TWO) a2[i] = *reinterpret_cast<const v4i *>(A2 + off);
            }
#pragma unroll
            for (int j = 0; j < 2; ++j)
                b[j] = *reinterpret_cast<const v4i *>(B + (((wn * 2 + j) * 2 + s) * 64 + lane) * 16);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
                    if (TWO)
                        acc2[i][j] =
                            __builtin_amdgcn_mfma_i32_32x32x32_i8(a2[i], b[j], acc2[i][j], 0, 0, 0);
                }
        }
        if (kt + 1 < nk) sstore(cur ^ 1);
        __syncthreads();
    }

    // ---- epilogue ----------------------------------------------------------
    // 32x32 accumulator layout: lane L, register r holds
    // row 8*(r/4) + 4*(L/32) + r%4, column L%32.
    int ncol[2], cs[2], rs[2];
    float swv[2], bv[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        ncol[j] = n0 + wn * 64 + j * 32 + (lane & 31);
        cs[j] = p.colsum[ncol[j]];  // padded to Np: always in bounds
        rs[j] = p.rowsum[ncol[j]];
        swv[j] = p.sw[ncol[j]];
        bv[j] = (EPI == EPI_LINEAR && p.bias && ncol[j] < p.N) ? p.bias[ncol[j]] : 0.0f;
    }
    const bool has_bias = EPI == EPI_LINEAR && p.bias != nullptr;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = m0 + wm * 64 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
            if (m >= p.M) continue;
            const float sx1 = p.sx1[m];
            const int zx1 = p.zx1[m];
            float sx2 = 0.0f;
            int zx2 = 0;
            if (TWO) {
                sx2 = p.sx2[m];
                zx2 = p.zx2[m];
            }
            float yv[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int raw = acc[i][j][r] + 128 * rs[j];
                const float t = (float)(raw - zx1 * cs[j]);
                const float c = sx1 * swv[j];
                float y;
                if (EPI == EPI_LINEAR) {
                    if (ncol[j] >= p.N) {
                        yv[j] = 0.0f;
                        continue;
                    }
                    const size_t yi = (size_t)m * p.ldy + ncol[j];
                    const float yold = p.accumulate ? p.y[yi] : 0.0f;
                    y = lin_out<CONV>(t, c, bv[j], has_bias, p.accumulate != 0, yold);
                    if (p.work) p.work[(size_t)m * p.ldw + ncol[j]] = raw;
                } else {
                    y = t * c;
                }
                if (TWO) {
                    const int raw2 = acc2[i][j][r] + 128 * rs[j];
                    const float t2 = (float)(raw2 - zx2 * cs[j]);
                    const float c2 = sx2 * swv[j];
                    y = add_term<CONV>(y, t2, c2);
                }
                yv[j] = y;
                if (EPI == EPI_LINEAR) {
                    p.y[(size_t)m * p.ldy + ncol[j]] = y;
                } else if (EPI == EPI_QKVG) {
                    if (ncol[j] < p.N) {
                        const int sg = ncol[j] / p.seg_n;
                        float *dst = sg == 0 ? p.seg0 : (sg == 1 ? p.seg1 : (sg == 2 ? p.seg2 : p.seg3));
                        dst[(size_t)m * p.seg_n + (ncol[j] - sg * p.seg_n)] = y;
                    }
                } else if (EPI == EPI_GATED) {
                    if (ncol[j] < p.N) {
                        const size_t xi = (size_t)m * p.ldx + ncol[j];
                        const float g = p.gate[(size_t)(m / p.rows_per_branch) * p.ldg + ncol[j]];
                        const float x = p.xres[xi];
                        p.xres[xi] = CONV == 1 ? __builtin_fmaf(g, y, x) : x + g * y;
                    }
                }
            }
            if (EPI == EPI_SWIGLU) {
                const int hcol = ((n0 + wn * 64) >> 6) * 32 + (lane & 31);
                if (hcol < p.hidden_n) p.hidden[(size_t)m * p.ldh + hcol] = silu_mul(yv[0], yv[1]);
            }
        }
    }
}

template <int CONV, int EPI>
void launch_t(const KParams &kp, bool two, dim3 grid, hipStream_t st) {
    if (two)
        hipLaunchKernelGGL((gemm_i8_kernel<CONV, EPI, true>), grid, dim3(256), 0, st, kp);
    else
        hipLaunchKernelGGL((gemm_i8_kernel<CONV, EPI, false>), grid, dim3(256), 0, st, kp);
}

template <int CONV>
void launch_c(const KParams &kp, Epi epi, bool two, dim3 grid, hipStream_t st) {
    switch (epi) {
        case EPI_LINEAR: launch_t<CONV, EPI_LINEAR>(kp, two, grid, st); break;
        case EPI_QKVG: launch_t<CONV, EPI_QKVG>(kp, two, grid, st); break;
        case EPI_SWIGLU: launch_t<CONV, EPI_SWIGLU>(kp, two, grid, st); break;
        case EPI_GATED: launch_t<CONV, EPI_GATED>(kp, two, grid, st); break;
    }
}

}  // namespace

int launch_gemm(IroHipContext *ctx, const IroHipWeight *w, const GemmArgs &a, Epi epi) {
    if (a.M <= 0) return 0;
    if (a.K <= 0 || a.K % 16 || a.K > w->Kp || a.lda % 16 || (((uintptr_t)a.a1) & 15) ||
        (a.a2 && (((uintptr_t)a.a2) & 15)) || w->Np % BN)
        return set_error(ctx, "gemm: unsupported operand shape (K=%d lda=%d Kp=%d Np=%d)", a.K,
                         a.lda, w->Kp, w->Np);
    if (epi == EPI_SWIGLU && (w->layout != 1 || w->part_N[0] % 32))
        return set_error(ctx, "gemm: SwiGLU epilogue needs an interleaved W1/W3 weight");
    if (epi == EPI_QKVG && (a.seg_n <= 0 || w->N > 4 * a.seg_n))
        return set_error(ctx, "gemm: QKVG epilogue needs N <= 4 * segment width");
    KParams kp;
    kp.a1 = a.a1;
    kp.a2 = a.a2;
    kp.lda = a.lda;
    kp.bp = w->packed;
    kp.kb_count = w->Kp / 32;
    kp.M = a.M;
    kp.N = w->N;
    kp.K = a.K;
    kp.sx1 = a.sx1;
    kp.sx2 = a.sx2;
    kp.zx1 = a.zx1;
    kp.zx2 = a.zx2;
    kp.sw = w->scale;
    kp.colsum = w->colsum;
    kp.rowsum = w->rowsum;
    kp.bias = a.bias;
    kp.y = a.y;
    kp.ldy = a.ldy;
    kp.work = a.work;
    kp.ldw = a.ldw;
    kp.accumulate = a.accumulate;
    kp.seg0 = a.seg[0];
    kp.seg1 = a.seg[1];
    kp.seg2 = a.seg[2];
    kp.seg3 = a.seg[3];
    kp.seg_n = a.seg_n;
    kp.hidden = a.hidden;
    kp.ldh = a.ldh;
    kp.hidden_n = w->layout == 1 ? w->part_N[0] : 0;
    kp.xres = a.xres;
    kp.gate = a.gate;
    kp.ldg = a.ldg > 0 ? a.ldg : a.ldx;
    kp.ldx = a.ldx;
    kp.rows_per_branch = a.rows_per_branch > 0 ? a.rows_per_branch : 1;
    const dim3 grid(w->Np / BN, (a.M + BM - 1) / BM);
    const bool two = a.a2 != nullptr;
    prof_begin(ctx);
    if (ctx->convention == IRO_HIP_GCC_FASTMATH)
        launch_c<1>(kp, epi, two, grid, ctx->stream);
    else
        launch_c<0>(kp, epi, two, grid, ctx->stream);
    IRO_HIP_CHECK_LAUNCH(ctx);
    // Algorithmic work: 2*M*N*K per plane; bytes = codes + weights + outputs.
    const double M = a.M, N = w->N, K = w->K, planes = two ? 2 : 1;
    double out_bytes = 4 * M * N;
    ProfKind kind = two ? PK_GEMM_LINEAR_2T : PK_GEMM_LINEAR;
    if (epi == EPI_LINEAR) {
        out_bytes *= 1 + (a.accumulate ? 1 : 0) + (a.work ? 1 : 0);
    } else if (epi == EPI_QKVG) {
        kind = two ? PK_GEMM_QKVG_2T : PK_GEMM_QKVG;
    } else if (epi == EPI_SWIGLU) {
        kind = two ? PK_GEMM_SWIGLU_2T : PK_GEMM_SWIGLU;
        out_bytes /= 2;
    } else {
        kind = two ? PK_GEMM_GATED_2T : PK_GEMM_GATED;
        out_bytes *= 2;
    }
    prof_end(ctx, kind, 2 * M * N * K * planes, M * K * planes + N * K + out_bytes);
    return 0;
}

}  // namespace iro
