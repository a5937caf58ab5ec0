// iro_adaln.hip -- the adaLN parameters of a DiT block on gfx950 (dit.c:543-588):
// per adaLN and branch (shift, scale, gate), SiLU of the branch's slice of
// cond, a rank-R down linear, an up linear plus bias, the slice of cond added
// back, and glibc's tanhf on the gate -- every sum in the scalar build's
// index order, so the parameters are bit-identical to it.
#include <hip/hip_runtime.h>

#include <type_traits>

#include <cstdint>

#include "iro_expf.h"
#include "iro_hip.h"
#include "iro_internal.h"

namespace iro {
namespace {

/* The expm1f / tanhf below follow fdlibm's s_expm1f.c and s_tanhf.c, whose
 * notice is preserved as its licence asks:
 *
 * ====================================================
 * Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
 *
 * Developed at SunPro, a Sun Microsystems, Inc. business.
 * Permission to use, copy, modify, and distribute this
 * software is freely granted, provided that this notice
 * is preserved.
 * ====================================================
 *
 * (float conversion by Ian Lance Taylor, Cygnus Support.)
 */
// expm1f and tanhf as glibc 2.35 computes them: the float port of fdlibm
// 5.3's s_expm1f.c (reduction by ln2 in a high and a low part, the rational
// correction with coefficients Q1..Q5 in x^2/2) and s_tanhf.c (tanh from
// expm1 of 2|x|).  Only IEEE-rounded float operations and bit moves, so the
// device gives libm's bits; checked on all 2^32 inputs by
// iro_hip_selfcheck_tanhf.
__device__ float expm1f_fdlibm(float x) {
    const float one = 1.0f, tiny = 1.0e-30f, huge = 1.0e+30f;
    const float o_threshold = 8.8721679688e+01f, ln2_hi = 6.9313812256e-01f,
                ln2_lo = 9.0580006145e-06f, invln2 = 1.4426950216e+00f;
    const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f,
                Q4 = 4.0082177293e-06f, Q5 = -2.0109921195e-07f;
    float y, hi, lo, c = 0.0f, t, e, hxs, hfx, r1;
    int k;
    uint32_t hx = __float_as_uint(x);
    const uint32_t xsb = hx & 0x80000000u;
    hx &= 0x7fffffffu;
    if (hx >= 0x4195b844u) {  // |x| >= 27 ln2
        if (hx >= 0x42b17218u) {
            if (hx > 0x7f800000u) return x + x;
            if (hx == 0x7f800000u) return xsb == 0 ? x : -1.0f;
            if (x > o_threshold) return huge * huge;
        }
        if (xsb != 0) return tiny - one;
    }
    if (hx > 0x3eb17218u) {  // |x| > ln2 / 2
        if (hx < 0x3F851592u) {  // and < 1.5 ln2
            if (xsb == 0) {
                hi = x - ln2_hi;
                lo = ln2_lo;
                k = 1;
            } else {
                hi = x + ln2_hi;
                lo = -ln2_lo;
                k = -1;
            }
        } else {
            k = (int)(invln2 * x + (xsb == 0 ? 0.5f : -0.5f));
            t = (float)k;
            hi = x - t * ln2_hi;
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000u) {  // |x| < 2^-25
        t = huge + x;
        return x - (t - (huge + x));
    } else {
        k = 0;
    }
    hfx = 0.5f * x;
    hxs = x * hfx;
    r1 = one + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    t = 3.0f - r1 * hfx;
    e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = (x * (e - c) - c);
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) {
        if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
        return one + 2.0f * (x - e);
    }
    if (k <= -2 || k > 56) {
        y = one - (e - x);
        y = __uint_as_float(__float_as_uint(y) + ((uint32_t)k << 23));
        return y - one;
    }
    if (k < 23) {
        t = __uint_as_float(0x3f800000u - (0x1000000u >> k));
        y = t - (e - x);
        y = __uint_as_float(__float_as_uint(y) + ((uint32_t)k << 23));
    } else {
        t = __uint_as_float((uint32_t)(0x7f - k) << 23);
        y = x - (e + t);
        y += one;
        y = __uint_as_float(__float_as_uint(y) + ((uint32_t)k << 23));
    }
    return y;
}

__device__ float tanhf_fdlibm(float x) {
    const float one = 1.0f, two = 2.0f, tiny = 1.0e-30f;
    float t, z;
    const int32_t jx = (int32_t)__float_as_uint(x), ix = jx & 0x7fffffff;
    if (ix >= 0x7f800000) return jx >= 0 ? one / x + one : one / x - one;
    if (ix < 0x41b00000) {  // |x| < 22
        if (ix == 0) return x;
        if (ix < 0x24000000) return x * (one + x);  // |x| < 2^-55
        if (ix >= 0x3f800000) {                     // |x| >= 1
            t = expm1f_fdlibm(two * __builtin_fabsf(x));
            z = one - two / (t + two);
        } else {
            t = expm1f_fdlibm(-two * __builtin_fabsf(x));
            z = -t / (t + two);
        }
    } else {
        z = one - tiny;
    }
    return jx >= 0 ? z : -z;
}

// Digest of tanhf over inputs base .. base + 2^28 - 1: the sum over u of
// (u * K1) ^ (bits(tanhf(u)) * K2), NaN results as 0x7FC00000.
__global__ __launch_bounds__(256) void tanhf_selfcheck_kernel(unsigned long long *out,
                                                              unsigned base) {
    __shared__ unsigned long long part[4];
    const unsigned u = base + blockIdx.x * 256u + threadIdx.x;
    const float t = tanhf_fdlibm(__uint_as_float(u));
    const unsigned ut = t != t ? 0x7FC00000u : __float_as_uint(t);
    unsigned long long h = ((unsigned long long)u * 0x9E3779B97F4A7C15ull) ^
                           ((unsigned long long)ut * 0xC2B2AE3D27D4EB4Full);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) h += __shfl_xor(h, off, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = h;
    __syncthreads();
    if (threadIdx.x == 0) atomicAdd(out, part[0] + part[1] + part[2] + part[3]);
}

struct AdaWeights {
    const float *w[18];  // per adaLN: down, up, bias of shift, scale, gate
};

// act [3][B][D] = silu(cond[b, br*D + d]) as x / (1 + expf(-x)) (ops.c:776-779).
__global__ __launch_bounds__(256) void ada_act_kernel(const float *__restrict__ cond, int B, int D,
                                                      float *__restrict__ act) {
    __shared__ uint64_t exptab[32];
    if (threadIdx.x < 32) exptab[threadIdx.x] = kExp2Tab[threadIdx.x];
    __syncthreads();
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= 3 * B * D) return;
    const int br = i / (B * D), rem = i - br * B * D, b = rem / D, d = rem - b * D;
    const float x = cond[(size_t)b * 3 * D + (size_t)br * D + d];
    act[i] = x / (1.0f + expf_glibc(-x, exptab));
}

// sum_d x[d] * w[d] for d = 0 .. n-1 in index order (each product rounded,
// then added): x in LDS (the block's shared row), w this lane's row in
// global memory.  When w is 16-byte aligned the row streams through
// registers 64 values at a time, the next 64 loaded while the current ones
// are added, so the chain waits on memory once per row rather than per term.
__device__ __forceinline__ float dot_in_order(const float *x, const float *__restrict__ w,
                                              int n) {
    float acc = 0.0f;
    int d = 0;
    if ((((uintptr_t)w) & 15) == 0) {
        const int nc = n / 64;
        float4 cur[16], nxt[16];
        if (nc > 0) {
#pragma unroll
            for (int j = 0; j < 16; ++j) cur[j] = reinterpret_cast<const float4 *>(w)[j];
        }
        for (int c = 0; c < nc; ++c) {
            if (c + 1 < nc) {
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    nxt[j] = reinterpret_cast<const float4 *>(w + (c + 1) * 64)[j];
            }
            const float *xc = x + c * 64;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                acc = acc + xc[4 * j] * cur[j].x;
                acc = acc + xc[4 * j + 1] * cur[j].y;
                acc = acc + xc[4 * j + 2] * cur[j].z;
                acc = acc + xc[4 * j + 3] * cur[j].w;
            }
#pragma unroll
            for (int j = 0; j < 16; ++j) cur[j] = nxt[j];
        }
        d = nc * 64;
    }
    for (; d < n; ++d) acc = acc + x[d] * w[d];
    return acc;
}

// low [A][3][B][R]: lane r of (adaLN a, branch br, batch b) sums act * down
// over d in index order, then adds the scalar linear's zero bias.  The
// block's act row is staged in LDS (D <= kAdaMaxD).
constexpr int kAdaMaxD = 8192;
__global__ __launch_bounds__(64) void ada_low_kernel(const float *__restrict__ act, AdaWeights w,
                                                     int B, int D, int R,
                                                     float *__restrict__ low) {
    __shared__ __attribute__((aligned(16))) float xs[kAdaMaxD];
    const int br = blockIdx.y / B, b = blockIdx.y - br * B, a = blockIdx.z;
    const float *x = act + ((size_t)br * B + b) * D;
    for (int d = threadIdx.x; d < D; d += 64) xs[d] = x[d];
    __syncthreads();
    const int r = blockIdx.x * 64 + threadIdx.x;
    if (r >= R) return;
    const float acc = dot_in_order(xs, w.w[a * 9 + br * 3] + (size_t)r * D, D);
    low[(((size_t)a * 3 + br) * B + b) * R + r] = acc + 0.0f;
}

// The same sums with the down rows through LDS, for B <= 4 batch rows and
// D % 4 == 0 with 16-byte aligned rows: a block takes 64 rows r of one
// (adaLN a, branch br) for every batch row; its four waves read 64 x 64
// tiles of those rows (each row's 256 bytes by 16 consecutive lanes) and of
// the act rows into a three-deep LDS ring, two tiles ahead of the sums (the
// loads themselves go out six tiles ahead, through registers), and
// wave b runs the in-order sums of batch row b from LDS.  Each down row is
// read once per block instead of once per batch row with one strided load
// per lane and step.
constexpr int kRingK = 64, kRingP = 65;
__global__ __launch_bounds__(256) void ada_low_ring_kernel(const float *__restrict__ act,
                                                           AdaWeights w, int B, int D, int R,
                                                           float *__restrict__ low) {
    __shared__ float tile[3][64 * kRingP];
    __shared__ __attribute__((aligned(16))) float xs[3][4][kRingK];
    const int br = blockIdx.y, a = blockIdx.z, r0 = blockIdx.x * 64;
    const float *down = w.w[a * 9 + br * 3];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nc = (D + kRingK - 1) / kRingK;
    // Loads of chunk c: float4 q = tid + 256 i of the tile (row q / 16,
    // columns 4 (q % 16) ..), and for tid < 16 B the float4 of act row
    // tid / 16.  Past D or R: zeros (never summed or stored).
    float4 rt[4][4], rx[4];
    auto load = [&](float4 (&t)[4], float4 &x, int c) {
        const int k0 = c * kRingK;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = tid + 256 * i, rr = q >> 4, k = k0 + (q & 15) * 4;
            t[i] = (c < nc && r0 + rr < R && k < D)
                       ? *reinterpret_cast<const float4 *>(down + (size_t)(r0 + rr) * D + k)
                       : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        const int k = k0 + (tid & 15) * 4;
        x = (c < nc && tid < 16 * B && k < D)
                ? *reinterpret_cast<const float4 *>(act + ((size_t)br * B + (tid >> 4)) * D + k)
                : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    };
    auto store = [&](const float4 (&t)[4], const float4 &x, int slot) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = tid + 256 * i;
            float *dst = &tile[slot][(q >> 4) * kRingP + (q & 15) * 4];
            dst[0] = t[i].x;
            dst[1] = t[i].y;
            dst[2] = t[i].z;
            dst[3] = t[i].w;
        }
        if (tid < 64) *reinterpret_cast<float4 *>(&xs[slot][tid >> 4][(tid & 15) * 4]) = x;
    };
    float acc = 0.0f;
    // Iteration c stores chunk c + 2 (loaded four iterations before) into
    // the slot chunk c - 1 left, loads chunk c + 6, and sums chunk c.
    auto iter = [&](int c, auto par) {
        constexpr int P = decltype(par)::value;  // c % 4
        __syncthreads();
        store(rt[P], rx[P], (c + 2) % 3);
        load(rt[P], rx[P], c + 6);
        if (wave < B) {
            const float *tr = &tile[c % 3][lane * kRingP];
            const float *xr = xs[c % 3][wave];
            const int n = D - c * kRingK < kRingK ? D - c * kRingK : kRingK;
            if (n == kRingK) {
#pragma unroll 16
                for (int k = 0; k < kRingK; ++k) acc = acc + xr[k] * tr[k];
            } else {
                for (int k = 0; k < n; ++k) acc = acc + xr[k] * tr[k];
            }
        }
    };
    load(rt[0], rx[0], 0);
    load(rt[1], rx[1], 1);
    store(rt[0], rx[0], 0);
    store(rt[1], rx[1], 1);
    load(rt[0], rx[0], 2);
    load(rt[1], rx[1], 3);
    load(rt[2], rx[2], 4);
    load(rt[3], rx[3], 5);
    for (int c = 0; c < nc; c += 4) {
        iter(c, std::integral_constant<int, 0>{});
        if (c + 1 < nc) iter(c + 1, std::integral_constant<int, 1>{});
        if (c + 2 < nc) iter(c + 2, std::integral_constant<int, 2>{});
        if (c + 3 < nc) iter(c + 3, std::integral_constant<int, 3>{});
    }
    const int r = r0 + lane;
    if (wave < B && r < R) low[(((size_t)a * 3 + br) * B + wave) * R + r] = acc + 0.0f;
}

// out [A][3][B][D]: (sum_r low * up in index order) + bias, + the cond slice;
// the gate branch through tanhf.  The block's low row is staged in LDS.
__global__ __launch_bounds__(64) void ada_out_kernel(const float *__restrict__ low,
                                                     const float *__restrict__ cond, AdaWeights w,
                                                     int B, int D, int R, float *__restrict__ out) {
    __shared__ __attribute__((aligned(16))) float ls[kAdaMaxD];
    const int br = blockIdx.y / B, b = blockIdx.y - br * B, a = blockIdx.z;
    const float *l = low + (((size_t)a * 3 + br) * B + b) * R;
    for (int r = threadIdx.x; r < R; r += 64) ls[r] = l[r];
    __syncthreads();
    const int n = blockIdx.x * 64 + threadIdx.x;
    if (n >= D) return;
    const float acc = dot_in_order(ls, w.w[a * 9 + br * 3 + 1] + (size_t)n * R, R);
    const float y = acc + w.w[a * 9 + br * 3 + 2][n];
    float o = y + cond[(size_t)b * 3 * D + (size_t)br * D + n];
    if (br == 2) o = tanhf_fdlibm(o);
    out[(((size_t)a * 3 + br) * B + b) * D + n] = o;
}

}  // namespace
}  // namespace iro

using namespace iro;

extern "C" {

int iro_hip_dit_adaln_params(IroHipContext *ctx, const float *cond, int B, int D, int R,
                             const float *const *weights, int n_adaln, float *out) {
    if (!ctx || !cond || !weights || !out || B <= 0 || D <= 0 || R <= 0 ||
        (n_adaln != 1 && n_adaln != 2))
        return set_error(ctx, "dit_adaln_params: invalid arguments");
    if ((long long)3 * B * D > INT32_MAX / 2 || 3LL * B > 65535 || D > kAdaMaxD || R > kAdaMaxD)
        return set_error(ctx, "dit_adaln_params: shape too large (D, R <= %d)", kAdaMaxD);
    AdaWeights w{};
    for (int i = 0; i < 9 * n_adaln; ++i) {
        if (!weights[i]) return set_error(ctx, "dit_adaln_params: weight %d is NULL", i);
        w.w[i] = weights[i];
    }
    Workspace ws{ctx};
    const size_t o_act = ws.reserve(sizeof(float) * 3 * (size_t)B * D);
    const size_t o_low = ws.reserve(sizeof(float) * (size_t)n_adaln * 3 * B * R);
    if (ws.commit()) return -1;
    float *act = ws.at<float>(o_act), *low = ws.at<float>(o_low);
    hipLaunchKernelGGL(ada_act_kernel, dim3((3 * B * D + 255) / 256), dim3(256), 0, ctx->stream,
                       cond, B, D, act);
    IRO_HIP_CHECK_LAUNCH(ctx);
    bool ring = B <= 4 && D % 4 == 0;
    for (int i = 0; i < n_adaln * 3; ++i)
        ring = ring && (((uintptr_t)w.w[(i / 3) * 9 + (i % 3) * 3]) & 15) == 0;
    if (ring)
        hipLaunchKernelGGL(ada_low_ring_kernel, dim3((R + 63) / 64, 3, n_adaln), dim3(256), 0,
                           ctx->stream, act, w, B, D, R, low);
    else
        hipLaunchKernelGGL(ada_low_kernel, dim3((R + 63) / 64, 3 * B, n_adaln), dim3(64), 0,
                           ctx->stream, act, w, B, D, R, low);
    IRO_HIP_CHECK_LAUNCH(ctx);
    hipLaunchKernelGGL(ada_out_kernel, dim3((D + 63) / 64, 3 * B, n_adaln), dim3(64), 0,
                       ctx->stream, low, cond, w, B, D, R, out);
    IRO_HIP_CHECK_LAUNCH(ctx);
    return 0;
}

int iro_hip_selfcheck_tanhf(IroHipContext *ctx, unsigned long long *digest) {
    if (!ctx || !digest) return set_error(ctx, "selfcheck_tanhf: invalid arguments");
    Workspace ws{ctx};
    const size_t o = ws.reserve(sizeof(unsigned long long));
    if (ws.commit()) return -1;
    unsigned long long *d = ws.at<unsigned long long>(o);
    if (launch_fill(ctx, d, 0, sizeof(unsigned long long))) return -1;
    for (unsigned long long base = 0; base < (1ull << 32); base += (1ull << 28)) {
        hipLaunchKernelGGL(tanhf_selfcheck_kernel, dim3(1u << 20), dim3(256), 0, ctx->stream, d,
                           (unsigned)base);
        IRO_HIP_CHECK_LAUNCH(ctx);
    }
    IRO_HIP_TRY(ctx, hipMemcpyAsync(digest, d, sizeof(unsigned long long), hipMemcpyDeviceToHost,
                                    ctx->stream));
    IRO_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return 0;
}

}  // extern "C"
