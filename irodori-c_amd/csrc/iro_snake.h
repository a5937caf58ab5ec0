// iro_snake.h -- the snake activation of one element, shared by the snake
// kernels (iro_codec.hip) and the quantizer that applies it on the fly
// (iro_quant.hip).  Inline device code in an anonymous namespace.
#pragma once

#include "iro_sincosf.h"

namespace iro {
namespace {

constexpr int kSnakeMaxChannels = 1536;  // dacvae.c:808 SNAKE_MAX_CHANNELS

// y = x + sin(a x)^2 / a as the reference computes it per element
// (dacvae.c:827-857, dacvae.c:910-931), x already biased: INV takes the
// hoisted reciprocal inv = 1 / (a + 1e-9) (channels <= 1536), y = x +
// (s * s) * inv, which the fast build (FMA) contracts into one fma; the
// quotient form is y = x + (s * s) / (a + 1e-9).  sinf is glibc's.
template <bool INV, bool FMA>
__device__ __forceinline__ float snake_finish(float xv, float s, float a, float inv) {
    const float ss = s * s;
    if (INV) return FMA ? __builtin_fmaf(ss, inv, xv) : xv + ss * inv;
    return xv + ss / (a + 1e-9f);
}

template <bool INV, bool FMA>
__device__ __forceinline__ float snake_value(float xv, float a, float inv) {
    return snake_finish<INV, FMA>(xv, sinf_glibc(a * xv), a, inv);
}

// A kernel's LDS copy of kInvPio4 for the large reduction (a per-lane
// table read then comes from LDS): threads 0..23 fill it, and a barrier must
// follow before snake_value4 reads it.
__device__ __forceinline__ void stage_invpio4(uint32_t *dst, int tid) {
    if (tid < 24) dst[tid] = kInvPio4[tid];
}

// snake_value of four elements: sinf's fast reduction, branch-free, on all
// four (a large y replaced by 0 there), the large reduction for the elements
// with |y| >= 120 only, then one polynomial each, so the evaluations
// interleave and a wave holding both kinds runs the polynomial once.
template <bool INV, bool FMA>
__device__ __forceinline__ float4 snake_value4(float4 xv, float4 a, float4 inv,
                                               const uint32_t *invpio4 = kInvPio4) {
    const float y[4] = {a.x * xv.x, a.y * xv.y, a.z * xv.z, a.w * xv.w};
    SinCosArg r[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        // selected in single precision (the empty asm keeps the compiler from
        // moving the select past the widening, which would take two)
        float ys = sincosf_is_small(y[k]) ? y[k] : 0.0f;
        asm("" : "+v"(ys));
        r[k] = sincosf_reduce_small(ys);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (__builtin_expect(!sincosf_is_small(y[k]), 0))
            r[k] = sincosf_reduce_large(y[k], invpio4);
    const SinCosAddends ad = sincos_addends();
    return make_float4(snake_finish<INV, FMA>(xv.x, sincosf_finish(y[0], r[0], 0, ad), a.x, inv.x),
                       snake_finish<INV, FMA>(xv.y, sincosf_finish(y[1], r[1], 0, ad), a.y, inv.y),
                       snake_finish<INV, FMA>(xv.z, sincosf_finish(y[2], r[2], 0, ad), a.z, inv.z),
                       snake_finish<INV, FMA>(xv.w, sincosf_finish(y[3], r[3], 0, ad), a.w, inv.w));
}

// The reciprocal the INV form hoists out of its loop (dacvae.c:827-828).
__device__ __forceinline__ float snake_inv(float a) { return 1.0f / (a + 1e-9f); }

}  // namespace
}  // namespace iro
