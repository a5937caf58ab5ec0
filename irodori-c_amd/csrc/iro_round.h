// iro_round.h -- the reference's quantization arithmetic, per convention,
// as device functions.  The library is built with -ffp-contract=off, so
// every float operation rounds where it is written; fused multiply-adds
// appear only where the reference's fast-math build emits one.
//
// CONV 0 (strict, ops.c built -O2):    s = d/255, inv = 1/s,
//     zp = rne(-lo*inv), q = rne(x*inv + zp)                 (ops.c:321-348)
// CONV 1 (GCC 11 -O3 -ffast-math):     s = d*fl(1/255),
//     inv = fl(1/fl(1/255))/d, zp = rne(-(lo*inv)), q = rne(fma(x, inv, zp))
// with d = max(0, max x) - min(0, min x).  Degenerate rows (s not > 0) use
// s = 1, inv = 1.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace iro {

__device__ __forceinline__ float f32_bits(uint32_t u) { return __uint_as_float(u); }

// Constants GCC 11 folds into the fast-math build: x/255 -> x*fl(1/255),
// 1/(d/255) -> fl(1/fl(1/255))/d, 255/(d/255) -> fl(255/fl(1/255))/d,
// x/127 -> x*fl(1/127).
__device__ __forceinline__ float c_inv255() { return f32_bits(0x3B808081u); }      // fl(1/255)
__device__ __forceinline__ float c_255_inv255() { return f32_bits(0x437EFFFFu); }  // fl(1/fl(1/255))
__device__ __forceinline__ float c_255_inv255_b() { return f32_bits(0x477E00FFu); }  // fl(255/fl(1/255))
__device__ __forceinline__ float c_inv127() { return f32_bits(0x3C010204u); }      // fl(1/127)

__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

struct RowQ {
    float s, inv, zpf;
    int zp;
};

template <int CONV>
__device__ __forceinline__ RowQ row_params(float lo, float hi) {
    RowQ r;
    const float d = hi - lo;
    if (CONV == 1) {
        r.s = d * c_inv255();
        if (!(r.s > 0.0f)) {
            r.s = 1.0f;
            r.inv = 1.0f;
            r.zp = clampi((int)__builtin_rintf(-lo), 0, 255);
        } else {
            r.inv = c_255_inv255() / d;
            r.zp = clampi((int)__builtin_rintf(-(lo * r.inv)), 0, 255);
        }
    } else {
        r.s = d / 255.0f;
        if (!(r.s > 0.0f)) r.s = 1.0f;
        r.inv = 1.0f / r.s;
        r.zp = clampi((int)__builtin_rintf(-lo * r.inv), 0, 255);
    }
    r.zpf = (float)r.zp;
    return r;
}

// Code as a float in [0, 255] (the reference keeps it as a float `v`).
template <int CONV>
__device__ __forceinline__ float quant_value(float x, const RowQ &r) {
    float v = CONV == 1 ? __builtin_rintf(__builtin_fmaf(x, r.inv, r.zpf))
                        : __builtin_rintf(x * r.inv + r.zpf);
    v = v < 0.0f ? 0.0f : v;
    v = v > 255.0f ? 255.0f : v;
    return v;
}

// ops.c:437-439 residual: r = x - s1*(q1 - zp1).
template <int CONV>
__device__ __forceinline__ float residual_value(float x, float v, const RowQ &r) {
    return CONV == 1 ? __builtin_fmaf(r.s, r.zpf - v, x) : x - r.s * (v - r.zpf);
}

// Reference select semantics: lo = x < lo ? x : lo, hi = x > hi ? x : hi.
__device__ __forceinline__ float sel_min(float a, float b) { return b < a ? b : a; }
__device__ __forceinline__ float sel_max(float a, float b) { return b > a ? b : a; }

__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = sel_min(v, __shfl_xor(v, off, 64));
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = sel_max(v, __shfl_xor(v, off, 64));
    return v;
}
__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

}  // namespace iro
