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

// Code as a float in [0, 255] (the reference keeps it as a float `v` and
// clamps it with `v < 0 ? 0 : v`, `v > 255 ? 255 : v`).  fmax / fmin give
// the same value for every non-NaN v; a NaN v (NaN input) becomes 0 here,
// where the reference's clamp keeps NaN and its conversion to u8 then
// yields code 0 as well, so the stored code is the same.
template <int CONV>
__device__ __forceinline__ float quant_value(float x, const RowQ &r) {
    const float v = CONV == 1 ? __builtin_rintf(__builtin_fmaf(x, r.inv, r.zpf))
                              : __builtin_rintf(x * r.inv + r.zpf);
    return __builtin_fminf(__builtin_fmaxf(v, 0.0f), 255.0f);
}

// The value the reference rounds: x*inv + zp (fma in the fast build).
template <int CONV>
__device__ __forceinline__ float quant_pre(float x, const RowQ &r) {
    return CONV == 1 ? __builtin_fmaf(x, r.inv, r.zpf) : x * r.inv + r.zpf;
}

// Four codes packed little-endian into a u32.  v_cvt_pk_u8_f32 rounds to
// nearest even and saturates to [0, 255], NaN to 0 -- clamp(rint(v), 0,
// 255) for every float v, as iro_hip_selfcheck_codes checks on the device
// -- so it takes either the codes or the unrounded quant_pre values.
__device__ __forceinline__ uint32_t pack_codes4(float a, float b, float c, float d) {
    uint32_t w = __builtin_amdgcn_cvt_pk_u8_f32(a, 0, 0u);
    w = __builtin_amdgcn_cvt_pk_u8_f32(b, 1, w);
    w = __builtin_amdgcn_cvt_pk_u8_f32(c, 2, w);
    return __builtin_amdgcn_cvt_pk_u8_f32(d, 3, w);
}

// The four codes of a packed word as floats (v_cvt_f32_ubyte0..3).
__device__ __forceinline__ float4 unpack_codes4(uint32_t w) {
    return make_float4((float)(w & 0xffu), (float)((w >> 8) & 0xffu), (float)((w >> 16) & 0xffu),
                       (float)(w >> 24));
}

// ops.c:437-439 residual: r = x - s1*(q1 - zp1).
template <int CONV>
__device__ __forceinline__ float residual_value(float x, float v, const RowQ &r) {
    return CONV == 1 ? __builtin_fmaf(r.s, r.zpf - v, x) : x - r.s * (v - r.zpf);
}

// Row ranges.  The reference accumulates lo = x < lo ? x : lo and
// hi = x > hi ? x : hi from lo = hi = 0 (ops.c:327-331), which skips NaN
// and never leaves [-inf, 0] resp. [0, inf].  fmin / fmax (one instruction,
// any order) skip NaN too and give the same values, except that a zero
// result may come out as -0 where the reference keeps +0; a zero lo or hi
// of either sign yields the same range, scale, inverse and zero point
// (hi - lo, -lo * inv and rint of them are +-0 alike), so codes and row
// parameters do not change.  Every caller accumulates such a range (or a
// range of |w| from +0).
__device__ __forceinline__ float sel_min(float a, float b) { return __builtin_fminf(a, b); }
__device__ __forceinline__ float sel_max(float a, float b) { return __builtin_fmaxf(a, b); }

// Cross-lane moves for wavefront reductions: DPP within rows of 16 lanes,
// a swizzle across the two rows of each 32-lane half, and the two halves
// combined through scalar reads.  The result is in every lane.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float swz_xor16(float v) {
    // bitmask mode: and 0x1f, or 0, xor 0x10 (lane ^ 16 within 32 lanes)
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}
template <bool MAX>
__device__ __forceinline__ float wave_range(float v) {
    auto op = [](float a, float b) { return MAX ? __builtin_fmaxf(a, b) : __builtin_fminf(a, b); };
    v = op(v, dpp_mov<0xB1>(v));   // quad_perm [1,0,3,2]
    v = op(v, dpp_mov<0x4E>(v));   // quad_perm [2,3,0,1]
    v = op(v, dpp_mov<0x141>(v));  // row_half_mirror
    v = op(v, dpp_mov<0x140>(v));  // row_mirror
    v = op(v, swz_xor16(v));
    const int bits = __builtin_bit_cast(int, v);
    return op(__builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 0)),
              __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 32)));
}
// The same over each 32-lane half of the wave (the result in every lane of
// the half; no lane of the other half is read).
template <bool MAX>
__device__ __forceinline__ float half_range(float v) {
    auto op = [](float a, float b) { return MAX ? __builtin_fmaxf(a, b) : __builtin_fminf(a, b); };
    v = op(v, dpp_mov<0xB1>(v));
    v = op(v, dpp_mov<0x4E>(v));
    v = op(v, dpp_mov<0x141>(v));
    v = op(v, dpp_mov<0x140>(v));
    return op(v, swz_xor16(v));
}
// The same over each aligned group of eight lanes (quad swaps, then the
// half-row mirror pairs lane i with lane 7 - i of its group).
template <bool MAX>
__device__ __forceinline__ float group8_range(float v) {
    auto op = [](float a, float b) { return MAX ? __builtin_fmaxf(a, b) : __builtin_fminf(a, b); };
    v = op(v, dpp_mov<0xB1>(v));
    v = op(v, dpp_mov<0x4E>(v));
    return op(v, dpp_mov<0x141>(v));
}
__device__ __forceinline__ float wave_min(float v) { return wave_range<false>(v); }
__device__ __forceinline__ float wave_max(float v) { return wave_range<true>(v); }
__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

}  // namespace iro
