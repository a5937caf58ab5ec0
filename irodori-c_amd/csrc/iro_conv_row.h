// iro_conv_row.h -- the per-output-step quantization of the int8 Conv1d
// (dacvae.c:617-663), shared by the im2col kernels (iro_conv.hip) and the
// GEMM that codes its activation rows itself (iro_conv_gemm.hip).  Inline
// device code in an anonymous namespace.
#pragma once

#include "iro_round.h"

namespace iro {
namespace {

// Second-plane scale and inverse of an output step from its window range
// (dacvae.c:637-652): scale s / 255, zero point 128.
template <int CONV>
__device__ __forceinline__ void conv_plane2_params(const RowQ &q, float lo, float hi, float &sc2,
                                                   float &inv2) {
    if (CONV == 1) {
        const float d = hi - lo;
        sc2 = q.s * c_inv255();
        inv2 = d * c_inv255() > 0.0f ? c_255_inv255_b() / d : 255.0f;
    } else {
        sc2 = q.s / 255.0f;
        inv2 = 255.0f / q.s;
    }
}

// Plane-2 code of one element before rounding (dacvae.c:656-660), for
// pack_codes4; v is the element's plane-1 code.
template <int CONV>
__device__ __forceinline__ float plane2_pre(float x, float v, const RowQ &r, float inv2) {
    const float rem = residual_value<CONV>(x, v, r);
    return CONV == 1 ? __builtin_fmaf(rem, inv2, 128.0f) : rem * inv2 + 128.0f;
}

}  // namespace
}  // namespace iro
