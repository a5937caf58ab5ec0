// iro_quant_row.h -- one activation row quantized by one wavefront
// (ops.c:321-348, two-term ops.c:427-442), shared by the quantization
// kernels (iro_quant.hip) and the persistent DiT stack kernel
// (iro_persist.hip).  Inline device code in an anonymous namespace.
#pragma once

#include "iro_internal.h"
#include "iro_round.h"

namespace iro {
namespace {

// Byte offset of the code of (row, col) in a code buffer: row-major with
// row pitch ldq, or, when ldq < 0, the MFMA fragment layout with -ldq k
// blocks per 32-row block: fragment (row / 32, col / 32) is 1 KiB, lane
// (row % 32) + 32 ((col / 16) % 2) holds columns col & ~15 .. +15, so a
// GEMM copies one fragment as one contiguous 1 KiB read.
__device__ __forceinline__ size_t code_off(int row, int col, int ldq) {
    if (ldq < 0)
        return ((size_t)((row >> 5) * -ldq + (col >> 5)) * 64 + (row & 31) + ((col >> 4) & 1) * 32) *
                   16 + (col & 15);
    return (size_t)row * ldq + col;
}

template <int CONV>
__device__ __forceinline__ uint32_t codes4(const float4 &v, const RowQ &r, float4 *vals) {
    const uint32_t w = pack_codes4(quant_pre<CONV>(v.x, r), quant_pre<CONV>(v.y, r),
                                   quant_pre<CONV>(v.z, r), quant_pre<CONV>(v.w, r));
    if (vals) *vals = unpack_codes4(w);
    return w;
}

// Vector path, one row held in registers as CH float4 per lane (lane L
// holds columns 4*(64c + L) .. +3 of chunk c).  EXACT: K == 256*CH, so no
// column is out of range.
template <int CH, bool EXACT>
__device__ __forceinline__ void load_row(const float *__restrict__ xr, int K, int lane,
                                         float4 (&v)[CH]) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int col = (c * 64 + lane) * 4;
        if (EXACT || col < K)
            v[c] = *reinterpret_cast<const float4 *>(xr + col);
        else
            v[c] = make_float4(0.f, 0.f, 0.f, 0.f);  // zero is inside every range
    }
}

// ops.c:321-348 (and, with RES, ops.c:427-442) on one row already in
// registers: range, codes (xor sflip), row scale and zero point; the
// two-term variant forms the remainder in place and quantizes it again.
// HALF: the row is held by one 32-lane half of the wavefront (K <= 128,
// lane counted within the half) and the reductions stay inside the half.
template <int CONV, int CH, bool RES, bool EXACT, bool HALF = false>
__device__ __forceinline__ void quant_row(float4 (&v)[CH], int row, int K, int lane,
                                          uint8_t *__restrict__ q1, int ldq,
                                          float *__restrict__ s1, int32_t *__restrict__ z1,
                                          float *__restrict__ res, uint8_t *__restrict__ q2,
                                          float *__restrict__ s2, int32_t *__restrict__ z2,
                                          uint32_t sflip) {
    float lo = 0.0f, hi = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        lo = sel_min(lo, v[c].x); lo = sel_min(lo, v[c].y);
        lo = sel_min(lo, v[c].z); lo = sel_min(lo, v[c].w);
        hi = sel_max(hi, v[c].x); hi = sel_max(hi, v[c].y);
        hi = sel_max(hi, v[c].z); hi = sel_max(hi, v[c].w);
    }
    lo = HALF ? half_range<false>(lo) : wave_min(lo);
    hi = HALF ? half_range<true>(hi) : wave_max(hi);
    const RowQ r = row_params<CONV>(lo, hi);
    float lo2 = 0.0f, hi2 = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int col = (c * 64 + lane) * 4;
        float4 qv;
        const uint32_t packed = codes4<CONV>(v[c], r, RES ? &qv : nullptr);
        if (EXACT || col < K)
            *reinterpret_cast<uint32_t *>(q1 + code_off(row, col, ldq)) = packed ^ sflip;
        if (RES) {
            if (EXACT || col < K) {
                v[c].x = residual_value<CONV>(v[c].x, qv.x, r);
                v[c].y = residual_value<CONV>(v[c].y, qv.y, r);
                v[c].z = residual_value<CONV>(v[c].z, qv.z, r);
                v[c].w = residual_value<CONV>(v[c].w, qv.w, r);
            }
            lo2 = sel_min(lo2, v[c].x); lo2 = sel_min(lo2, v[c].y);
            lo2 = sel_min(lo2, v[c].z); lo2 = sel_min(lo2, v[c].w);
            hi2 = sel_max(hi2, v[c].x); hi2 = sel_max(hi2, v[c].y);
            hi2 = sel_max(hi2, v[c].z); hi2 = sel_max(hi2, v[c].w);
        }
    }
    if (lane == 0) {
        s1[row] = r.s;
        z1[row] = r.zp;
    }
    if (RES) {
        lo2 = HALF ? half_range<false>(lo2) : wave_min(lo2);
        hi2 = HALF ? half_range<true>(hi2) : wave_max(hi2);
        const RowQ r2 = row_params<CONV>(lo2, hi2);
        float *rr = res ? res + (size_t)row * K : nullptr;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int col = (c * 64 + lane) * 4;
            const uint32_t packed = codes4<CONV>(v[c], r2, nullptr);
            if (EXACT || col < K) {
                *reinterpret_cast<uint32_t *>(q2 + code_off(row, col, ldq)) = packed ^ sflip;
                if (rr) *reinterpret_cast<float4 *>(rr + col) = v[c];
            }
        }
        if (lane == 0) {
            s2[row] = r2.s;
            z2[row] = r2.zp;
        }
    }
}

// quant_row with eight lanes per row (an aligned group of eight; `lane` is
// 0..7 within it): lane L holds columns 4*(8c + L) .. +3 for c < nch (nch
// the same in every lane, K == 32 nch), so every held column is in range
// and the reductions stay inside the group.  Same arithmetic, codes and
// row parameters as quant_row.
template <int CONV, int CHM, bool RES>
__device__ __forceinline__ void quant_row_g8(float4 (&v)[CHM], int nch, int row, int lane,
                                             uint8_t *__restrict__ q1, int ldq,
                                             float *__restrict__ s1, int32_t *__restrict__ z1,
                                             uint8_t *__restrict__ q2, float *__restrict__ s2,
                                             int32_t *__restrict__ z2, uint32_t sflip) {
    float lo = 0.0f, hi = 0.0f;
#pragma unroll
    for (int c = 0; c < CHM; ++c)
        if (c < nch) {
            lo = sel_min(lo, v[c].x); lo = sel_min(lo, v[c].y);
            lo = sel_min(lo, v[c].z); lo = sel_min(lo, v[c].w);
            hi = sel_max(hi, v[c].x); hi = sel_max(hi, v[c].y);
            hi = sel_max(hi, v[c].z); hi = sel_max(hi, v[c].w);
        }
    lo = group8_range<false>(lo);
    hi = group8_range<true>(hi);
    const RowQ r = row_params<CONV>(lo, hi);
    float lo2 = 0.0f, hi2 = 0.0f;
#pragma unroll
    for (int c = 0; c < CHM; ++c)
        if (c < nch) {
            const int col = (c * 8 + lane) * 4;
            float4 qv;
            const uint32_t packed = codes4<CONV>(v[c], r, RES ? &qv : nullptr);
            *reinterpret_cast<uint32_t *>(q1 + code_off(row, col, ldq)) = packed ^ sflip;
            if (RES) {
                v[c].x = residual_value<CONV>(v[c].x, qv.x, r);
                v[c].y = residual_value<CONV>(v[c].y, qv.y, r);
                v[c].z = residual_value<CONV>(v[c].z, qv.z, r);
                v[c].w = residual_value<CONV>(v[c].w, qv.w, r);
                lo2 = sel_min(lo2, v[c].x); lo2 = sel_min(lo2, v[c].y);
                lo2 = sel_min(lo2, v[c].z); lo2 = sel_min(lo2, v[c].w);
                hi2 = sel_max(hi2, v[c].x); hi2 = sel_max(hi2, v[c].y);
                hi2 = sel_max(hi2, v[c].z); hi2 = sel_max(hi2, v[c].w);
            }
        }
    if (lane == 0) {
        s1[row] = r.s;
        z1[row] = r.zp;
    }
    if (RES) {
        lo2 = group8_range<false>(lo2);
        hi2 = group8_range<true>(hi2);
        const RowQ r2 = row_params<CONV>(lo2, hi2);
#pragma unroll
        for (int c = 0; c < CHM; ++c)
            if (c < nch) {
                const int col = (c * 8 + lane) * 4;
                const uint32_t packed = codes4<CONV>(v[c], r2, nullptr);
                *reinterpret_cast<uint32_t *>(q2 + code_off(row, col, ldq)) = packed ^ sflip;
            }
        if (lane == 0) {
            s2[row] = r2.s;
            z2[row] = r2.zp;
        }
    }
}

}  // namespace
}  // namespace iro
