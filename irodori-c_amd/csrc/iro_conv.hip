// iro_conv.hip -- the DACVAE int8 Conv1d (dacvae.c:543-688) as an implicit
// GEMM: quantized im2col rows, then the MFMA GEMM of iro_gemm.hip; and the
// scatter-add tail of the int8 ConvTranspose1d (dacvae.c:696-795), whose
// GEMM is the plain linear of iro_gemm.hip.
//
// Quantization is per OUTPUT time step over its whole kernel*C window
// (dacvae.c:617-636): each input element is coded under up to `kernel`
// different (scale, zero point) pairs, so the codes cannot be produced once
// per input row.  Two passes:
//   conv_rows    per input time step lo/hi over channels (dacvae.c:607-616),
//                one wavefront per row;
//   conv_im2col  per output time step: window lo/hi from the tap rows that
//                fall inside [0, T), the row scale/zero point, and the u8
//                im2col row [tap*C + c] (padding taps hold the zero point);
//                with `residual`, the second plane with scale s/255 and zero
//                point 128 (dacvae.c:637-663).
// Roofline: HBM.  conv_im2col reads kernel*C*4 bytes (mostly L2 hits: the
// taps of neighbouring rows overlap) and writes kernel*C (x2) bytes per row.
#include "iro_internal.h"
#include "iro_conv_row.h"

namespace iro {

namespace {

__global__ __launch_bounds__(256) void conv_rows_kernel(const float *__restrict__ x, int T, int C,
                                                        float *__restrict__ row_lo,
                                                        float *__restrict__ row_hi) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (t >= T) return;
    const float *xr = x + (size_t)t * C;
    float lo = 0.0f, hi = 0.0f;
    if ((C & 3) == 0) {
        for (int c = lane * 4; c < C; c += 256) {
            const float4 v = *reinterpret_cast<const float4 *>(xr + c);
            lo = sel_min(lo, v.x); lo = sel_min(lo, v.y); lo = sel_min(lo, v.z); lo = sel_min(lo, v.w);
            hi = sel_max(hi, v.x); hi = sel_max(hi, v.y); hi = sel_max(hi, v.z); hi = sel_max(hi, v.w);
        }
    } else {
        for (int c = lane; c < C; c += 64) {
            lo = sel_min(lo, xr[c]);
            hi = sel_max(hi, xr[c]);
        }
    }
    lo = wave_min(lo);
    hi = wave_max(hi);
    if (lane == 0) {
        row_lo[t] = lo;
        row_hi[t] = hi;
    }
}

// Plane-2 code of one element (dacvae.c:656-660).
template <int CONV>
__device__ __forceinline__ uint32_t plane2_code(float x, float v, const RowQ &r, float inv2) {
    const float rem = residual_value<CONV>(x, v, r);
    float v2 = CONV == 1 ? __builtin_rintf(__builtin_fmaf(rem, inv2, 128.0f))
                         : __builtin_rintf(rem * inv2 + 128.0f);
    v2 = v2 < 0.0f ? 0.0f : v2;
    v2 = v2 > 255.0f ? 255.0f : v2;
    return (uint32_t)v2;
}

template <int CONV, bool RES>
__global__ __launch_bounds__(256) void conv_im2col_kernel(
    const float *__restrict__ x, int T, int C, int T_out, int kernel, int stride, int dilation,
    int padding, const float *__restrict__ row_lo, const float *__restrict__ row_hi,
    uint8_t *__restrict__ cols1, uint8_t *__restrict__ cols2, int ldc, float *__restrict__ s1,
    int32_t *__restrict__ z1, float *__restrict__ s2, int32_t *__restrict__ z2) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= T_out) return;
    // Window range: taps inside [0, T) only (dacvae.c:619-627).
    float lo = 0.0f, hi = 0.0f;
    for (int tap = 0; tap < kernel; ++tap) {
        const int it = r * stride - padding + tap * dilation;
        if (it < 0 || it >= T) continue;
        lo = sel_min(lo, row_lo[it]);
        hi = sel_max(hi, row_hi[it]);
    }
    const RowQ q = row_params<CONV>(lo, hi);
    float sc2 = 0.0f, inv2 = 0.0f;
    if (RES) conv_plane2_params<CONV>(q, lo, hi, sc2, inv2);
    uint8_t *d1 = cols1 + (size_t)r * ldc;
    uint8_t *d2 = RES ? cols2 + (size_t)r * ldc : nullptr;
    const uint32_t zp4 = 0x01010101u * (uint32_t)q.zp;
    const uint32_t h4 = 0x80808080u;
    for (int tap = 0; tap < kernel; ++tap) {
        const int it = r * stride - padding + tap * dilation;
        uint8_t *t1 = d1 + (size_t)tap * C;
        uint8_t *t2 = RES ? d2 + (size_t)tap * C : nullptr;
        const bool inside = it >= 0 && it < T;
        const float *xr = x + (size_t)(inside ? it : 0) * C;
        if ((C & 3) == 0 && (ldc & 3) == 0) {
            for (int c = lane * 4; c < C; c += 256) {
                if (!inside) {
                    *reinterpret_cast<uint32_t *>(t1 + c) = zp4;
                    if (RES) *reinterpret_cast<uint32_t *>(t2 + c) = h4;
                    continue;
                }
                const float4 v = *reinterpret_cast<const float4 *>(xr + c);
                const float a = quant_value<CONV>(v.x, q), b = quant_value<CONV>(v.y, q);
                const float e = quant_value<CONV>(v.z, q), f = quant_value<CONV>(v.w, q);
                *reinterpret_cast<uint32_t *>(t1 + c) = pack_codes4(a, b, e, f);
                if (RES) {
                    *reinterpret_cast<uint32_t *>(t2 + c) =
                        plane2_code<CONV>(v.x, a, q, inv2) | (plane2_code<CONV>(v.y, b, q, inv2) << 8) |
                        (plane2_code<CONV>(v.z, e, q, inv2) << 16) |
                        (plane2_code<CONV>(v.w, f, q, inv2) << 24);
                }
            }
        } else {
            for (int c = lane; c < C; c += 64) {
                if (!inside) {
                    t1[c] = (uint8_t)q.zp;
                    if (RES) t2[c] = 128;
                    continue;
                }
                const float v = quant_value<CONV>(xr[c], q);
                t1[c] = (uint8_t)v;
                if (RES) t2[c] = (uint8_t)plane2_code<CONV>(xr[c], v, q, inv2);
            }
        }
    }
    if (lane == 0) {
        s1[r] = q.s;
        z1[r] = q.zp;
        if (RES) {
            s2[r] = sc2;
            z2[r] = 128;
        }
    }
}

// Kernel-7 convolutions with C <= 1024 (every Conv7 of the decoder) in one
// pass: the wavefront of output step r loads its seven tap rows into
// registers (CHN float4 per lane per tap, all loads in flight at once),
// reduces the window's lo/hi itself -- min(0, window) and max(0, window)
// equal the reference's min over the taps' row ranges (dacvae.c:607-627),
// whatever the order, since both only select -- and codes the rows from
// registers.  Taps outside [0, T) load nothing and hold the zero point.
// flip: XOR applied to every stored code word (0x80808080 stores the
// signed operand form a - 128 the LDS-pipelined GEMM reads, 0 keeps u8).
// Workgroup w runs on XCD w % 8; XCD x takes the contiguous run of row
// blocks x*per .. x*per + per - 1, so the tap rows neighbouring blocks
// share are read through one L2.
constexpr int kIm2colRows = 4;  // output steps (wavefronts) per workgroup

// CHN == 0 (C <= 128): each 32-lane half of a wavefront takes its own
// output step, so narrow rows fill the lanes.
template <int CONV, bool RES, int CHN0>
__global__ __launch_bounds__(64 * kIm2colRows) void conv_im2col7_kernel(
    const float *__restrict__ x, int T, int C, int T_out, int stride, int dilation, int padding,
    uint8_t *__restrict__ cols1, uint8_t *__restrict__ cols2, int ldc, float *__restrict__ s1,
    int32_t *__restrict__ z1, float *__restrict__ s2, int32_t *__restrict__ z2, uint32_t flip,
    int per) {
    constexpr int KT = 7;
    constexpr bool HALF = CHN0 == 0;
    constexpr int CHN = HALF ? 1 : CHN0;
    const int blk = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    const int r = HALF ? (blk * kIm2colRows + (threadIdx.x >> 6)) * 2 + ((threadIdx.x >> 5) & 1)
                       : blk * kIm2colRows + (threadIdx.x >> 6);
    const int lane = threadIdx.x & (HALF ? 31 : 63);
    if (r >= T_out) return;
    float4 v[KT][CHN];
    bool inside[KT];
#pragma unroll
    for (int tap = 0; tap < KT; ++tap) {
        const int it = r * stride - padding + tap * dilation;
        inside[tap] = it >= 0 && it < T;
        const float *xr = x + (size_t)(inside[tap] ? it : 0) * C;
#pragma unroll
        for (int j = 0; j < CHN; ++j) {
            const int c = j * 256 + lane * 4;
            v[tap][j] = inside[tap] && c < C ? *reinterpret_cast<const float4 *>(xr + c)
                                             : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
    float lo = 0.0f, hi = 0.0f;
#pragma unroll
    for (int tap = 0; tap < KT; ++tap)
#pragma unroll
        for (int j = 0; j < CHN; ++j) {
            const float4 e = v[tap][j];
            lo = sel_min(lo, e.x); lo = sel_min(lo, e.y); lo = sel_min(lo, e.z); lo = sel_min(lo, e.w);
            hi = sel_max(hi, e.x); hi = sel_max(hi, e.y); hi = sel_max(hi, e.z); hi = sel_max(hi, e.w);
        }
    lo = HALF ? half_range<false>(lo) : wave_min(lo);
    hi = HALF ? half_range<true>(hi) : wave_max(hi);
    const RowQ q = row_params<CONV>(lo, hi);
    float sc2 = 0.0f, inv2 = 0.0f;
    if (RES) conv_plane2_params<CONV>(q, lo, hi, sc2, inv2);
    const uint32_t zp4 = (0x01010101u * (uint32_t)q.zp) ^ flip;
    const uint32_t h4 = 0x80808080u ^ flip;
    uint8_t *d1 = cols1 + (size_t)r * ldc;
    uint8_t *d2 = RES ? cols2 + (size_t)r * ldc : nullptr;
#pragma unroll
    for (int tap = 0; tap < KT; ++tap)
#pragma unroll
        for (int j = 0; j < CHN; ++j) {
            const int c = j * 256 + lane * 4;
            if (c >= C) continue;
            const size_t o = (size_t)tap * C + c;
            if (!inside[tap]) {
                *reinterpret_cast<uint32_t *>(d1 + o) = zp4;
                if (RES) *reinterpret_cast<uint32_t *>(d2 + o) = h4;
                continue;
            }
            const float4 e = v[tap][j];
            const uint32_t w1 = pack_codes4(quant_pre<CONV>(e.x, q), quant_pre<CONV>(e.y, q),
                                            quant_pre<CONV>(e.z, q), quant_pre<CONV>(e.w, q));
            *reinterpret_cast<uint32_t *>(d1 + o) = w1 ^ flip;
            if (RES) {
                const float4 c4 = unpack_codes4(w1);
                *reinterpret_cast<uint32_t *>(d2 + o) =
                    pack_codes4(plane2_pre<CONV>(e.x, c4.x, q, inv2),
                                plane2_pre<CONV>(e.y, c4.y, q, inv2),
                                plane2_pre<CONV>(e.z, c4.z, q, inv2),
                                plane2_pre<CONV>(e.w, c4.w, q, inv2)) ^
                    flip;
            }
        }
    if (lane == 0) {
        s1[r] = q.s;
        z1[r] = q.zp;
        if (RES) {
            s2[r] = sc2;
            z2[r] = 128;
        }
    }
}

// ConvTranspose1d tail (dacvae.c:708-712, 779-790): y[t, c] = bias[c] plus,
// for every input row r whose taps reach t (tap = t + padding - r*stride in
// [0, kernel)), expanded[r, tap*C_out + c], added in ascending r exactly as
// the reference's scatter loop visits them.  A gather: one thread per four
// output channels of one time step, no atomics, so the order is fixed.
template <bool VEC>
__global__ __launch_bounds__(256) void convt_gather_kernel(const float *__restrict__ expanded,
                                                           int T_in, int C_out, int kernel,
                                                           int stride, int padding, int T_out,
                                                           const float *__restrict__ bias,
                                                           float *__restrict__ y) {
    const int groups = VEC ? C_out / 4 : C_out;
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (long long)T_out * groups) return;
    const int t = (int)(idx / groups);
    const int c = (int)(idx - (long long)t * groups) * (VEC ? 4 : 1);
    const int num = t + padding - kernel + 1;
    int r = num <= 0 ? 0 : (num + stride - 1) / stride;
    int r_hi = (t + padding) / stride;
    r_hi = r_hi < T_in - 1 ? r_hi : T_in - 1;
    const size_t ncols = (size_t)kernel * C_out;
    if (VEC) {
        float4 acc = bias ? *reinterpret_cast<const float4 *>(bias + c) : make_float4(0.f, 0.f, 0.f, 0.f);
        for (; r <= r_hi; ++r) {
            const int tap = t + padding - r * stride;
            const float4 e =
                *reinterpret_cast<const float4 *>(expanded + (size_t)r * ncols + (size_t)tap * C_out + c);
            acc.x += e.x;
            acc.y += e.y;
            acc.z += e.z;
            acc.w += e.w;
        }
        *reinterpret_cast<float4 *>(y + (size_t)t * C_out + c) = acc;
    } else {
        float acc = bias ? bias[c] : 0.0f;
        for (; r <= r_hi; ++r) {
            const int tap = t + padding - r * stride;
            acc += expanded[(size_t)r * ncols + (size_t)tap * C_out + c];
        }
        y[(size_t)t * C_out + c] = acc;
    }
}

}  // namespace

int launch_convt_gather(IroHipContext *ctx, const float *expanded, int T_in, int C_out,
                        int kernel, int stride, int padding, int T_out, const float *bias,
                        float *y) {
    const bool vec = C_out % 4 == 0 && (((uintptr_t)expanded | (uintptr_t)y) & 15) == 0 &&
                     (!bias || (((uintptr_t)bias) & 15) == 0);
    const long long n = (long long)T_out * (vec ? C_out / 4 : C_out);
    const dim3 grid((unsigned)((n + 255) / 256)), block(256);
    prof_begin(ctx);
    if (vec)
        hipLaunchKernelGGL((convt_gather_kernel<true>), grid, block, 0, ctx->stream, expanded, T_in,
                           C_out, kernel, stride, padding, T_out, bias, y);
    else
        hipLaunchKernelGGL((convt_gather_kernel<false>), grid, block, 0, ctx->stream, expanded,
                           T_in, C_out, kernel, stride, padding, T_out, bias, y);
    IRO_HIP_CHECK_LAUNCH(ctx);
    // Each expanded value is read once, each output written once.
    prof_end(ctx, PK_CONVT_GATHER, 0, 4.0 * T_in * kernel * C_out + 4.0 * T_out * C_out);
    return 0;
}

int launch_conv_rows(IroHipContext *ctx, const float *x, int T, int C, float *lo, float *hi) {
    prof_begin(ctx);
    hipLaunchKernelGGL(conv_rows_kernel, dim3((T + 3) / 4), dim3(256), 0, ctx->stream, x, T, C, lo,
                       hi);
    IRO_HIP_CHECK_LAUNCH(ctx);
    prof_end(ctx, PK_CONV_ROWS, 0, 4.0 * T * C + 8.0 * T);
    return 0;
}

bool conv_im2col7_ok(int C, int kernel, int ldc) {
    return kernel == 7 && C % 4 == 0 && C <= 1024 && ldc % 4 == 0;
}

int launch_conv_im2col7(IroHipContext *ctx, const float *x, int T, int C, int T_out, int stride,
                        int dilation, int padding, uint8_t *cols1, uint8_t *cols2, int ldc,
                        float *s1, int32_t *z1, float *s2, int32_t *z2, bool signed_codes) {
    const uint32_t flip = signed_codes ? 0x80808080u : 0u;
    const int chn = C <= 128 ? 0 : (C + 255) / 256;
    const int rows_per_block = kIm2colRows * (chn == 0 ? 2 : 1);
    const int per = ((T_out + rows_per_block - 1) / rows_per_block + 7) / 8;  // row blocks per XCD
    const dim3 grid(8 * per), block(64 * kIm2colRows);
    const bool res = cols2 != nullptr;
    prof_begin(ctx);
#define IRO_IM2COL7(CV, RS, CH)                                                                 \
    hipLaunchKernelGGL((conv_im2col7_kernel<CV, RS, CH>), grid, block, 0, ctx->stream, x, T, C, \
                       T_out, stride, dilation, padding, cols1, cols2, ldc, s1, z1, s2, z2, flip, per)
#define IRO_IM2COL7_C(CV, RS)          \
    switch (chn) {                     \
        case 0: IRO_IM2COL7(CV, RS, 0); break; \
        case 1: IRO_IM2COL7(CV, RS, 1); break; \
        case 2: IRO_IM2COL7(CV, RS, 2); break; \
        case 3: IRO_IM2COL7(CV, RS, 3); break; \
        default: IRO_IM2COL7(CV, RS, 4); break; \
    }
    if (ctx->convention == IRO_HIP_GCC_FASTMATH) {
        if (res) { IRO_IM2COL7_C(1, true); } else { IRO_IM2COL7_C(1, false); }
    } else {
        if (res) { IRO_IM2COL7_C(0, true); } else { IRO_IM2COL7_C(0, false); }
    }
#undef IRO_IM2COL7_C
#undef IRO_IM2COL7
    IRO_HIP_CHECK_LAUNCH(ctx);
    // Algorithmic HBM bytes: the input once, the code plane(s) out.
    prof_end(ctx, PK_CONV_IM2COL, 0,
             4.0 * T * C + (res ? 2.0 : 1.0) * ((double)T_out * 7 * C + 8.0 * T_out));
    return 0;
}

int launch_conv_im2col(IroHipContext *ctx, const float *x, int T, int C, int T_out, int kernel,
                       int stride, int dilation, int padding, const float *row_lo,
                       const float *row_hi, uint8_t *cols1, uint8_t *cols2, int ldc, float *s1,
                       int32_t *z1, float *s2, int32_t *z2) {
    const dim3 grid((T_out + 3) / 4), block(256);
    const bool res = cols2 != nullptr;
    prof_begin(ctx);
#define IRO_IM2COL(CV, RS)                                                                     \
    hipLaunchKernelGGL((conv_im2col_kernel<CV, RS>), grid, block, 0, ctx->stream, x, T, C, T_out, \
                       kernel, stride, dilation, padding, row_lo, row_hi, cols1, cols2, ldc, s1, \
                       z1, s2, z2)
    if (ctx->convention == IRO_HIP_GCC_FASTMATH) {
        if (res) IRO_IM2COL(1, true);
        else IRO_IM2COL(1, false);
    } else {
        if (res) IRO_IM2COL(0, true);
        else IRO_IM2COL(0, false);
    }
#undef IRO_IM2COL
    IRO_HIP_CHECK_LAUNCH(ctx);
    // Algorithmic HBM bytes: the input once, the code plane(s) out.
    prof_end(ctx, PK_CONV_IM2COL, 0,
             4.0 * T * C + (res ? 2.0 : 1.0) * ((double)T_out * kernel * C + 8.0 * T_out));
    return 0;
}

}  // namespace iro
