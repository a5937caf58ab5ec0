// iro_expf.h -- glibc's expf, bit for bit, on gfx950.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace iro {
namespace {

// expf as glibc >= 2.28 computes it on x86-64 with FMA (the __expf_fma
// ifunc variant the reference's libm call resolves to): the published
// exp2f table method of ARM optimized-routines, N = 32:
//   x*N/ln2 = k + r,  exp(x) = 2^(k/N) * (1 + C2 r + C1 r^2 + C0 r^3),
// in double, with GCC's contraction of both uses of InvLn2N*x into FMAs.
// Bit-identical to glibc's expf for every float input.  The 2^(i/32)
// table is copied into LDS by the kernels that use it.
__constant__ uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

// Branch-free: the table path runs on x clamped into its domain (the clamp
// is the identity there; a NaN x takes whatever value the median gives, the
// table index stays in range, and the result is replaced) and the special
// cases are selected afterwards, so a wavefront never splits on them.  The
// scale 2^(k/32) is built in 32-bit halves: (k << 47) only touches the high
// word of the table entry.
constexpr float kExpfHi = 0x1.62e42ep6f, kExpfLo = -0x1.9fe368p6f;  // overflow / underflow bounds

// The table path alone, on x clamped into [kExpfLo, kExpfHi]: expf(x) for
// every x in that range; outside it (and for NaN) the callers select.
__device__ __forceinline__ float expf_glibc_table(float x, const uint64_t *tab) {
    const float xc = __builtin_amdgcn_fmed3f(x, kExpfLo, kExpfHi);
    const double invln2n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)xc;
    double kd = __builtin_fma(invln2n, xd, shift);
    const uint32_t klo = (uint32_t)__double_as_longlong(kd);
    kd -= shift;
    const double r = __builtin_fma(invln2n, xd, -kd);
    const uint64_t tv = tab[klo & 31];
    const uint32_t thi = (uint32_t)(tv >> 32) + (klo << 15);
    const double s = __hiloint2double((int)thi, (int)(uint32_t)tv);
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    return (float)(y * s);
}

__device__ __forceinline__ float expf_glibc(float x, const uint64_t *tab) {
    float e = expf_glibc_table(x, tab);
    e = x > kExpfHi ? __builtin_inff() : e;  // overflow
    e = x < kExpfLo ? 0.0f : e;              // underflow (and -inf)
    return x != x ? x + x : e;
}

}  // namespace
}  // namespace iro
