// iro_sincosf.h -- glibc's sinf and cosf, bit for bit, on gfx950.
//
// glibc 2.35 on x86-64 resolves sinf/cosf to the FMA build of ARM
// optimized-routines' sincosf method, which the reference's scalar code
// calls (the snake activations of dacvae.c:810-925, the timestep embedding
// of dit.c:486-499):
//   |x| < pi/4   an odd (sin) or even (cos) polynomial in double;
//   |x| < 120    n = round(x * 2/pi) through a 2^24-scaled product and an
//                integer shift, r = fma(-n, pi/2, x), then the polynomial of
//                quadrant n with its sign (the cosine coefficients negated for
//                n & 2);
//   larger |x|   a 32 x 96-bit product of the mantissa with 4/pi (a 192-bit
//                table, 8 new bits per word) gives the quadrant and a 2.62
//                fixed-point remainder, scaled by pi * 2^-62.
// Every "a + b * c" of the polynomials and of the fast reduction is one fma
// in that build; double operations on the device round as on the host, so
// the results are libm's (iro_hip_selfcheck_sincosf hashes all 2^32 inputs
// for comparison with the same hash of glibc's results).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace iro {
namespace {

// 4/pi in 192 bits; word i holds bits 8i .. 8i+31 of the expansion.
__constant__ uint32_t kInvPio4[24] = {
    0xa2,       0xa2f9,     0xa2f983,   0xa2f9836e, 0xf9836e4e, 0x836e4e44,
    0x6e4e4415, 0x4e441529, 0x441529fc, 0x1529fc27, 0x29fc2757, 0xfc2757d1,
    0x2757d1f5, 0x57d1f534, 0xd1f534dd, 0xf534ddc0, 0x34ddc0db, 0xddc0db62,
    0xc0db6295, 0xdb629599, 0x6295993c, 0x95993c43, 0x993c4390, 0x3c439041};

// The polynomial of quadrant k: sin (even k) or cos (odd k) of x, with
// x2 = x * x, in double, rounded to float.  glibc keeps a second table for
// quadrants 2 and 3 whose cosine coefficients are exactly the first's
// negated; negation commutes with every rounding, so `neg` negates the
// cosine result instead.  Both polynomials are formed from constants (no
// per-lane table loads) and the lane's one selected.  ad holds the two
// coefficients that enter a fused multiply-add as its addend (s2, c3).
struct SinCosAddends {
    double s2, c3;
};
constexpr SinCosAddends kSinCosAddends = {0x1.1107605230bc4p-7, -0x1.6c087e89a359dp-10};

// The addends in vector registers: a fused multiply-add reads at most one
// scalar operand, so with both operands constant each evaluation would first
// copy the addend into a register pair; a caller that evaluates several
// elements takes them from here once (the empty asm hides the values, so the
// copies are not re-created per element).
__device__ __forceinline__ SinCosAddends sincos_addends() {
    SinCosAddends ad = kSinCosAddends;
    asm("" : "+v"(ad.s2), "+v"(ad.c3));
    return ad;
}

__device__ __forceinline__ float sincos_poly_sel(double x, double x2, int k, bool neg,
                                                 const SinCosAddends &ad = kSinCosAddends) {
    constexpr double c0 = 0x1p0, c1 = -0x1.ffffffd0c621cp-2, c2 = 0x1.55553e1068f19p-5,
                     c4 = 0x1.99343027bf8c3p-16;
    constexpr double s1 = -0x1.555545995a603p-3, s3 = -0x1.994eb3774cf24p-13;
    const double s2 = ad.s2, c3 = ad.c3;
    const double x3 = x * x2;
    const double sp = __builtin_fma(x2, s3, s2);
    const double x7 = x3 * x2;
    const double sq = __builtin_fma(x3, s1, x);
    const float rs = (float)__builtin_fma(x7, sp, sq);
    const double x4 = x2 * x2;
    const double cp = __builtin_fma(x2, c4, c3);
    const double cq = __builtin_fma(x2, c1, c0);
    const double x6 = x4 * x2;
    const double cr = __builtin_fma(x4, c2, cq);
    float rc = (float)__builtin_fma(x6, cp, cr);
    rc = neg ? -rc : rc;
    return (k & 1) ? rc : rs;
}

// Whether y takes the fast reduction: |y| < 120 (NaN excluded).
__device__ __forceinline__ bool sincosf_is_small(float y) {
    return (__float_as_uint(y) & 0x7ff00000u) < 0x42f00000u;  // top 12 bits < 0x42f
}

// y reduced to x (double, |x| <= pi/4) in quadrant n; m is n plus the sign
// bit of y on the large path (n on the fast one): quadrant m & 3 gives the
// sign of x (+, -, -, +) and, for 2 and 3, the negated cosine.
struct SinCosArg {
    double x;
    int n, m;
};

// The fast reduction, for sincosf_is_small(y): n = round(y * 2/pi) through
// a 2^24-scaled product and an integer shift, x = fma(-n, pi/2, y).  Below
// pi/4 it gives n = 0 and x = y exactly, glibc's |y| < pi/4 case.  No
// branches, so callers can run several side by side.
__device__ __forceinline__ SinCosArg sincosf_reduce_small(float y) {
    const double x = y;
    const double r = x * 0x1.45F306DC9C883p+23;
    const int n = ((int32_t)r + 0x800000) >> 24;
    return {__builtin_fma(-(double)n, 0x1.921FB54442D18p0, x), n, n};
}

// The large reduction, for finite |y| >= 120 (other y give some SinCosArg
// that sincosf_finish replaces): a 32 x 96-bit product of the mantissa with
// 4/pi gives n and a 2.62 fixed-point remainder, scaled by pi * 2^-62.
// invpio4: kInvPio4 or a copy of it (in LDS, where a kernel stages one).
__device__ __forceinline__ SinCosArg sincosf_reduce_large(float y,
                                                          const uint32_t *invpio4 = kInvPio4) {
    const uint32_t yi = __float_as_uint(y);
    const uint32_t *arr = &invpio4[(yi >> 26) & 15];
    const int shift = (yi >> 23) & 7;
    uint32_t xi = ((yi & 0xffffff) | 0x800000) << shift;
    uint64_t res0 = (uint32_t)(xi * arr[0]);
    const uint64_t res1 = (uint64_t)xi * arr[4];
    const uint64_t res2 = (uint64_t)xi * arr[8];
    res0 = (res2 >> 32) | (res0 << 32);
    res0 += res1;
    const uint64_t nn = (res0 + (1ull << 61)) >> 62;
    res0 -= nn << 62;
    const int n = (int)nn;
    return {(double)(int64_t)res0 * 0x1.921FB54442D18p-62, n, n + (int)(yi >> 31)};
}

// cosine = 0: sinf(y); 1: cosf(y) from y's reduction: the quadrant's
// polynomial, or glibc's own result for |y| < 2^-12 (y, or 1) and for
// non-finite y (NaN).
__device__ __forceinline__ float sincosf_finish(float y, const SinCosArg &a, int cosine,
                                                const SinCosAddends &ad = kSinCosAddends) {
    // x negated when bit 1 of m + 1 is set: that bit moved to the sign bit
    const uint64_t flip = (uint64_t)(((uint32_t)(a.m + 1) << 30) & 0x80000000u) << 32;
    const double xs = __builtin_bit_cast(double, __builtin_bit_cast(uint64_t, a.x) ^ flip);
    const float v = sincos_poly_sel(xs, a.x * a.x, a.n ^ cosine, (a.m & 2) != 0, ad);
    const uint32_t top = __float_as_uint(y) & 0x7ff00000u;  // top 12 bits, in place
    if (top >= 0x7f800000u) return (y - y) / (y - y);
    return top < 0x39800000u ? (cosine ? 1.0f : y) : v;
}

// cosine = 0: sinf(y); 1: cosf(y), every float y.
__device__ __forceinline__ float sincosf_glibc(float y, int cosine) {
    const SinCosArg a = __builtin_expect(sincosf_is_small(y), 1) ? sincosf_reduce_small(y)
                                                                  : sincosf_reduce_large(y);
    return sincosf_finish(y, a, cosine);
}

__device__ __forceinline__ float sinf_glibc(float y) { return sincosf_glibc(y, 0); }
__device__ __forceinline__ float cosf_glibc(float y) { return sincosf_glibc(y, 1); }

}  // namespace
}  // namespace iro
