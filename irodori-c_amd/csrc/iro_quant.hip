// iro_quant.hip -- per-row activation quantization, per-output-row weight
// quantization and MFMA pre-packing for gfx950.
//
// Activations (ops.c:321-348, ops.c:427-442): one 64-lane wavefront per
// row.  Codes are u8 as the reference stores them, or, for buffers only the
// GEMM reads, the same codes with the top bit flipped (a ^ 0x80 = a - 128
// as s8), the operand form of the signed int8 MFMA.  The row is read once into registers (CH float4 per lane, coalesced
// 1 KiB per wave instruction), min/max are wave reductions, and the codes
// are written as one u32 (4 codes) per lane per chunk.  The two-term
// variant keeps the row in registers, forms the remainder in place and
// quantizes it again, so the input is read from HBM exactly once.
// Roofline: HBM, 4K + K (+K) + 8 bytes per row.
#include "iro_quant_row.h"
#include "iro_snake.h"

namespace iro {

namespace {

// Vector path: K % 4 == 0, 16-byte aligned rows, K <= 256*CH (EXACT:
// K == 256*CH); one wavefront per row.
template <int CONV, int CH, bool RES, bool EXACT>
__global__ __launch_bounds__(256) void quant_rows_vec(const float *__restrict__ x, int M, int K,
                                                      int ldx, uint8_t *__restrict__ q1, int ldq,
                                                      float *__restrict__ s1,
                                                      int32_t *__restrict__ z1,
                                                      float *__restrict__ res,
                                                      uint8_t *__restrict__ q2,
                                                      float *__restrict__ s2,
                                                      int32_t *__restrict__ z2, uint32_t sflip) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M) return;
    float4 v[CH];
    load_row<CH, EXACT>(x + (size_t)row * ldx, K, lane, v);
    quant_row<CONV, CH, RES, EXACT>(v, row, K, lane, q1, ldq, s1, z1, res, q2, s2, z2, sflip);
}

// Narrow rows (K <= 128, the vector path's conditions otherwise): each
// 32-lane half of a wavefront holds one row, eight rows per block.
template <int CONV, bool RES>
__global__ __launch_bounds__(256) void quant_rows_half(const float *__restrict__ x, int M, int K,
                                                       int ldx, uint8_t *__restrict__ q1, int ldq,
                                                       float *__restrict__ s1,
                                                       int32_t *__restrict__ z1,
                                                       float *__restrict__ res,
                                                       uint8_t *__restrict__ q2,
                                                       float *__restrict__ s2,
                                                       int32_t *__restrict__ z2, uint32_t sflip) {
    const int row = blockIdx.x * 8 + (threadIdx.x >> 5);
    const int lane = threadIdx.x & 31;
    if (row >= M) return;
    float4 v[1];
    load_row<1, false>(x + (size_t)row * ldx, K, lane, v);
    quant_row<CONV, 1, RES, false, true>(v, row, K, lane, q1, ldq, s1, z1, res, q2, s2, z2, sflip);
}

// The residual unit's in-place snake of conv0's biased output
// (snake_bias_forward, dacvae.c:910-931, called at dacvae.c:967-968) fused
// into the quantization of the 1x1 projection's input rows, the snaked rows'
// only reader (dacvae.c:983-1012): they never reach HBM.  Reciprocal form
// only (K <= 1536).  A block takes R rows.  Phase 1 reads them as flat
// float4 chunks, so every lane works whatever K is (the decoder's 3 * 2^k
// channels would leave a quarter of a row-per-wave layout idle), snakes them
// with per-channel bias, alpha and reciprocal staged in LDS, and writes the
// tile [R, K] to LDS.  Phase 2 quantizes the tile's rows as quant_rows_vec
// (HALF: quant_rows_half) does.  Dynamic LDS: 3 K + R K floats.
template <int CONV, int CH, bool RES, bool HALF, bool BIAS, bool G8>
__global__ __launch_bounds__(256) void quant_rows_snake(const float *__restrict__ x, int M, int K,
                                                        int ldx, int R, unsigned k4_magic,
                                                        const float *__restrict__ bias,
                                                        const float *__restrict__ alpha,
                                                        uint8_t *__restrict__ q1, int ldq,
                                                        float *__restrict__ s1,
                                                        int32_t *__restrict__ z1,
                                                        uint8_t *__restrict__ q2,
                                                        float *__restrict__ s2,
                                                        int32_t *__restrict__ z2, uint32_t sflip) {
    static_assert(!HALF || CH == 1, "a half-wave row holds at most 128 columns");
    extern __shared__ __attribute__((aligned(16))) float snake_lds[];
    __shared__ uint32_t s_pio4[24];
    float *s_b = snake_lds, *s_a = s_b + K, *s_i = s_a + K, *tile = s_i + K;
    stage_invpio4(s_pio4, threadIdx.x);
    for (int c = threadIdx.x; c < K; c += 256) {
        const float a = alpha[c];
        s_b[c] = BIAS ? bias[c] : 0.0f;
        s_a[c] = a;
        s_i[c] = snake_inv(a);
    }
    const int row0 = blockIdx.x * R;
    const int rows = min(R, M - row0);
    const int k4 = K >> 2, chunks = rows * k4;
    // Phase 1: at most 4 chunks per thread (R K <= 4096); loads first.
    float4 v4[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int f = threadIdx.x + 256 * j;
        if (f < chunks) {
            const int r = __umulhi(2u * f, k4_magic), c4 = f - r * k4;
            v4[j] = *reinterpret_cast<const float4 *>(x + (size_t)(row0 + r) * ldx + 4 * c4);
        }
    }
    __syncthreads();  // the staged parameters
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int f = threadIdx.x + 256 * j;
        if (f < chunks) {
            const int r = __umulhi(2u * f, k4_magic), c4 = f - r * k4;
            const float4 b = *reinterpret_cast<const float4 *>(s_b + 4 * c4);
            const float4 a = *reinterpret_cast<const float4 *>(s_a + 4 * c4);
            const float4 i = *reinterpret_cast<const float4 *>(s_i + 4 * c4);
            // No bias (the snake before an upsample): the rows as they are
            // (adding 0 would turn -0 into +0).
            const float4 xv = BIAS ? make_float4(v4[j].x + b.x, v4[j].y + b.y, v4[j].z + b.z,
                                                 v4[j].w + b.w)
                                   : v4[j];
            *reinterpret_cast<float4 *>(tile + r * K + 4 * c4) =
                snake_value4<true, CONV == 1>(xv, a, i, s_pio4);
        }
    }
    __syncthreads();
    if (G8) {
        // Phase 2 with eight lanes per row (32 rows per pass), K / 32 float4
        // per lane (K a multiple of 32, at most 256).
        const int sub = threadIdx.x & 7, nch = K >> 5;
        for (int r = threadIdx.x >> 3; r < rows; r += 32) {
            float4 v[8];
#pragma unroll
            for (int c = 0; c < 8; ++c)
                v[c] = c < nch ? *reinterpret_cast<const float4 *>(tile + r * K + (c * 8 + sub) * 4)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
            quant_row_g8<CONV, 8, RES>(v, nch, row0 + r, sub, q1, ldq, s1, z1, q2, s2, z2, sflip);
        }
        return;
    }
    // Phase 2: rows of the tile, one per wave (HALF: per 32-lane half).
    constexpr int WL = HALF ? 32 : 64, RPB = 256 / WL;
    const int lane = threadIdx.x & (WL - 1);
    for (int r = threadIdx.x / WL; r < rows; r += RPB) {
        float4 v[CH];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int col = (c * 64 + lane) * 4;
            v[c] = col < K ? *reinterpret_cast<const float4 *>(tile + r * K + col)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        quant_row<CONV, CH, RES, false, HALF>(v, row0 + r, K, lane, q1, ldq, s1, z1, nullptr, q2,
                                              s2, z2, sflip);
    }
}

// Generic path: any K and alignment; the row is re-read from cache.
template <int CONV, bool RES>
__global__ __launch_bounds__(256) void quant_rows_any(const float *__restrict__ x, int M, int K,
                                                      int ldx, uint8_t *__restrict__ q1, int ldq,
                                                      float *__restrict__ s1,
                                                      int32_t *__restrict__ z1,
                                                      float *__restrict__ res,
                                                      uint8_t *__restrict__ q2,
                                                      float *__restrict__ s2,
                                                      int32_t *__restrict__ z2, uint32_t sflip) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M) return;
    const float *xr = x + (size_t)row * ldx;
    const uint8_t fb = (uint8_t)(sflip & 0xff);
    float lo = 0.0f, hi = 0.0f;
    for (int k = lane; k < K; k += 64) {
        lo = sel_min(lo, xr[k]);
        hi = sel_max(hi, xr[k]);
    }
    lo = wave_min(lo);
    hi = wave_max(hi);
    const RowQ r = row_params<CONV>(lo, hi);
    float lo2 = 0.0f, hi2 = 0.0f;
    for (int k = lane; k < K; k += 64) {
        const float v = quant_value<CONV>(xr[k], r);
        q1[code_off(row, k, ldq)] = (uint8_t)v ^ fb;
        if (RES) {
            const float rv = residual_value<CONV>(xr[k], v, r);
            lo2 = sel_min(lo2, rv);
            hi2 = sel_max(hi2, rv);
        }
    }
    if (lane == 0) {
        s1[row] = r.s;
        z1[row] = r.zp;
    }
    if (RES) {
        lo2 = wave_min(lo2);
        hi2 = wave_max(hi2);
        const RowQ r2 = row_params<CONV>(lo2, hi2);
        for (int k = lane; k < K; k += 64) {
            const float rv =
                residual_value<CONV>(xr[k], (float)(uint8_t)(q1[code_off(row, k, ldq)] ^ fb), r);
            q2[code_off(row, k, ldq)] = (uint8_t)quant_value<CONV>(rv, r2) ^ fb;
            if (res) res[(size_t)row * K + k] = rv;
        }
        if (lane == 0) {
            s2[row] = r2.s;
            z2[row] = r2.zp;
        }
    }
}

// ops.c:259-293: one wave per output row.  Source element (n, k) is
// w[n*stride_n + k*stride_k] so the [K,N] source of ops.c:295-306 needs no
// transposed copy.
template <int CONV>
__global__ __launch_bounds__(256) void weight_quant_kernel(const float *__restrict__ w, int N,
                                                           int K, long long stride_n,
                                                           long long stride_k,
                                                           int8_t *__restrict__ q,
                                                           float *__restrict__ scale,
                                                           int32_t *__restrict__ colsum) {
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (n >= N) return;
    const float *wr = w + n * stride_n;
    float amax = 0.0f;
    for (int k = lane; k < K; k += 64) {
        const float a = fabsf(wr[k * stride_k]);
        amax = a > amax ? a : amax;
    }
    amax = wave_max(amax);
    float s, inv;
    if (CONV == 1) {
        if (amax > 0.0f) {
            s = amax * c_inv127();
            inv = 127.0f / amax;
        } else {
            s = 1.0f;
            inv = 1.0f;
        }
    } else {
        s = amax > 0.0f ? amax / 127.0f : 1.0f;
        inv = 1.0f / s;
    }
    int sum = 0;
    int8_t *qr = q + (size_t)n * K;
    for (int k = lane; k < K; k += 64) {
        const int v = clampi((int)__builtin_rintf(wr[k * stride_k] * inv), -127, 127);
        qr[k] = (int8_t)v;
        sum += v;
    }
    sum = wave_sum(sum);
    if (lane == 0) {
        scale[n] = s;
        colsum[n] = sum;
    }
}

// Logical row of packed 32-row block `pb` (see IroHipWeight), or -1.
__device__ __forceinline__ int packed_block_source(int pb, int layout, int half_blocks) {
    if (layout == 1) {
        const int t = pb >> 1;
        if (t >= half_blocks) return -1;
        return (pb & 1) ? half_blocks + t : t;
    }
    return pb;
}

// One thread per 16-byte chunk of the packed buffer.
__global__ __launch_bounds__(256) void pack_kernel(const int8_t *__restrict__ q, int N, int K,
                                                   int Np, int Kp, int layout, int half_blocks,
                                                   int8_t *__restrict__ packed) {
    const long long chunk = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long total = (long long)Np * Kp / 16;
    if (chunk >= total) return;
    const int kb_count = Kp / 32;
    const long long frag = chunk >> 6;
    const int lane = (int)(chunk & 63);
    const int pb = (int)(frag / kb_count);
    const int kb = (int)(frag % kb_count);
    const int lb = packed_block_source(pb, layout, half_blocks);
    const int n = lb * 32 + (lane & 31);
    const int k0 = kb * 32 + (lane >> 5) * 16;
    union {
        int8_t b[16];
        int4 v;
    } u;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int k = k0 + i;
        u.b[i] = (lb >= 0 && n < N && k < K) ? q[(size_t)n * K + k] : (int8_t)0;
    }
    *reinterpret_cast<int4 *>(packed + chunk * 16) = u.v;
}

__global__ __launch_bounds__(256) void pack_cols_kernel(const float *__restrict__ scale,
                                                        const int32_t *__restrict__ colsum,
                                                        const int32_t *__restrict__ rowsum, int N,
                                                        int Np, int layout, int half_blocks,
                                                        float *__restrict__ pscale,
                                                        int32_t *__restrict__ pcolsum,
                                                        int32_t *__restrict__ prowsum) {
    const int pc = blockIdx.x * 256 + threadIdx.x;
    if (pc >= Np) return;
    const int lb = packed_block_source(pc >> 5, layout, half_blocks);
    const int n = lb * 32 + (pc & 31);
    const bool ok = lb >= 0 && n < N;
    pscale[pc] = ok ? scale[n] : 0.0f;
    pcolsum[pc] = ok ? colsum[n] : 0;
    if (prowsum) prowsum[pc] = ok ? rowsum[n] : 0;
}

__global__ __launch_bounds__(256) void fill_kernel(uint8_t *__restrict__ dst, uint8_t value,
                                                   size_t bytes) {
    size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 16;
    const size_t stride = (size_t)gridDim.x * 256 * 16;
    const uint32_t v4 = 0x01010101u * value;
    for (; i < bytes; i += stride) {
        if (i + 16 <= bytes && (((uintptr_t)(dst + i)) & 15) == 0) {
            *reinterpret_cast<uint4 *>(dst + i) = make_uint4(v4, v4, v4, v4);
        } else {
            for (size_t j = i; j < i + 16 && j < bytes; ++j) dst[j] = value;
        }
    }
}

// The shapes quant_rows_snake takes: the vector path's, at most 1536 columns.
bool quant_snake_ok(const float *x, int K, int ldx, const uint8_t *q1, int ldq,
                    const uint8_t *q2, const SnakePre &sp) {
    return (K % 4 == 0) && (ldx % 4 == 0) && (ldq % 4 == 0) && (((uintptr_t)x) & 15) == 0 &&
           (((uintptr_t)q1) & 3) == 0 && (((uintptr_t)q2) & 3) == 0 && sp.alpha &&
           K <= kSnakeMaxChannels;
}

// Rows per block of quant_rows_snake: the tile holds at most 4096 floats,
// a whole number of phase-2 passes where it holds that many rows.
int snake_tile_rows(int K) {
    const int rpp = K <= 128 ? 8 : 4, fit = 4096 / K;
    return fit >= rpp ? fit / rpp * rpp : fit;
}

template <int CONV, bool RES>
int quant_rows_snake_dispatch(IroHipContext *ctx, const float *x, int M, int K, int ldx,
                              const SnakePre &sp, uint8_t *q1, int ldq, float *s1, int32_t *z1,
                              uint8_t *q2, float *s2, int32_t *z2, uint32_t sflip) {
    // Eight lanes per row where every lane holds whole float4 of the row.
    const bool g8 = K % 32 == 0 && K <= 256;
    const int fit = 4096 / K;
    const int R = g8 ? (fit >= 32 ? fit / 32 * 32 : fit) : snake_tile_rows(K);
    const unsigned k4 = (unsigned)K / 4;
    // floor(f / k4) == umulhi(2 f, ceil(2^31 / k4)) for the chunk indices
    // f < 1024 used: the rounding adds less than 2^11 / 2^32 < 1 / k4.
    const unsigned magic = (unsigned)((0x80000000ull + k4 - 1) / k4);
    const dim3 grid((unsigned)((M + R - 1) / R)), block(256);
    const size_t lds = sizeof(float) * ((size_t)3 * K + (size_t)R * K);
    hipStream_t st = ctx->stream;
#define IRO_QS(CH, HALF, G8)                                                                      \
    do {                                                                                           \
        if (sp.bias)                                                                               \
            hipLaunchKernelGGL((quant_rows_snake<CONV, CH, RES, HALF, true, G8>), grid, block, lds, \
                               st, x, M, K, ldx, R, magic, sp.bias, sp.alpha, q1, ldq, s1, z1, q2,  \
                               s2, z2, sflip);                                                     \
        else                                                                                       \
            hipLaunchKernelGGL((quant_rows_snake<CONV, CH, RES, HALF, false, G8>), grid, block,     \
                               lds, st, x, M, K, ldx, R, magic, sp.bias, sp.alpha, q1, ldq, s1, z1, \
                               q2, s2, z2, sflip);                                                 \
    } while (0)
    const int ch = (K + 255) / 256;
    if (g8) IRO_QS(1, false, true);
    else if (K <= 128) IRO_QS(1, true, false);
    else if (ch <= 1) IRO_QS(1, false, false);
    else if (ch <= 2) IRO_QS(2, false, false);
    else if (ch <= 4) IRO_QS(4, false, false);
    else IRO_QS(6, false, false);
#undef IRO_QS
    IRO_HIP_CHECK_LAUNCH(ctx);
    return 0;
}

template <int CONV, bool RES>
int quant_rows_dispatch(IroHipContext *ctx, const float *x, int M, int K, int ldx, uint8_t *q1,
                        int ldq, float *s1, int32_t *z1, float *res, uint8_t *q2, float *s2,
                        int32_t *z2, uint32_t sflip) {
    const dim3 grid((M + 3) / 4), block(256);
    const bool vec = (K % 4 == 0) && (ldx % 4 == 0) && (ldq % 4 == 0) &&
                     (((uintptr_t)x) & 15) == 0 && (((uintptr_t)q1) & 3) == 0 &&
                     (!RES || (((uintptr_t)q2) & 3) == 0) &&
                     (!RES || !res || (((uintptr_t)res) & 15) == 0);
    const int ch = (K + 255) / 256;
    hipStream_t st = ctx->stream;
#define IRO_QR(CH, EX)                                                                        \
    hipLaunchKernelGGL((quant_rows_vec<CONV, CH, RES, EX>), grid, block, 0, st, x, M, K, ldx, q1, \
                       ldq, s1, z1, res, q2, s2, z2, sflip)
    // The DiT row widths (1024, 2816) fill whole 256-column chunks: no
    // per-chunk bounds.
    if (vec && K <= 128)
        hipLaunchKernelGGL((quant_rows_half<CONV, RES>), dim3((M + 7) / 8), block, 0, st, x, M, K,
                           ldx, q1, ldq, s1, z1, res, q2, s2, z2, sflip);
    else if (vec && K == 1024) IRO_QR(4, true);
    else if (vec && K == 2816) IRO_QR(11, true);
    else if (vec && ch <= 1) IRO_QR(1, false);
    else if (vec && ch <= 2) IRO_QR(2, false);
    else if (vec && ch <= 4) IRO_QR(4, false);
    else if (vec && ch <= 8) IRO_QR(8, false);
    else if (vec && ch <= 12) IRO_QR(12, false);
    else if (vec && ch <= 16) IRO_QR(16, false);
    else
        hipLaunchKernelGGL((quant_rows_any<CONV, RES>), grid, block, 0, st, x, M, K, ldx, q1, ldq,
                           s1, z1, res, q2, s2, z2, sflip);
#undef IRO_QR
    IRO_HIP_CHECK_LAUNCH(ctx);
    return 0;
}

}  // namespace

int launch_quant_rows(IroHipContext *ctx, const float *x, int M, int K, int ldx, uint8_t *q1,
                      int ldq, float *s1, int32_t *z1, float *res, uint8_t *q2, float *s2,
                      int32_t *z2, bool signed_codes, const SnakePre *snake) {
    const uint32_t sflip = signed_codes ? 0x80808080u : 0u;
    if (M <= 0 || K <= 0) return 0;
    const bool two = q2 != nullptr;
    // The fused snake keeps no remainder rows and takes the vector shapes only.
    if (snake && (res || !quant_snake_ok(x, K, ldx, q1, ldq, q2, *snake))) return 1;
    prof_begin(ctx);
    int rc;
    if (snake && ctx->convention == IRO_HIP_GCC_FASTMATH)
        rc = two ? quant_rows_snake_dispatch<1, true>(ctx, x, M, K, ldx, *snake, q1, ldq, s1, z1, q2, s2, z2, sflip)
                 : quant_rows_snake_dispatch<1, false>(ctx, x, M, K, ldx, *snake, q1, ldq, s1, z1, q2, s2, z2, sflip);
    else if (snake)
        rc = two ? quant_rows_snake_dispatch<0, true>(ctx, x, M, K, ldx, *snake, q1, ldq, s1, z1, q2, s2, z2, sflip)
                 : quant_rows_snake_dispatch<0, false>(ctx, x, M, K, ldx, *snake, q1, ldq, s1, z1, q2, s2, z2, sflip);
    else if (ctx->convention == IRO_HIP_GCC_FASTMATH)
        rc = two ? quant_rows_dispatch<1, true>(ctx, x, M, K, ldx, q1, ldq, s1, z1, res, q2, s2, z2, sflip)
                 : quant_rows_dispatch<1, false>(ctx, x, M, K, ldx, q1, ldq, s1, z1, res, q2, s2, z2, sflip);
    else
        rc = two ? quant_rows_dispatch<0, true>(ctx, x, M, K, ldx, q1, ldq, s1, z1, res, q2, s2, z2, sflip)
                 : quant_rows_dispatch<0, false>(ctx, x, M, K, ldx, q1, ldq, s1, z1, res, q2, s2, z2, sflip);
    // HBM: fp32 row in, one (two) code planes and row scale/zero out.
    const double mk = (double)M * K, planes = two ? 2 : 1;
    prof_end(ctx, two ? PK_QUANT_RESIDUAL : PK_QUANT, 0,
             4 * mk + planes * (mk + 8.0 * M) + (res ? 4 * mk : 0));
    return rc;
}

int launch_weight_quant(IroHipContext *ctx, const float *w, int N, int K, long long stride_n,
                        long long stride_k, int8_t *q, float *scale, int32_t *colsum) {
    const dim3 grid((N + 3) / 4), block(256);
    if (ctx->convention == IRO_HIP_GCC_FASTMATH)
        hipLaunchKernelGGL((weight_quant_kernel<1>), grid, block, 0, ctx->stream, w, N, K,
                           stride_n, stride_k, q, scale, colsum);
    else
        hipLaunchKernelGGL((weight_quant_kernel<0>), grid, block, 0, ctx->stream, w, N, K,
                           stride_n, stride_k, q, scale, colsum);
    IRO_HIP_CHECK_LAUNCH(ctx);
    return 0;
}

int launch_pack(IroHipContext *ctx, const int8_t *q, const float *scale, const int32_t *colsum,
                const int32_t *rowsum, IroHipWeight *w) {
    const int half_blocks = w->layout == 1 ? w->part_N[0] / 32 : 0;
    const long long chunks = (long long)w->Np * w->Kp / 16;
    hipLaunchKernelGGL(pack_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0,
                       ctx->stream, q, w->N, w->K, w->Np, w->Kp, w->layout, half_blocks,
                       w->packed);
    IRO_HIP_CHECK_LAUNCH(ctx);
    hipLaunchKernelGGL(pack_cols_kernel, dim3((w->Np + 255) / 256), dim3(256), 0, ctx->stream,
                       scale, colsum, rowsum, w->N, w->Np, w->layout, half_blocks, w->scale,
                       w->colsum, w->rowsum != w->colsum ? w->rowsum : nullptr);
    IRO_HIP_CHECK_LAUNCH(ctx);
    return 0;
}

namespace {
// Inputs v in [base, base + 2^28) whose packed code differs from the
// reference's clamp(rint(v), 0, 255) (NaN: code 0), counted into *out.
__global__ __launch_bounds__(256) void codes_selfcheck_kernel(unsigned long long *out,
                                                              unsigned base) {
    __shared__ unsigned part[4];
    const unsigned u = base + blockIdx.x * 256u + threadIdx.x;
    const float v = __uint_as_float(u);
    float r = __builtin_rintf(v);
    r = r < 0.0f ? 0.0f : r;
    r = r > 255.0f ? 255.0f : r;
    const unsigned want = v != v ? 0u : (unsigned)r;
    const unsigned got = pack_codes4(v, 0.0f, 0.0f, 0.0f) & 0xffu;
    const unsigned long long m = __ballot(got != want);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = (unsigned)__popcll(m);
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned n = part[0] + part[1] + part[2] + part[3];
        if (n) atomicAdd(out, (unsigned long long)n);
    }
}
}  // namespace

// All 2^32 inputs in 16 launches; *out must start zeroed.
int launch_codes_selfcheck(IroHipContext *ctx, unsigned long long *out) {
    for (unsigned long long base = 0; base < (1ull << 32); base += (1ull << 28)) {
        hipLaunchKernelGGL(codes_selfcheck_kernel, dim3(1u << 20), dim3(256), 0, ctx->stream, out,
                           (unsigned)base);
        IRO_HIP_CHECK_LAUNCH(ctx);
    }
    return 0;
}

int launch_fill(IroHipContext *ctx, void *dst, int value, size_t bytes) {
    if (!bytes) return 0;
    size_t blocks = (bytes + 256 * 16 - 1) / (256 * 16);
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(fill_kernel, dim3((unsigned)blocks), dim3(256), 0, ctx->stream,
                       static_cast<uint8_t *>(dst), (uint8_t)value, bytes);
    IRO_HIP_CHECK_LAUNCH(ctx);
    return 0;
}

}  // namespace iro
