// iro_dit.hip -- the DiT int8 projections (dit.c:739-981) as fused device
// calls, and the int8 linear stack of one Euler step over all blocks.
//
// Each projection group quantizes its input once (dit.c:469-475, shared by
// Q/K/V/gate and by W1/W3) and runs one GEMM whose epilogue finishes the
// group: the split Q/K/V/gate store, silu(w1)*w3, or the gated residual
// x += gate * y (dit.c:1013-1020, 1032-1039), so the projection outputs of
// Wo and W2 never round-trip HBM.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <new>
#include <vector>

#include "iro_internal.h"

#include <mutex>

// The scratch of iro_hip_dit_linear_gated_noalloc: the quantized activation
// (one or two planes of codes, row scales and zero points) of one call.
// Every GPU the library runs on holds its own copy from module load to
// process end; calls on one GPU share it (so calls that overlap on one GPU
// race).  Host code never passes `scratch` itself to a kernel: its device
// address on each GPU comes from hipGetSymbolAddress (noalloc_scratch_init).
static constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace iro {

// Looks up `scratch`'s device address once per device (the caller has made
// ctx->device current) and keeps it in the context.
int noalloc_scratch_init(IroHipContext *ctx) {
    static std::mutex mu;
    static std::vector<void *> per_device;
    std::lock_guard<std::mutex> lock(mu);
    if (per_device.size() <= (size_t)ctx->device) per_device.resize(ctx->device + 1, nullptr);
    if (!per_device[ctx->device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_error(ctx, "no-alloc scratch: hipGetSymbolAddress failed: %s",
                             hipGetErrorString(e));
        per_device[ctx->device] = p;
    }
    ctx->noalloc_scratch = per_device[ctx->device];
    ctx->noalloc_scratch_bytes = kNoAllocScratchBytes;
    return 0;
}

namespace {

// dit.c:593-606, the adaLN RMSNorm modulate of a DiT block, as the strict
// build evaluates it: per row, ms accumulates x[d] * x[d] in index order
// (each square rounded, then added -- a serial chain, so one lane owns a
// row), inv = 1 / sqrtf(ms / D + eps), and h = ((x * inv) * (1 + scale)) +
// shift with the row's branch b = row / S.  A block takes ROWS rows.  Their
// columns pass through LDS 256 at a time (coalesced loads by the whole
// block, the next chunk in flight while the current one is summed; rows
// padded to 260 floats so the row owners' 16-byte reads are conflict-free);
// ROWS lanes of wave 0 own one row each and run the chains.  Then every
// wave writes ROWS / 4 rows with coalesced accesses.  V4: D % 4 == 0 and 16-byte
// aligned rows.
constexpr int kAdaCols = 256, kAdaPitch = 260;

template <bool V4, int ROWS>
__global__ __launch_bounds__(256) void adaln_apply_kernel(const float *__restrict__ x,
                                                          const float *__restrict__ shift,
                                                          const float *__restrict__ scale, int M,
                                                          int S, int D, float eps,
                                                          float *__restrict__ h) {
    constexpr int PP = ROWS / 4;  // pieces per thread per chunk; rows per wave
    __shared__ __attribute__((aligned(16))) float tile[2][ROWS * kAdaPitch];
    __shared__ float inv_s[ROWS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r0 = blockIdx.x * ROWS;
    const int nch = (D + kAdaCols - 1) / kAdaCols;
    // Chunk c, piece i (0..PP-1) of this thread: row i * 4 + tid / 64, float4
    // column tid % 64; rows past M repeat row M-1, columns past D read 0.
    float4 st[PP];
    auto load = [&](int c) {
#pragma unroll
        for (int i = 0; i < PP; ++i) {
            int row = r0 + i * 4 + wave;
            row = row < M ? row : M - 1;
            const int col = c * kAdaCols + lane * 4;
            const float *src = x + (size_t)row * D + col;
            if (V4) {
                st[i] = col < D ? *reinterpret_cast<const float4 *>(src) : make_float4(0, 0, 0, 0);
            } else {
                st[i].x = col + 0 < D ? src[0] : 0.0f;
                st[i].y = col + 1 < D ? src[1] : 0.0f;
                st[i].z = col + 2 < D ? src[2] : 0.0f;
                st[i].w = col + 3 < D ? src[3] : 0.0f;
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < PP; ++i)
            *reinterpret_cast<float4 *>(&tile[buf][(i * 4 + wave) * kAdaPitch + lane * 4]) = st[i];
    };
    load(0);
    store(0);
    __syncthreads();
    float ms = 0.0f;
    for (int c = 0; c < nch; ++c) {
        if (c + 1 < nch) load(c + 1);
        if (wave == 0 && lane < ROWS) {
            const float *tr = &tile[c & 1][lane * kAdaPitch];
            const int n = D - c * kAdaCols < kAdaCols ? D - c * kAdaCols : kAdaCols;
            // 64 values per batch read ahead of their additions, so the
            // chain waits on LDS once per batch.
            int d = 0;
            for (; d + 64 <= n; d += 64) {
                float4 v[16];
#pragma unroll
                for (int j = 0; j < 16; ++j) v[j] = *reinterpret_cast<const float4 *>(tr + d + 4 * j);
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    ms = ms + v[j].x * v[j].x;
                    ms = ms + v[j].y * v[j].y;
                    ms = ms + v[j].z * v[j].z;
                    ms = ms + v[j].w * v[j].w;
                }
            }
            for (; d < n; ++d) ms = ms + tr[d] * tr[d];
        }
        if (c + 1 < nch) store((c + 1) & 1);
        __syncthreads();
    }
    if (wave == 0 && lane < ROWS) inv_s[lane] = 1.0f / __builtin_sqrtf(ms / (float)D + eps);
    __syncthreads();
    // Wave w writes rows PP w .. PP w + PP-1, eight rows per batch: the
    // batch's loads of x, scale and shift all go out before any is used.
    constexpr int RB = PP < 8 ? PP : 8;
    static_assert(PP % RB == 0, "whole batches per wave");
    for (int i0 = 0; i0 < PP; i0 += RB) {
        int rows[RB];
        const float *xr[RB], *sc[RB], *sh[RB];
        float *hr[RB];
        float inv[RB];
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            const int rl = wave * PP + i0 + i;
            rows[i] = r0 + rl;
            const int row = rows[i] < M ? rows[i] : M - 1;
            const int b = row / S;
            xr[i] = x + (size_t)row * D;
            sc[i] = scale + (size_t)b * D;
            sh[i] = shift + (size_t)b * D;
            hr[i] = h + (size_t)row * D;
            inv[i] = inv_s[rl];
        }
        if (V4) {
            for (int d = lane * 4; d < D; d += 256) {
                float4 v[RB], cs[RB], t[RB];
#pragma unroll
                for (int i = 0; i < RB; ++i) {
                    v[i] = *reinterpret_cast<const float4 *>(xr[i] + d);
                    cs[i] = *reinterpret_cast<const float4 *>(sc[i] + d);
                    t[i] = *reinterpret_cast<const float4 *>(sh[i] + d);
                }
#pragma unroll
                for (int i = 0; i < RB; ++i) {
                    if (rows[i] >= M) continue;
                    float4 o;
                    o.x = ((v[i].x * inv[i]) * (1.0f + cs[i].x)) + t[i].x;
                    o.y = ((v[i].y * inv[i]) * (1.0f + cs[i].y)) + t[i].y;
                    o.z = ((v[i].z * inv[i]) * (1.0f + cs[i].z)) + t[i].z;
                    o.w = ((v[i].w * inv[i]) * (1.0f + cs[i].w)) + t[i].w;
                    *reinterpret_cast<float4 *>(hr[i] + d) = o;
                }
            }
        } else {
            for (int d = lane; d < D; d += 64) {
                float v[RB], cs[RB], t[RB];
#pragma unroll
                for (int i = 0; i < RB; ++i) {
                    v[i] = xr[i][d];
                    cs[i] = sc[i][d];
                    t[i] = sh[i][d];
                }
#pragma unroll
                for (int i = 0; i < RB; ++i)
                    if (rows[i] < M) hr[i][d] = ((v[i] * inv[i]) * (1.0f + cs[i])) + t[i];
            }
        }
    }
}

// The same computation with one wave per block and RW rows per wave, for
// rows that fit in LDS whole: the wave loads its rows once (every load in
// flight together), lanes 0..RW-1 run the rows' chains from LDS, and h is
// written from the LDS copy, so x is read from HBM once and no block barrier
// stands between the waves.  The chain is the floor: D dependent additions
// per row, which a wave pays once whatever RW is, so RW sets how many waves
// share the rows.
template <bool V4, int RW>
__global__ __launch_bounds__(64) void adaln_rows_kernel(const float *__restrict__ x,
                                                        const float *__restrict__ shift,
                                                        const float *__restrict__ scale, int M,
                                                        int S, int D, float eps,
                                                        float *__restrict__ h) {
    extern __shared__ __attribute__((aligned(16))) float rows_lds[];
    const int lane = threadIdx.x;
    const int pitch = ((D + 3) & ~3) + 4;
    const int r0 = blockIdx.x * RW;
    int row[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) row[r] = r0 + r < M ? r0 + r : M - 1;
    // 1) The rows into LDS, 1024 columns of every row per batch.
    for (int c0 = 0; c0 < D; c0 += 1024) {
        if (V4) {
            float4 v[RW][4];
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int col = c0 + j * 256 + lane * 4;
                    v[r][j] = col < D ? *reinterpret_cast<const float4 *>(x + (size_t)row[r] * D + col)
                                      : make_float4(0, 0, 0, 0);
                }
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int col = c0 + j * 256 + lane * 4;
                    if (col < D) *reinterpret_cast<float4 *>(&rows_lds[r * pitch + col]) = v[r][j];
                }
        } else {
            float v[RW][16];
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int col = c0 + j * 64 + lane;
                    v[r][j] = col < D ? x[(size_t)row[r] * D + col] : 0.0f;
                }
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int col = c0 + j * 64 + lane;
                    if (col < D) rows_lds[r * pitch + col] = v[r][j];
                }
        }
    }
    __syncthreads();
    // 2) Lane r < RW runs row r's chain in index order.
    float inv = 0.0f;
    if (lane < RW) {
        const float *tr = &rows_lds[lane * pitch];
        float ms = 0.0f;
        int d = 0;
        for (; d + 64 <= D; d += 64) {
            float4 v[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = *reinterpret_cast<const float4 *>(tr + d + 4 * j);
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                ms = ms + v[j].x * v[j].x;
                ms = ms + v[j].y * v[j].y;
                ms = ms + v[j].z * v[j].z;
                ms = ms + v[j].w * v[j].w;
            }
        }
        for (; d < D; ++d) ms = ms + tr[d] * tr[d];
        inv = 1.0f / __builtin_sqrtf(ms / (float)D + eps);
    }
    // 3) h from the LDS rows; scale and shift rows of the row's branch.
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        if (r0 + r >= M) break;
        const float ir = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inv), r));
        const int b = row[r] / S;
        const float *sc = scale + (size_t)b * D, *sh = shift + (size_t)b * D;
        float *hr = h + (size_t)row[r] * D;
        const float *tr = &rows_lds[r * pitch];
        if (V4) {
            for (int c0 = 0; c0 < D; c0 += 1024) {
                float4 v[4], cs[4], t[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int col = c0 + j * 256 + lane * 4;
                    if (col < D) {
                        v[j] = *reinterpret_cast<const float4 *>(tr + col);
                        cs[j] = *reinterpret_cast<const float4 *>(sc + col);
                        t[j] = *reinterpret_cast<const float4 *>(sh + col);
                    }
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int col = c0 + j * 256 + lane * 4;
                    if (col >= D) continue;
                    float4 o;
                    o.x = ((v[j].x * ir) * (1.0f + cs[j].x)) + t[j].x;
                    o.y = ((v[j].y * ir) * (1.0f + cs[j].y)) + t[j].y;
                    o.z = ((v[j].z * ir) * (1.0f + cs[j].z)) + t[j].z;
                    o.w = ((v[j].w * ir) * (1.0f + cs[j].w)) + t[j].w;
                    *reinterpret_cast<float4 *>(hr + col) = o;
                }
            }
        } else {
            for (int c0 = 0; c0 < D; c0 += 1024) {
                float v[16], cs[16], t[16];
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int col = c0 + j * 64 + lane;
                    if (col < D) {
                        v[j] = tr[col];
                        cs[j] = sc[col];
                        t[j] = sh[col];
                    }
                }
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int col = c0 + j * 64 + lane;
                    if (col < D) hr[col] = ((v[j] * ir) * (1.0f + cs[j])) + t[j];
                }
            }
        }
    }
}

// Register-resident form for D % 4 == 0, D <= 256 NJ: each lane loads its
// NJ float4 columns of x, scale and shift for the wave's RW rows at once
// (every load in flight together, none behind a branch, x first in column
// order).  The rounded squares x[d] * x[d] of each 256-column chunk go to LDS
// as soon as that chunk has arrived, and lanes 0..RW-1 add them in index
// order -- the same values and order as the serial loop, with the multiplies
// off the chain -- while the later chunks are still in flight.  The chain is
// the floor (one dependent add per column, about 4 ns each on gfx950); h is
// computed from the registers, so x crosses HBM once.
// NORM: the plain RMSNorm of ops.c:738-747 instead -- h = (x * inv) * w[d]
// with w passed as scale (one row, S = M) and no shift.
template <int RW, int NJ, bool NORM = false>
__global__ __launch_bounds__(64) void adaln_reg_kernel(const float *__restrict__ x,
                                                       const float *__restrict__ shift,
                                                       const float *__restrict__ scale, int M,
                                                       int S, int D, float eps,
                                                       float *__restrict__ h) {
    extern __shared__ __attribute__((aligned(16))) float sq_lds[];
    const int lane = threadIdx.x;
    const int pitch = D + 4;
    const int r0 = blockIdx.x * RW;
    float4 v[RW][NJ], cs[RW][NJ], t[RW][NJ];
    int row[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) row[r] = r0 + r < M ? r0 + r : M - 1;
    // Columns past D load column D-4 (in bounds, never used).
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            int col = j * 256 + lane * 4;
            col = col < D ? col : D - 4;
            v[r][j] = *reinterpret_cast<const float4 *>(x + (size_t)row[r] * D + col);
        }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const int b = row[r] / S;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            int col = j * 256 + lane * 4;
            col = col < D ? col : D - 4;
            cs[r][j] = *reinterpret_cast<const float4 *>(scale + (size_t)b * D + col);
            if (!NORM) t[r][j] = *reinterpret_cast<const float4 *>(shift + (size_t)b * D + col);
        }
    }
    float ms = 0.0f;
    const float *tr = &sq_lds[(lane < RW ? lane : 0) * pitch];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int col = j * 256 + lane * 4;
#pragma unroll
        for (int r = 0; r < RW; ++r)
            if (col < D) {
                float4 q;
                q.x = v[r][j].x * v[r][j].x;
                q.y = v[r][j].y * v[r][j].y;
                q.z = v[r][j].z * v[r][j].z;
                q.w = v[r][j].w * v[r][j].w;
                *reinterpret_cast<float4 *>(&sq_lds[r * pitch + col]) = q;
            }
        __syncthreads();
        if (lane < RW) {
            const int c0 = j * 256;
            if (c0 + 256 <= D) {
                // 16 reads ahead of their additions: one LDS wait per 64.
#pragma unroll
                for (int k0 = 0; k0 < 64; k0 += 16) {
                    float4 q[16];
#pragma unroll
                    for (int k = 0; k < 16; ++k)
                        q[k] = *reinterpret_cast<const float4 *>(tr + c0 + 4 * (k0 + k));
#pragma unroll
                    for (int k = 0; k < 16; ++k) {
                        ms = ms + q[k].x;
                        ms = ms + q[k].y;
                        ms = ms + q[k].z;
                        ms = ms + q[k].w;
                    }
                }
            } else {
                for (int d = c0; d < D; ++d) ms = ms + tr[d];
            }
        }
    }
    float inv = 0.0f;
    if (lane < RW) inv = 1.0f / __builtin_sqrtf(ms / (float)D + eps);
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const float ir = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inv), r));
        const bool live = r0 + r < M;
        float *hr = h + (size_t)row[r] * D;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int col = j * 256 + lane * 4;
            if (!live || col >= D) continue;
            float4 o;
            if (NORM) {
                o.x = (v[r][j].x * ir) * cs[r][j].x;
                o.y = (v[r][j].y * ir) * cs[r][j].y;
                o.z = (v[r][j].z * ir) * cs[r][j].z;
                o.w = (v[r][j].w * ir) * cs[r][j].w;
            } else {
                o.x = ((v[r][j].x * ir) * (1.0f + cs[r][j].x)) + t[r][j].x;
                o.y = ((v[r][j].y * ir) * (1.0f + cs[r][j].y)) + t[r][j].y;
                o.z = ((v[r][j].z * ir) * (1.0f + cs[r][j].z)) + t[r][j].z;
                o.w = ((v[r][j].w * ir) * (1.0f + cs[r][j].w)) + t[r][j].w;
            }
            *reinterpret_cast<float4 *>(hr + col) = o;
        }
    }
}

// dit.c:619-706, the per-head RMSNorm of q and k and the half-RoPE: each
// 64-wide head row's mean square is summed in index order (the strict
// build's serial chain), inv = 1 / sqrtf(ms / 64 + eps), x' = x * (inv * w);
// with ROPE, heads h < heads / 2 rotate the pairs (x'0, x'1) by the table
// entry of the row's position s = token % S: (x'0 c - x'1 s, x'0 s + x'1 c),
// each product rounded.  Rows are the head rows of q then of k ([M, heads,
// 64] each, updated in place); a wave takes 32 of them: 16 lanes per row load
// float4s (four rows per load), the rounded squares go to LDS, lanes 0..31
// run the rows' chains, and the same lanes that loaded a row write it.
constexpr int kHeadRows = 32, kHeadPitch = 68;

template <bool ROPE>
__global__ __launch_bounds__(64) void head_norm_kernel(float *__restrict__ q,
                                                       const float *__restrict__ qw,
                                                       float *__restrict__ k,
                                                       const float *__restrict__ kw,
                                                       const float *__restrict__ rope, int M,
                                                       int S, int heads, int G, float eps) {
    __shared__ __attribute__((aligned(16))) float sq[kHeadRows * kHeadPitch];
    __shared__ float inv_s[kHeadRows];
    const int lane = threadIdx.x, sub = lane >> 4, c4 = (lane & 15) * 4;
    const int g0 = blockIdx.x * kHeadRows;
    const int MH = M * heads;
    float4 v[8];
    float *rowp[8];
    int head[8], pos[8];
    bool live[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        int g = g0 + 4 * j + sub;
        live[j] = g < G;
        g = live[j] ? g : G - 1;
        const int t = g >= MH;
        const int local = g - (t ? MH : 0);
        const int token = local / heads;
        head[j] = local - token * heads;
        pos[j] = token % S;
        rowp[j] = (t ? k : q) + (size_t)local * 64;
        v[j] = *reinterpret_cast<const float4 *>(rowp[j] + c4);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        float4 e;
        e.x = v[j].x * v[j].x;
        e.y = v[j].y * v[j].y;
        e.z = v[j].z * v[j].z;
        e.w = v[j].w * v[j].w;
        *reinterpret_cast<float4 *>(&sq[(4 * j + sub) * kHeadPitch + c4]) = e;
    }
    __syncthreads();
    if (lane < kHeadRows) {
        const float *tr = &sq[lane * kHeadPitch];
        float ms = 0.0f;
#pragma unroll
        for (int b0 = 0; b0 < 16; b0 += 8) {
            float4 e[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) e[i] = *reinterpret_cast<const float4 *>(tr + 4 * (b0 + i));
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                ms = ms + e[i].x;
                ms = ms + e[i].y;
                ms = ms + e[i].z;
                ms = ms + e[i].w;
            }
        }
        inv_s[lane] = 1.0f / __builtin_sqrtf(ms / 64.0f + eps);
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        if (!live[j]) continue;
        const float inv = inv_s[4 * j + sub];
        const int g = g0 + 4 * j + sub;
        const float *w = (g >= MH ? kw : qw) + head[j] * 64 + c4;
        const float4 wv = *reinterpret_cast<const float4 *>(w);
        float4 o;
        o.x = v[j].x * (inv * wv.x);
        o.y = v[j].y * (inv * wv.y);
        o.z = v[j].z * (inv * wv.z);
        o.w = v[j].w * (inv * wv.w);
        if (ROPE && head[j] < heads / 2) {
            // Pairs c4/2 and c4/2 + 1 of this position.
            const float *tab = rope + (size_t)pos[j] * 64 + (c4 >> 1);
            const float2 cs = *reinterpret_cast<const float2 *>(tab);
            const float2 sn = *reinterpret_cast<const float2 *>(tab + 32);
            float4 r;
            r.x = (o.x * cs.x) - (o.y * sn.x);
            r.y = (o.x * sn.x) + (o.y * cs.x);
            r.z = (o.z * cs.y) - (o.w * sn.y);
            r.w = (o.z * sn.y) + (o.w * cs.y);
            o = r;
        }
        *reinterpret_cast<float4 *>(rowp[j] + c4) = o;
    }
}

int qkvg_impl(IroHipContext *ctx, const float *x, int M, const IroHipWeight *w, float *q,
              float *k, float *v, float *gate, int residual) {
    const int D = w->K;
    // codes in the fragment layout when the LDS-pipelined kernel runs the GEMM
    const bool packed = gemm_lds_cfg(ctx, EPI_QKVG, residual != 0, M, D) != 0;
    Workspace ws{ctx};
    size_t off[6];
    act_reserve(ws, M, D, residual != 0, off, packed);
    if (ws.commit()) return -1;
    const ActBufs b = act_at(ws, D, residual != 0, off, packed);
    if (quantize_into(ctx, x, M, D, D, b)) return -1;
    GemmArgs a = gemm_args(b, M, D);
    a.seg[0] = q;
    a.seg[1] = k;
    a.seg[2] = v;
    a.seg[3] = gate;
    a.seg_n = w->part_N[0];
    return launch_gemm(ctx, w, a, EPI_QKVG);
}

// y = lin(quant(x)) [two-term] with the codes staged in b;
// x_res += gate[m / S] * y, or out = y.
int linear_gated_run(IroHipContext *ctx, const ActBufs &b, const float *x, int M, int ldx_in,
                     const IroHipWeight *w, float *out, int ldo, float *x_res,
                     const float *gate, int ldg, int S) {
    const int K = w->K;
    if (quantize_into(ctx, x, M, K, ldx_in, b)) return -1;
    GemmArgs a = gemm_args(b, M, K);
    if (x_res) {
        a.xres = x_res;
        a.gate = gate;
        a.ldg = ldg;
        a.ldx = w->N;
        a.rows_per_branch = S;
        return launch_gemm(ctx, w, a, EPI_GATED);
    }
    a.y = out;
    a.ldy = ldo;
    return launch_gemm(ctx, w, a, EPI_LINEAR);
}

// The same with the codes in the context workspace.
int linear_gated_impl(IroHipContext *ctx, const float *x, int M, int ldx_in,
                      const IroHipWeight *w, int residual, float *out, int ldo, float *x_res,
                      const float *gate, int ldg, int S) {
    const bool packed =
        gemm_lds_cfg(ctx, x_res ? EPI_GATED : EPI_LINEAR, residual != 0, M, w->K) != 0;
    Workspace ws{ctx};
    size_t off[6];
    act_reserve(ws, M, w->K, residual != 0, off, packed);
    if (ws.commit()) return -1;
    const ActBufs b = act_at(ws, w->K, residual != 0, off, packed);
    return linear_gated_run(ctx, b, x, M, ldx_in, w, out, ldo, x_res, gate, ldg, S);
}

// hidden [M, H] = silu(W1 h) * W3 h from one int8 GEMM (dit.c:939-956).
int swiglu_w13(IroHipContext *ctx, const float *h, int M, const IroHipWeight *w13,
               int residual_w13, float *hidden) {
    const int D = w13->K, H = w13->part_N[0];
    const bool p1 = gemm_lds_cfg(ctx, EPI_SWIGLU, residual_w13 != 0, M, D) != 0;
    Workspace ws{ctx};
    size_t off1[6];
    act_reserve(ws, M, D, residual_w13 != 0, off1, p1);
    if (ws.commit()) return -1;
    const ActBufs b1 = act_at(ws, D, residual_w13 != 0, off1, p1);
    if (quantize_into(ctx, h, M, D, D, b1)) return -1;
    GemmArgs a = gemm_args(b1, M, D);
    a.hidden = hidden;
    a.ldh = H;
    return launch_gemm(ctx, w13, a, EPI_SWIGLU);
}

// keep_hidden: the caller reads the fp32 hidden state; otherwise the W1/W3
// kernel may quantize it for W2 itself (same codes) and not store it.
int swiglu_impl(IroHipContext *ctx, const float *h, int M, const IroHipWeight *w13,
                const IroHipWeight *w2, int residual_w13, int residual_w2, float *hidden,
                bool keep_hidden, float *out, float *x_res, const float *gate, int ldg, int S) {
    const int D = w13->K, H = w13->part_N[0];
    const bool p1 = gemm_lds_cfg(ctx, EPI_SWIGLU, residual_w13 != 0, M, D) != 0;
    const bool p2 = gemm_lds_cfg(ctx, x_res ? EPI_GATED : EPI_LINEAR, residual_w2 != 0, M, H) != 0;
    Workspace ws{ctx};
    size_t off1[6], off2[6], oh = 0;
    act_reserve(ws, M, D, residual_w13 != 0, off1, p1);
    act_reserve(ws, M, H, residual_w2 != 0, off2, p2);
    if (!hidden) oh = ws.reserve(sizeof(float) * (size_t)M * H);
    if (ws.commit()) return -1;
    const ActBufs b1 = act_at(ws, D, residual_w13 != 0, off1, p1);
    const ActBufs b2 = act_at(ws, H, residual_w2 != 0, off2, p2);
    float *hid = hidden ? hidden : ws.at<float>(oh);
    if (quantize_into(ctx, h, M, D, D, b1)) return -1;
    GemmArgs a = gemm_args(b1, M, D);
    a.hidden = hid;
    a.ldh = H;
    int fused = 1;
    if (!keep_hidden && !p2) {
        GemmArgs aq = a;
        aq.hq1 = b2.q1;
        aq.hq2 = b2.q2;
        aq.ldhq = b2.ld;
        aq.hs1 = b2.s1;
        aq.hz1 = b2.z1;
        aq.hs2 = b2.s2;
        aq.hz2 = b2.z2;
        fused = launch_gemm(ctx, w13, aq, EPI_SWIGLU);
        if (fused < 0) return -1;
    }
    if (fused && (launch_gemm(ctx, w13, a, EPI_SWIGLU) || quantize_into(ctx, hid, M, H, H, b2)))
        return -1;
    GemmArgs a2 = gemm_args(b2, M, H);
    if (x_res) {
        a2.xres = x_res;
        a2.gate = gate;
        a2.ldg = ldg;
        a2.ldx = D;
        a2.rows_per_branch = S;
        return launch_gemm(ctx, w2, a2, EPI_GATED);
    }
    a2.y = out;
    a2.ldy = D;
    return launch_gemm(ctx, w2, a2, EPI_LINEAR);
}

}  // namespace
}  // namespace iro

// A captured sequence of launches and the arguments it was captured with:
// replayed while the arguments (pointers, sizes, the workspace epoch) stay
// the same; the first call with new arguments runs eagerly (sizing every
// buffer), the second captures.
struct GraphCache {
    std::vector<long long> args;
    unsigned epoch = 0;  // the workspace epoch the launches were recorded at
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int seen = 0;
    void drop() {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        exec = nullptr;
        graph = nullptr;
        seen = 0;
        args.clear();
    }
};

constexpr int kMaxChains = 4;  // concurrent row runs of a linear-stack step

// A few graph caches for alternating argument sets (a sampler's CFG steps
// at batch 3 and its plain steps at batch 1): the slot holding the same
// arguments, else a free one, else the oldest.
struct GraphSet {
    GraphCache slot[4];
    int next = 0;
    GraphCache &pick(const std::vector<long long> &args) {
        for (GraphCache &g : slot)
            if (g.seen && g.args == args) return g;
        for (GraphCache &g : slot)
            if (!g.seen) return g;
        return slot[next++ & 3];
    }
    void drop() {
        for (GraphCache &g : slot) g.drop();
    }
};

// The int8 weights of one DiT linear stack, device resident and pre-packed
// once (the reference builds them once in iro_engine_init,
// generate.c:527-579), plus the per-step activation buffers.
//
// The modulation linears of all blocks read the same conditioning rows, so
// their weights are stacked into one [blocks * ada_np, D] weight (block b at
// rows b * ada_np) and a step computes every block's modulation with one
// quantization and one GEMM; block b's modulation is columns
// b * ada_np .. + 6D of that output.  Integer sums and per-element
// epilogues do not depend on the stacking, so the result is the one of
// per-block linears.
//
// A step with the same buffers and shape as the previous one replays a HIP
// graph of the whole step (captured on the second such call), so the
// launch cost of its ~9 kernels per block is paid once.
struct IroHipDiTStack {
    IroHipContext *ctx = nullptr;
    int blocks = 0, D = 0, H = 0;
    int residual_mask = 8;
    // IRO_INT8_MASK (dit.c:273-291): groups whose bit is clear (1 QKVG, 2 Wo,
    // 4 W1/W3, 8 W2) run through the fp32 linear on device copies of their
    // fp32 weights, kept by set_block; the int8 weights are built anyway, as
    // the reference's iro_dit_int8_quantize builds all of them.
    int int8_mask = 15;
    struct F32Weights {
        float *wq = nullptr, *wk = nullptr, *wv = nullptr, *wg = nullptr, *wo = nullptr,
              *w1 = nullptr, *w3 = nullptr, *w2 = nullptr;
    };
    std::vector<F32Weights> f32w;
    int any_set = 0;  // some block's weights were set (the mask is then fixed)
    IroHipWeight *ada_all = nullptr;
    int ada_np = 0;
    std::vector<char> ada_set;  // block has its modulation weight (the stack step reads it)
    std::vector<char> w_set;    // block has its QKVG, Wo, W1/W3 and W2 weights
    std::vector<IroHipWeight *> qkvg, wo, w13, w2;
    int cap_rows = 0, cap_branches = 0;
    float *q = nullptr, *k = nullptr, *v = nullptr, *g = nullptr, *hidden = nullptr;
    float *mod = nullptr;
    float *h = nullptr, *mix = nullptr;  // block forward: normed input, attention output
    float *proj = nullptr, *params = nullptr;  // sampler step: hidden rows, adaLN parameters
    float *branch = nullptr, *hidden3 = nullptr;  // fp32 groups: a branch [M, D], W3 rows [M, H]
    std::vector<IroHipDiTLayerF32> f32;        // sampler step: per-layer fp32 parameters
    std::vector<char> f32_set;
    IroHipDiTHead head{};
    int head_set = 0;
    // graphs of the linear-stack step, and of the sampler step's network
    // forward (its CFG / Euler update, whose scalars change every step, is
    // launched after it), per argument set
    int use_graph = 1;
    GraphSet graphs, sgraphs;
    // concurrent row runs of the linear-stack step (0: off)
    int chains = 0;
    hipStream_t side[kMaxChains] = {};
    hipEvent_t join[kMaxChains] = {};
    hipEvent_t fork = nullptr;
    int nstreams = 0;
    void *chain_ws[kMaxChains] = {};
    size_t chain_ws_bytes = 0;
    // the persistent kernel of the step (iro_persist.hip)
    int use_persist = 0;
    iro::PersistPlan *persist = nullptr;
    int persist_M = 0, persist_S = 0;  // shape the plan was prepared for (0: stale)
};

using namespace iro;

namespace {

void stack_free_acts(IroHipDiTStack *s) {
    for (float **p : {&s->q, &s->k, &s->v, &s->g, &s->hidden, &s->mod, &s->h, &s->mix,
                      &s->proj, &s->params, &s->branch, &s->hidden3}) {
        if (*p) (void)hipFree(*p);
        *p = nullptr;
    }
    s->cap_rows = s->cap_branches = 0;
}

void stack_drop_graph(IroHipDiTStack *s) {
    s->graphs.drop();
    s->sgraphs.drop();
    s->persist_M = s->persist_S = 0;  // weights or buffers may have changed
}

void f32_weights_free(IroHipDiTStack::F32Weights &f) {
    for (float *p : {f.wq, f.wk, f.wv, f.wg, f.wo, f.w1, f.w3, f.w2})
        if (p) (void)hipFree(p);
    f = IroHipDiTStack::F32Weights{};
}

bool stack_persistent(const IroHipDiTStack *s) {
    return s->use_persist && s->int8_mask == 15 && persist_supported(s->D, s->H, s->residual_mask);
}

// Buffers and weight table of the persistent kernel for this shape
// (allocates: outside graph capture).
int stack_persist_prepare(IroHipDiTStack *s, int B, int S) {
    const int M = B * S;
    if (s->persist_M == M && s->persist_S == S) return 0;
    s->graphs.drop();  // captured steps hold the previous plan's buffers
    std::vector<const IroHipWeight *> ws;
    for (int b = 0; b < s->blocks; ++b)
        for (const auto *v : {&s->qkvg, &s->wo, &s->w13, &s->w2}) ws.push_back((*v)[b]);
    if (persist_prepare(s->ctx, &s->persist, M, s->D, s->H, S, s->blocks,
                        (s->residual_mask & 8) != 0, ws.data(), s->q, s->k, s->v, s->g, s->hidden,
                        s->mod, s->blocks * s->ada_np, s->ada_np))
        return -1;
    s->persist_M = M;
    s->persist_S = S;
    return 0;
}

int stack_reserve(IroHipDiTStack *s, int M, int B) {
    if (M <= s->cap_rows && B <= s->cap_branches) return 0;
    IroHipContext *ctx = s->ctx;
    IRO_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    stack_drop_graph(s);
    stack_free_acts(s);
    const size_t md = sizeof(float) * (size_t)M * s->D;
    hipError_t e = hipMalloc(&s->q, md);
    if (e == hipSuccess) e = hipMalloc(&s->k, md);
    if (e == hipSuccess) e = hipMalloc(&s->v, md);
    if (e == hipSuccess) e = hipMalloc(&s->g, md);
    if (e == hipSuccess) e = hipMalloc(&s->h, md);
    if (e == hipSuccess) e = hipMalloc(&s->mix, md);
    if (e == hipSuccess) e = hipMalloc(&s->proj, md);
    if (e == hipSuccess) e = hipMalloc(&s->params, sizeof(float) * 6 * (size_t)B * s->D);
    if (e == hipSuccess) e = hipMalloc(&s->hidden, sizeof(float) * (size_t)M * s->H);
    if (e == hipSuccess)
        e = hipMalloc(&s->mod, sizeof(float) * (size_t)B * s->blocks * s->ada_np);
    if (e == hipSuccess && s->int8_mask != 15) e = hipMalloc(&s->branch, md);
    if (e == hipSuccess && s->int8_mask != 15)
        e = hipMalloc(&s->hidden3, sizeof(float) * (size_t)M * s->H);
    if (e != hipSuccess) {
        stack_free_acts(s);
        return set_error(ctx, "dit_stack: hipMalloc failed: %s", hipGetErrorString(e));
    }
    s->cap_rows = M;
    s->cap_branches = B;
    return 0;
}

// Runs `launch` through the graph cache gc: replays the graph captured with
// the same key (the arguments plus the workspace epoch), runs eagerly the
// first time a key is seen and captures on the second.
template <class F>
int graph_step(IroHipContext *ctx, GraphSet &set, bool use, const std::vector<long long> &args,
               F &&launch) {
    if (!use || ctx->prof) {
        set.drop();
        return launch();
    }
    GraphCache &gc = set.pick(args);
    if (gc.exec && gc.args == args && gc.epoch == ctx->ws_epoch) {
        IRO_HIP_TRY(ctx, hipGraphLaunch(gc.exec, ctx->stream));
        return 0;
    }
    if (gc.args != args || !gc.seen || gc.epoch != ctx->ws_epoch) {
        gc.drop();
        if (launch()) return -1;
        gc.args = args;
        gc.epoch = ctx->ws_epoch;  // after the eager run sized the workspace
        gc.seen = 1;
        return 0;
    }
    IRO_HIP_TRY(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    const int rc = launch();
    hipGraph_t graph = nullptr;
    const hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
    if (rc || e != hipSuccess || !graph || ctx->ws_epoch != gc.epoch) {
        if (graph) (void)hipGraphDestroy(graph);
        gc.drop();
        return set_error(ctx, "graph capture failed (%s)",
                         e != hipSuccess ? hipGetErrorString(e) : "a launch failed");
    }
    hipGraphExec_t exec = nullptr;
    const hipError_t ei = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (ei != hipSuccess) {
        (void)hipGraphDestroy(graph);
        gc.drop();
        return set_error(ctx, "graph instantiate failed: %s", hipGetErrorString(ei));
    }
    gc.graph = graph;
    gc.exec = exec;
    IRO_HIP_TRY(ctx, hipGraphLaunch(gc.exec, ctx->stream));
    return 0;
}

// The activation buffers a run of rows writes: the stack's, from row r0.
struct SiteBufs {
    float *q, *k, *v, *g, *hidden, *branch, *hidden3;
};

SiteBufs site_bufs(const IroHipDiTStack *s, int r0) {
    const size_t d = (size_t)r0 * s->D, h = (size_t)r0 * s->H;
    return SiteBufs{s->q + d, s->k + d, s->v + d, s->g + d, s->hidden + h,
                    s->branch ? s->branch + d : nullptr, s->hidden3 ? s->hidden3 + h : nullptr};
}

// The four projection sites of block blk, int8 or, for a group whose mask
// bit is clear, the fp32 linear (dit.c:780-798, 876-884, 939-972).
// dit.c:780-798: Q, K, V and the attention gate from `in` [M, D].
int site_qkvg(IroHipDiTStack *s, const SiteBufs &o, int blk, const float *in, int M) {
    IroHipContext *ctx = s->ctx;
    const int D = s->D;
    if (s->int8_mask & 1)
        return qkvg_impl(ctx, in, M, s->qkvg[blk], o.q, o.k, o.v, o.g, s->residual_mask & 1);
    const IroHipDiTStack::F32Weights &f = s->f32w[blk];
    return iro_hip_linear_f32(ctx, in, M, D, f.wq, D, nullptr, o.q) ||
           iro_hip_linear_f32(ctx, in, M, D, f.wk, D, nullptr, o.k) ||
           iro_hip_linear_f32(ctx, in, M, D, f.wv, D, nullptr, o.v) ||
           iro_hip_linear_f32(ctx, in, M, D, f.wg, D, nullptr, o.g);
}

// dit.c:876-884 and 1013-1020: x += gate[m / S] * Wo(mix).
int site_wo(IroHipDiTStack *s, const SiteBufs &o, int blk, const float *mix, int M, float *x,
            const float *gate, int ldg, int S) {
    IroHipContext *ctx = s->ctx;
    const int D = s->D;
    if (s->int8_mask & 2)
        return linear_gated_impl(ctx, mix, M, D, s->wo[blk], s->residual_mask & 2, nullptr, 0, x,
                                 gate, ldg, S);
    return iro_hip_linear_f32(ctx, mix, M, D, s->f32w[blk].wo, D, nullptr, o.branch) ||
           launch_gated_residual(ctx, x, gate, ldg, o.branch, M, D, S);
}

// dit.c:939-972 and 1032-1039: x += gate[m / S] * W2(silu(W1 h) * W3 h).
int site_mlp(IroHipDiTStack *s, const SiteBufs &o, int blk, const float *h, int M, float *x,
             const float *gate, int ldg, int S) {
    IroHipContext *ctx = s->ctx;
    const int D = s->D, H = s->H, rm = s->residual_mask;
    const bool i13 = (s->int8_mask & 4) != 0, i2 = (s->int8_mask & 8) != 0;
    if (i13 && i2)
        return swiglu_impl(ctx, h, M, s->w13[blk], s->w2[blk], rm & 4, rm & 8, o.hidden, false,
                           nullptr, x, gate, ldg, S);
    const IroHipDiTStack::F32Weights &f = s->f32w[blk];
    if (i13) {
        if (swiglu_w13(ctx, h, M, s->w13[blk], rm & 4, o.hidden)) return -1;
    } else if (iro_hip_linear_f32(ctx, h, M, D, f.w1, H, nullptr, o.hidden) ||
               iro_hip_linear_f32(ctx, h, M, D, f.w3, H, nullptr, o.hidden3) ||
               launch_silu(ctx, o.hidden, o.hidden3, (long long)M * H)) {
        return -1;
    }
    if (i2)
        return linear_gated_impl(ctx, o.hidden, M, H, s->w2[blk], rm & 8, nullptr, 0, x, gate,
                                 ldg, S);
    return iro_hip_linear_f32(ctx, o.hidden, M, H, f.w2, D, nullptr, o.branch) ||
           launch_gated_residual(ctx, x, gate, ldg, o.branch, M, D, S);
}

// Row runs that go through a step's blocks concurrently, each on its own
// stream: one per CFG branch when B > 1 (rows of one branch share their
// modulation rows), else S split into runs of whole 32-row blocks.  The
// runs' kernels overlap, which fills the GPU where one run's kernels leave
// it idle (their tails, their few tiles at one branch's 750 rows).
int stack_runs(const IroHipDiTStack *s, int B, int S, int *r0, int *rows) {
    int n = s->chains;
    if (n <= 1) return 1;
    if (B > 1) {
        if (B > kMaxChains) return 1;
        for (int b = 0; b < B; ++b) {
            r0[b] = b * S;
            rows[b] = S;
        }
        return B;
    }
    const int blocks = (S + 31) / 32;
    if (n > blocks) n = blocks;
    if (n <= 1) return 1;
    int start = 0;
    for (int c = 0; c < n; ++c) {
        const int nb = blocks / n + (c < blocks % n ? 1 : 0);
        r0[c] = start;
        rows[c] = (c == n - 1) ? S - start : nb * 32;
        start += rows[c];
    }
    return n;
}

// Streams, events and one inner-workspace region per run, sized for the
// largest run's codes (allocates: outside graph capture).
int stack_chain_prepare(IroHipDiTStack *s, int nrun, const int *rows) {
    IroHipContext *ctx = s->ctx;
    const int D = s->D, H = s->H, rm = s->residual_mask;
    size_t need = 0;
    for (int c = 0; c < nrun; ++c) {
        const int Mc = rows[c];
        size_t off[6], off2[6];
        Workspace a{ctx}, b{ctx}, w{ctx};
        act_reserve(a, Mc, D, rm & 1, off, gemm_lds_cfg(ctx, EPI_QKVG, rm & 1, Mc, D) != 0);
        act_reserve(b, Mc, D, rm & 2, off, gemm_lds_cfg(ctx, EPI_GATED, rm & 2, Mc, D) != 0);
        act_reserve(w, Mc, D, rm & 4, off, gemm_lds_cfg(ctx, EPI_SWIGLU, rm & 4, Mc, D) != 0);
        act_reserve(w, Mc, H, rm & 8, off2, gemm_lds_cfg(ctx, EPI_GATED, rm & 8, Mc, H) != 0);
        need = std::max(need, std::max(a.need, std::max(b.need, w.need)));
    }
    if (s->nstreams < nrun) {
        for (int c = s->nstreams; c < nrun; ++c) {
            IRO_HIP_TRY(ctx, hipStreamCreateWithFlags(&s->side[c], hipStreamNonBlocking));
            IRO_HIP_TRY(ctx, hipEventCreateWithFlags(&s->join[c], hipEventDisableTiming));
            s->nstreams = c + 1;
        }
    }
    if (!s->fork) IRO_HIP_TRY(ctx, hipEventCreateWithFlags(&s->fork, hipEventDisableTiming));
    if (need > s->chain_ws_bytes) {
        IRO_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        for (void *&p : s->chain_ws)
            if (p) {
                (void)hipFree(p);
                p = nullptr;
            }
        s->chain_ws_bytes = 0;
        for (int c = 0; c < kMaxChains; ++c) IRO_HIP_TRY(ctx, hipMalloc(&s->chain_ws[c], need));
        s->chain_ws_bytes = need;
        s->graphs.drop();  // captured steps hold the previous regions
    }
    return 0;
}

// The launches of one step (sampler.c:243-301 runs dit_block per layer).
int stack_launch(IroHipDiTStack *s, float *x, const float *cond, int B, int S) {
    IroHipContext *ctx = s->ctx;
    const int M = B * S, D = s->D;
    const int ldm = s->blocks * s->ada_np;
    // modulation rows of every block [B, blocks * ada_np]: shift/scale/gate
    // for attention and MLP, 6D columns per block
    if (linear_gated_impl(ctx, cond, B, D, s->ada_all, 0, s->mod, ldm, nullptr, nullptr, 0, 1))
        return -1;
    if (stack_persistent(s)) return persist_launch(ctx, s->persist, x);
    int r0[kMaxChains], rows[kMaxChains];
    const int nrun = stack_runs(s, B, S, r0, rows);
    if (nrun == 1) {
        const SiteBufs o = site_bufs(s, 0);
        for (int blk = 0; blk < s->blocks; ++blk) {
            const float *mod = s->mod + (size_t)blk * s->ada_np;
            if (site_qkvg(s, o, blk, x, M) || site_wo(s, o, blk, o.v, M, x, mod + 2 * D, ldm, S) ||
                site_mlp(s, o, blk, x, M, x, mod + 5 * D, ldm, S))
                return -1;
        }
        return 0;
    }
    // Fork the runs off the context stream after the modulation GEMM,
    // issue their launches block by block, join them back.
    hipStream_t main = ctx->stream;
    IRO_HIP_TRY(ctx, hipEventRecord(s->fork, main));
    for (int c = 0; c < nrun; ++c) IRO_HIP_TRY(ctx, hipStreamWaitEvent(s->side[c], s->fork, 0));
    int rc = 0;
    for (int blk = 0; blk < s->blocks && !rc; ++blk) {
        for (int c = 0; c < nrun && !rc; ++c) {
            ctx->stream = s->side[c];
            ctx->ws_override = s->chain_ws[c];
            ctx->ws_override_bytes = s->chain_ws_bytes;
            const SiteBufs o = site_bufs(s, r0[c]);
            float *xc = x + (size_t)r0[c] * D;
            const float *mod = s->mod + (size_t)(r0[c] / S) * ldm + (size_t)blk * s->ada_np;
            rc = site_qkvg(s, o, blk, xc, rows[c]) ||
                 site_wo(s, o, blk, o.v, rows[c], xc, mod + 2 * D, ldm, S) ||
                 site_mlp(s, o, blk, xc, rows[c], xc, mod + 5 * D, ldm, S);
        }
    }
    ctx->stream = main;
    ctx->ws_override = nullptr;
    ctx->ws_override_bytes = 0;
    for (int c = 0; c < nrun; ++c) {
        IRO_HIP_TRY(ctx, hipEventRecord(s->join[c], s->side[c]));
        IRO_HIP_TRY(ctx, hipStreamWaitEvent(main, s->join[c], 0));
    }
    return rc ? -1 : 0;
}

}  // namespace

extern "C" {

int iro_hip_dit_qkvg(IroHipContext *ctx, const float *x, int M, const IroHipWeight *w, float *q,
                     float *k, float *v, float *gate, int residual) {
    if (!ctx || !w || M < 0 || w->nparts != 4 || w->layout != 0 ||
        (M && (!x || !q || !k || !v || !gate)))
        return set_error(ctx, "dit_qkvg: needs a 4-part concatenated weight and q,k,v,gate");
    for (int i = 1; i < 4; ++i)
        if (w->part_N[i] != w->part_N[0]) return set_error(ctx, "dit_qkvg: unequal parts");
    if (M == 0) return 0;
    return qkvg_impl(ctx, x, M, w, q, k, v, gate, residual);
}

int iro_hip_dit_linear_gated(IroHipContext *ctx, const float *mix, int M, const IroHipWeight *w,
                             int residual, float *out, float *x_res, const float *gate, int S) {
    if (!ctx || !w || M < 0 || (M && (!mix || (!x_res && !out) || (x_res && (!gate || S <= 0)))))
        return set_error(ctx, "dit_linear_gated: invalid arguments");
    if (M == 0) return 0;
    return linear_gated_impl(ctx, mix, M, w->K, w, residual, out, w->N, x_res, gate, w->N, S);
}

int iro_hip_dit_linear_gated_noalloc(IroHipContext *ctx, const float *mix, int M,
                                     const IroHipWeight *w, int residual, float *out,
                                     float *x_res, const float *gate, int S) {
    if (!ctx || !w || M < 0 || (M && (!mix || (!x_res && !out) || (x_res && (!gate || S <= 0)))))
        return set_error(ctx, "dit_linear_gated_noalloc: invalid arguments");
    if (!ctx->noalloc_scratch)
        return set_error(ctx, "dit_linear_gated_noalloc: no scratch on this device");
    if (M == 0) return 0;
    // The codes' layout in the scratch is the workspace's (act_reserve):
    // offsets from 0, 256-byte aligned.
    const bool packed =
        gemm_lds_cfg(ctx, x_res ? EPI_GATED : EPI_LINEAR, residual != 0, M, w->K) != 0;
    Workspace lay{ctx};
    size_t off[6];
    act_reserve(lay, M, w->K, residual != 0, off, packed);
    if (lay.need > ctx->noalloc_scratch_bytes)
        return set_error(ctx,
                         "dit_linear_gated_noalloc: %d rows of %d codes%s need %zu bytes, above "
                         "the %zu-byte scratch",
                         M, w->K, residual ? " (two planes)" : "", lay.need,
                         ctx->noalloc_scratch_bytes);
    unsigned char *base = static_cast<unsigned char *>(ctx->noalloc_scratch);
    ActBufs b;
    b.ld = packed ? -(w->K / 32) : (int)round_up((size_t)w->K, 16);
    b.q1 = base + off[0];
    b.s1 = reinterpret_cast<float *>(base + off[1]);
    b.z1 = reinterpret_cast<int32_t *>(base + off[2]);
    b.q2 = residual ? base + off[3] : nullptr;
    b.s2 = residual ? reinterpret_cast<float *>(base + off[4]) : nullptr;
    b.z2 = residual ? reinterpret_cast<int32_t *>(base + off[5]) : nullptr;
    return linear_gated_run(ctx, b, mix, M, w->K, w, out, w->N, x_res, gate, w->N, S);
}

int iro_hip_dit_swiglu(IroHipContext *ctx, const float *h, int M, const IroHipWeight *w13,
                       const IroHipWeight *w2, int residual_w13, int residual_w2, float *hidden,
                       float *out, float *x_res, const float *gate, int S) {
    if (!ctx || !w13 || !w2 || M < 0 || w13->layout != 1 || w2->K != w13->part_N[0] ||
        w2->N != w13->K || (M && (!h || (!x_res && !out) || (x_res && (!gate || S <= 0)))))
        return set_error(ctx, "dit_swiglu: invalid arguments or weight shapes");
    if (M == 0) return 0;
    return swiglu_impl(ctx, h, M, w13, w2, residual_w13, residual_w2, hidden, hidden != nullptr,
                       out, x_res, gate, w13->K, S);
}

int iro_hip_dit_adaln_apply(IroHipContext *ctx, const float *x, int B, int S, int D,
                            const float *shift, const float *scale, float eps, float *h) {
    if (!ctx || B < 0 || S < 0 || D <= 0 || ((long long)B * S && (!x || !shift || !scale || !h)))
        return set_error(ctx, "dit_adaln_apply: invalid arguments");
    const int M = B * S;
    if (M == 0) return 0;
    const bool v4 = D % 4 == 0 && ((((uintptr_t)x) | ((uintptr_t)shift) | ((uintptr_t)scale) |
                                     ((uintptr_t)h)) & 15) == 0;
    // Register-resident rows up to D = 2048 (V4).
    if (v4 && D <= 2048) {
        const int nj = (D + 255) / 256;
        const size_t pitch_bytes = ((size_t)D + 4) * sizeof(float);
#define IRO_ADA_REG_LAUNCH(RWV, NJV)                                                              \
    hipLaunchKernelGGL((adaln_reg_kernel<RWV, NJV>), dim3((M + RWV - 1) / RWV), dim3(64),         \
                       RWV * pitch_bytes, ctx->stream, x, shift, scale, M, S, D, eps, h)
        if (nj <= 2)
            IRO_ADA_REG_LAUNCH(2, 2);
        else if (nj <= 4)
            IRO_ADA_REG_LAUNCH(2, 4);
        else if (nj <= 5)
            IRO_ADA_REG_LAUNCH(2, 5);
        else
            IRO_ADA_REG_LAUNCH(1, 8);
#undef IRO_ADA_REG_LAUNCH
        IRO_HIP_CHECK_LAUNCH(ctx);
        return 0;
    }
    // Rows resident in LDS when they fit in 64 KiB: two rows per wave up
    // to D = 8184, one up to D = 16380.
    const size_t row_bytes = ((size_t)((D + 3) & ~3) + 4) * sizeof(float);
    const int rw = 2 * row_bytes <= 65536 ? 2 : 1;
    if (rw * row_bytes <= 65536) {
        const dim3 g((M + rw - 1) / rw), blk(64);
        const size_t lds = rw * row_bytes;
#define IRO_ADA_ROWS_LAUNCH(RWV)                                                                 \
    if (v4)                                                                                     \
        hipLaunchKernelGGL((adaln_rows_kernel<true, RWV>), g, blk, lds, ctx->stream, x, shift,  \
                           scale, M, S, D, eps, h);                                             \
    else                                                                                        \
        hipLaunchKernelGGL((adaln_rows_kernel<false, RWV>), g, blk, lds, ctx->stream, x, shift, \
                           scale, M, S, D, eps, h);
        if (rw == 2) {
            IRO_ADA_ROWS_LAUNCH(2)
        } else {
            IRO_ADA_ROWS_LAUNCH(1)
        }
#undef IRO_ADA_ROWS_LAUNCH
        IRO_HIP_CHECK_LAUNCH(ctx);
        return 0;
    }
    constexpr int R = 16;
    const dim3 grid((M + R - 1) / R), block(256);
    if (v4)
        hipLaunchKernelGGL((adaln_apply_kernel<true, R>), grid, block, 0, ctx->stream, x, shift,
                           scale, M, S, D, eps, h);
    else
        hipLaunchKernelGGL((adaln_apply_kernel<false, R>), grid, block, 0, ctx->stream, x, shift,
                           scale, M, S, D, eps, h);
    IRO_HIP_CHECK_LAUNCH(ctx);
    return 0;
}

// The rotation table of dit.c:641-657 and 697-703 for positions 0..S-1, in
// the context: per pair p the double step (cos, sin) of 1 / 10000^(2p/64)
// from the C library, then position s+1 = position s times the step (each
// double product rounded, no fused multiply-add; this file is compiled with
// contraction off), stored as float.  Position s's entry does not depend on S,
// so a longer table serves every shorter sequence; it is rebuilt only when a
// call needs more positions (the first call per length allocates).
static int rope_table(IroHipContext *ctx, int S) {
    if (S <= ctx->rope_S) return 0;
    const int n = S < 1024 ? 1024 : S;
    std::vector<float> tab((size_t)n * 64);
    double cs[32], sn[32], c[32], s[32];
    for (int p = 0; p < 32; ++p) {
        const double theta = 1.0 / std::pow(10000.0, (double)(2 * p) / 64.0);
        cs[p] = std::cos(theta);
        sn[p] = std::sin(theta);
        c[p] = 1.0;
        s[p] = 0.0;
    }
    for (int t = 0; t < n; ++t) {
        for (int p = 0; p < 32; ++p) {
            tab[(size_t)t * 64 + p] = (float)c[p];
            tab[(size_t)t * 64 + 32 + p] = (float)s[p];
        }
        for (int p = 0; p < 32; ++p) {
            const double a = c[p] * cs[p], b = s[p] * sn[p];
            const double e = s[p] * cs[p], f = c[p] * sn[p];
            c[p] = a - b;
            s[p] = e + f;
        }
    }
    float *dev = nullptr;
    if (hipMalloc(&dev, tab.size() * sizeof(float)) != hipSuccess)
        return set_error(ctx, "dit_qk_norm_rope: out of device memory for the rotation table");
    if (hipMemcpyAsync(dev, tab.data(), tab.size() * sizeof(float), hipMemcpyHostToDevice,
                       ctx->stream) != hipSuccess ||
        hipStreamSynchronize(ctx->stream) != hipSuccess) {
        (void)hipFree(dev);
        return set_error(ctx, "dit_qk_norm_rope: rotation table upload failed");
    }
    if (ctx->rope) (void)hipFree(ctx->rope);
    ctx->rope = dev;
    ctx->rope_S = n;
    return 0;
}

static int head_norm(IroHipContext *ctx, float *q, const float *qw, float *k, const float *kw,
                     int B, int S, int D, float eps, bool rope, const char *name) {
    if (!ctx || B < 0 || S < 0 || D <= 0 || D % 64 || !q || !qw || (k && !kw) ||
        (rope && !k))
        return set_error(ctx, "%s: invalid arguments (D must be a multiple of 64)", name);
    const long long M = (long long)B * S;
    if (M == 0) return 0;
    const int heads = D / 64;
    const long long G = M * heads * (k ? 2 : 1);
    if (G > INT32_MAX - kHeadRows) return set_error(ctx, "%s: too many rows", name);
    if (((((uintptr_t)q) | ((uintptr_t)qw) | ((uintptr_t)k) | ((uintptr_t)kw)) & 15) != 0)
        return set_error(ctx, "%s: q, k and the weights must be 16-byte aligned", name);
    if (rope && rope_table(ctx, S)) return -1;
    const dim3 grid((unsigned)((G + kHeadRows - 1) / kHeadRows)), block(64);
    if (rope)
        hipLaunchKernelGGL((head_norm_kernel<true>), grid, block, 0, ctx->stream, q, qw, k, kw,
                           ctx->rope, (int)M, S, heads, (int)G, eps);
    else
        hipLaunchKernelGGL((head_norm_kernel<false>), grid, block, 0, ctx->stream, q, qw, k, kw,
                           nullptr, (int)M, S, heads, (int)G, eps);
    IRO_HIP_CHECK_LAUNCH(ctx);
    return 0;
}

int iro_hip_dit_qk_norm_rope(IroHipContext *ctx, float *q, const float *q_weight, float *k,
                             const float *k_weight, int B, int S, int D, float eps) {
    return head_norm(ctx, q, q_weight, k, k_weight, B, S, D, eps, true, "dit_qk_norm_rope");
}

int iro_hip_dit_head_rmsnorm(IroHipContext *ctx, float *x, const float *weight, int B, int S,
                             int D, float eps) {
    return head_norm(ctx, x, weight, nullptr, nullptr, B, S, D, eps, false, "dit_head_rmsnorm");
}

int iro_hip_rmsnorm_f32(IroHipContext *ctx, const float *x, int M, int D, const float *w,
                        float eps, float *y) {
    if (!ctx || !x || !w || !y || M < 0 || D <= 0)
        return set_error(ctx, "rmsnorm_f32: invalid arguments");
    if (M == 0) return 0;
    if (D % 4 || D > 2048 ||
        ((((uintptr_t)x) | ((uintptr_t)w) | ((uintptr_t)y)) & 15) != 0)
        return set_error(ctx, "rmsnorm_f32: needs D %% 4 == 0, D <= 2048 and 16-byte aligned rows");
    const int nj = (D + 255) / 256;
    const size_t pitch_bytes = ((size_t)D + 4) * sizeof(float);
#define IRO_NORM_LAUNCH(RWV, NJV)                                                              \
    hipLaunchKernelGGL((adaln_reg_kernel<RWV, NJV, true>), dim3((M + RWV - 1) / RWV), dim3(64), \
                       RWV * pitch_bytes, ctx->stream, x, nullptr, w, M, M, D, eps, y)
    if (nj <= 2)
        IRO_NORM_LAUNCH(2, 2);
    else if (nj <= 4)
        IRO_NORM_LAUNCH(2, 4);
    else if (nj <= 5)
        IRO_NORM_LAUNCH(2, 5);
    else
        IRO_NORM_LAUNCH(1, 8);
#undef IRO_NORM_LAUNCH
    IRO_HIP_CHECK_LAUNCH(ctx);
    return 0;
}

int iro_hip_dit_stack_create(IroHipContext *ctx, int blocks, int D, int H, int residual_mask,
                             IroHipDiTStack **out) {
    if (!ctx || !out || blocks <= 0 || D <= 0 || H <= 0 || H % 32)
        return set_error(ctx, "dit_stack: invalid shape (H must be a multiple of 32)");
    IroHipDiTStack *s = new (std::nothrow) IroHipDiTStack();
    if (!s) return set_error(ctx, "dit_stack: out of host memory");
    s->ctx = ctx;
    s->blocks = blocks;
    s->D = D;
    s->H = H;
    s->residual_mask = residual_mask & 15;
    s->ada_np = (int)round_up((size_t)6 * D, kNPad);
    if (weight_rows_alloc(ctx, blocks * s->ada_np, D, &s->ada_all)) {
        delete s;
        return -1;
    }
    s->ada_set.assign(blocks, 0);
    s->w_set.assign(blocks, 0);
    s->f32.assign(blocks, IroHipDiTLayerF32{});
    s->f32_set.assign(blocks, 0);
    s->qkvg.assign(blocks, nullptr);
    s->wo.assign(blocks, nullptr);
    s->w13.assign(blocks, nullptr);
    s->w2.assign(blocks, nullptr);
    s->f32w.assign(blocks, IroHipDiTStack::F32Weights{});
    *out = s;
    return 0;
}

int iro_hip_dit_stack_set_block(IroHipDiTStack *s, int block, const float *ada, const float *wq,
                                const float *wk, const float *wv, const float *wgate,
                                const float *wo, const float *w1, const float *w3,
                                const float *w2) {
    if (!s || block < 0 || block >= s->blocks) return -1;
    IroHipContext *ctx = s->ctx;
    if (!wq || !wk || !wv || !wgate || !wo || !w1 || !w3 || !w2)
        return set_error(ctx, "dit_stack: missing block weight");
    const int D = s->D, H = s->H;
    const float *qkvg_parts[4] = {wq, wk, wv, wgate};
    const int qkvg_n[4] = {D, D, D, D};
    const float *w13_parts[2] = {w1, w3};
    const int w13_n[2] = {H, H};
    IroHipWeight *na = nullptr, *nq = nullptr, *no = nullptr, *n13 = nullptr, *n2 = nullptr;
    // The modulation weight is optional: the sampler step and the block
    // forward take the fp32 adaLN parameters instead (dit.c:543-588 has no
    // int8 modulation linear), so only the linear-stack step needs it.
    if ((ada && (iro_hip_weight_create(ctx, ada, 6 * D, D, &na) ||
                 weight_rows_copy(ctx, s->ada_all, block * s->ada_np, na))) ||
        iro_hip_weight_create_fused(ctx, qkvg_parts, qkvg_n, 4, D, 0, &nq) ||
        iro_hip_weight_create(ctx, wo, D, D, &no) ||
        iro_hip_weight_create_fused(ctx, w13_parts, w13_n, 2, D, 1, &n13) ||
        iro_hip_weight_create(ctx, w2, D, H, &n2)) {
        for (IroHipWeight *w : {na, nq, no, n13, n2}) iro_hip_weight_destroy(w);
        return -1;
    }
    // fp32 copies of the groups the int8 mask sends to the fp32 linear
    IroHipDiTStack::F32Weights f;
    const int mask = s->int8_mask;
    const struct {
        float **dst;
        const float *src;
        size_t n;
        int bit;
    } keep[8] = {{&f.wq, wq, (size_t)D * D, 1},  {&f.wk, wk, (size_t)D * D, 1},
                 {&f.wv, wv, (size_t)D * D, 1},  {&f.wg, wgate, (size_t)D * D, 1},
                 {&f.wo, wo, (size_t)D * D, 2},  {&f.w1, w1, (size_t)H * D, 4},
                 {&f.w3, w3, (size_t)H * D, 4},  {&f.w2, w2, (size_t)D * H, 8}};
    hipError_t e = hipSuccess;
    for (const auto &k : keep) {
        if (mask & k.bit || e != hipSuccess) continue;
        e = hipMalloc(k.dst, sizeof(float) * k.n);
        if (e == hipSuccess)
            e = hipMemcpyAsync(*k.dst, k.src, sizeof(float) * k.n, hipMemcpyDeviceToDevice,
                               ctx->stream);
    }
    if (e != hipSuccess) {
        f32_weights_free(f);
        for (IroHipWeight *w : {na, nq, no, n13, n2}) iro_hip_weight_destroy(w);
        return set_error(ctx, "dit_stack: fp32 weight copy failed: %s", hipGetErrorString(e));
    }
    if (na) iro_hip_weight_destroy(na);  // drains the stream: its rows are copied
    for (auto *v : {&s->qkvg, &s->wo, &s->w13, &s->w2}) iro_hip_weight_destroy((*v)[block]);
    f32_weights_free(s->f32w[block]);
    s->f32w[block] = f;
    s->any_set = 1;
    s->qkvg[block] = nq;
    s->wo[block] = no;
    s->w13[block] = n13;
    s->w2[block] = n2;
    s->ada_set[block] = ada != nullptr;
    s->w_set[block] = 1;
    stack_drop_graph(s);
    return 0;
}

// One Euler step's int8 linears: the modulation linears of all blocks,
// then per block QKVG, Wo with the attention gated residual, and the
// SwiGLU MLP with the MLP gated residual.  x [B*S, D] is updated in place;
// cond is [B, D].  The attention core between QKVG and Wo and the
// RMSNorm-modulate before QKVG and W1/W3 are fp32 and outside this path:
// Wo reads V as its input and QKVG/W1W3 read x.
int iro_hip_dit_stack_step(IroHipDiTStack *s, float *x, const float *cond, int B, int S) {
    if (!s || !x || !cond || B <= 0 || S <= 0) return -1;
    IroHipContext *ctx = s->ctx;
    for (int b = 0; b < s->blocks; ++b)
        if (!s->ada_set[b] || !s->w_set[b])
            return set_error(ctx, "dit_stack: block %d has no weights or no modulation weight", b);
    if (stack_reserve(s, B * S, B)) return -1;
    if (stack_persistent(s) && stack_persist_prepare(s, B, S)) return -1;
    {
        int r0[kMaxChains], rows[kMaxChains];
        const int nrun = stack_persistent(s) ? 1 : stack_runs(s, B, S, r0, rows);
        if (nrun > 1 && stack_chain_prepare(s, nrun, rows)) return -1;
    }
    const std::vector<long long> args = {(long long)(uintptr_t)x, (long long)(uintptr_t)cond, B,
                                         S, s->chains};
    return graph_step(ctx, s->graphs, s->use_graph != 0, args,
                      [&]() { return stack_launch(s, x, cond, B, S); }) ||
                   ctx->has_err
               ? -1
               : 0;
}

int iro_hip_dit_stack_block_forward(IroHipDiTStack *s, int block, float *x, int B, int S,
                                    const float *ada_attn, const float *ada_mlp,
                                    const float *q_norm, const float *k_norm, float eps,
                                    const IroHipAttnContext *actx, const float *context_k,
                                    const float *context_v) {
    if (!s || !x || B <= 0 || S <= 0 || !ada_attn || !ada_mlp || !q_norm || !k_norm || !actx ||
        block < 0 || block >= s->blocks)
        return set_error(s ? s->ctx : nullptr, "dit_block_forward: invalid arguments");
    IroHipContext *ctx = s->ctx;
    if (!s->w_set[block]) return set_error(ctx, "dit_block_forward: block %d has no weights", block);
    const int M = B * S, D = s->D;
    if (stack_reserve(s, M, B)) return -1;
    const size_t BD = (size_t)B * D;
    // dit.c:1003-1006: h = RMSNorm-modulate(x) with the attention shift/scale.
    if (iro_hip_dit_adaln_apply(ctx, x, B, S, D, ada_attn, ada_attn + BD, eps, s->h)) return -1;
    // dit.c:785-792: one quantization of h, Q/K/V/gate from the fused weight.
    const SiteBufs o = site_bufs(s, 0);
    if (site_qkvg(s, o, block, s->h, M)) return -1;
    // dit.c:803, 808-870, 872: norm + RoPE, attention core, sigmoid gate.
    if (iro_hip_dit_qk_norm_rope(ctx, s->q, q_norm, s->k, k_norm, B, S, D, eps)) return -1;
    if (iro_hip_dit_attention(ctx, actx, s->q, s->k, s->v, s->g, B, S, D, context_k, context_v,
                              s->mix))
        return -1;
    // dit.c:878-881, 1012-1020: Wo, then x += gate * branch.
    if (site_wo(s, o, block, s->mix, M, x, ada_attn + 2 * BD, D, S)) return -1;
    // dit.c:1022-1039: the MLP half.
    if (iro_hip_dit_adaln_apply(ctx, x, B, S, D, ada_mlp, ada_mlp + BD, eps, s->h)) return -1;
    if (site_mlp(s, o, block, s->h, M, x, ada_mlp + 2 * BD, D, S)) return -1;
    return ctx->has_err ? -1 : 0;
}

int iro_hip_dit_stack_set_layer_f32(IroHipDiTStack *s, int layer, const IroHipDiTLayerF32 *p) {
    if (!s || !p || layer < 0 || layer >= s->blocks)
        return set_error(s ? s->ctx : nullptr, "dit_stack_set_layer_f32: invalid arguments");
    for (int i = 0; i < 18; ++i)
        if (!p->adaln[i]) return set_error(s->ctx, "dit_stack_set_layer_f32: adaLN array %d is NULL", i);
    if (!p->q_norm || !p->k_norm || !p->context_k || !p->context_v)
        return set_error(s->ctx, "dit_stack_set_layer_f32: NULL norm or context array");
    s->f32[layer] = *p;
    s->f32_set[layer] = 1;
    s->sgraphs.drop();  // a captured step holds the previous pointers
    return 0;
}

int iro_hip_dit_stack_set_head(IroHipDiTStack *s, const IroHipDiTHead *head) {
    if (!s || !head || !head->in_w || !head->in_b || !head->out_norm || !head->out_w ||
        !head->out_b || head->latent <= 0 || head->rank <= 0 || !(head->eps >= 0.0f))
        return set_error(s ? s->ctx : nullptr, "dit_stack_set_head: invalid arguments");
    s->head = *head;
    s->head_set = 1;
    s->sgraphs.drop();
    return 0;
}

// sampler.c:259-297 with the reference's calls in its order: iro_dit_input
// (dit.c:532-540) on the state, memcpy to the other CFG rows, per layer
// dit_adaln x 2 (dit.c:580-588) and the block (dit.c:984-1040) with the
// shared context, iro_dit_output (dit.c:1070-1089), the CFG / Euler update.
int iro_hip_dit_sampler_step(IroHipDiTStack *s, float *state, const float *cond, int batch,
                             int S, const IroHipAttnContext *actx, int use_cfg, int text_row,
                             int speaker_row, int caption_row, float scale_text,
                             float scale_speaker, float scale_caption, float dt,
                             float *velocity) {
    if (!s || !state || !cond || !actx || !velocity || batch < 1 || batch > 4 || S <= 0)
        return set_error(s ? s->ctx : nullptr, "dit_sampler_step: invalid arguments");
    IroHipContext *ctx = s->ctx;
    if (!s->head_set) return set_error(ctx, "dit_sampler_step: no head set");
    for (int l = 0; l < s->blocks; ++l)
        if (!s->w_set[l] || !s->f32_set[l])
            return set_error(ctx, "dit_sampler_step: layer %d is not fully set", l);
    // Everything the step reads is checked before its first launch: a plain
    // step (batch 1) may use a context made for the CFG batch (its mask row
    // 0), and the CFG rows must index this step's velocity rows.
    if (actx->ctx != ctx || batch > actx->B)
        return set_error(ctx, "dit_sampler_step: batch %d exceeds the attention context's %d",
                         batch, actx->B);
    if (use_cfg && batch < 2)
        return set_error(ctx, "dit_sampler_step: a CFG step needs at least two rows");
    for (int r : {text_row, speaker_row, caption_row})
        if (r < -1 || r == 0 || r > 3 || (use_cfg && r >= batch))
            return set_error(ctx, "dit_sampler_step: CFG row %d outside 1..%d", r,
                             use_cfg ? batch - 1 : 3);
    const IroHipDiTHead &hd = s->head;
    const int D = s->D, M = batch * S;
    if (stack_reserve(s, M, batch)) return -1;
    auto forward = [&]() -> int {
        if (iro_hip_linear_f32(ctx, state, S, hd.latent, hd.in_w, D, hd.in_b, s->proj)) return -1;
        const size_t rows = sizeof(float) * (size_t)S * D;
        for (int b = 1; b < batch; ++b)
            IRO_HIP_TRY(ctx, hipMemcpyAsync(s->proj + (size_t)b * S * D, s->proj, rows,
                                            hipMemcpyDeviceToDevice, ctx->stream));
        const size_t BD = (size_t)batch * D;
        for (int l = 0; l < s->blocks; ++l) {
            const IroHipDiTLayerF32 &p = s->f32[l];
            if (iro_hip_dit_adaln_params(ctx, cond, batch, D, hd.rank, p.adaln, 2, s->params))
                return -1;
            if (iro_hip_dit_stack_block_forward(s, l, s->proj, batch, S, s->params,
                                                s->params + 3 * BD, p.q_norm, p.k_norm, hd.eps,
                                                actx, p.context_k, p.context_v))
                return -1;
        }
        if (iro_hip_rmsnorm_f32(ctx, s->proj, M, D, hd.out_norm, hd.eps, s->h)) return -1;
        return iro_hip_linear_f32(ctx, s->h, M, D, hd.out_w, hd.latent, hd.out_b, velocity);
    };
    const std::vector<long long> key = {(long long)(uintptr_t)state, (long long)(uintptr_t)cond,
                                        batch, S, (long long)(uintptr_t)actx,
                                        (long long)(uintptr_t)velocity};
    if (graph_step(ctx, s->sgraphs, s->use_graph != 0, key, forward) || ctx->has_err) return -1;
    // sampler.c:281-297, outside the graph: its scalars change every step.
    if (iro_hip_euler_update(ctx, state, velocity, S * hd.latent, batch, use_cfg, text_row,
                             speaker_row, caption_row, scale_text, scale_speaker, scale_caption,
                             dt))
        return -1;
    return ctx->has_err ? -1 : 0;
}

int iro_hip_dit_stack_use_graph(IroHipDiTStack *s, int on) {
    if (!s) return -1;
    s->use_graph = on != 0;
    if (!on) stack_drop_graph(s);
    return 0;
}

int iro_hip_dit_stack_use_persistent(IroHipDiTStack *s, int on) {
    if (!s) return -1;
    IRO_HIP_TRY(s->ctx, hipStreamSynchronize(s->ctx->stream));
    s->use_persist = on != 0;
    stack_drop_graph(s);
    return 0;
}

int iro_hip_dit_stack_set_int8_mask(IroHipDiTStack *s, int mask) {
    if (!s) return -1;
    if (mask < 0 || mask > 15) return set_error(s->ctx, "dit_stack: int8 mask %d outside 0..15", mask);
    if (s->any_set && mask != s->int8_mask)
        return set_error(s->ctx, "dit_stack: set the int8 mask before the blocks' weights");
    s->int8_mask = mask;
    return 0;
}

int iro_hip_dit_stack_get_int8_mask(const IroHipDiTStack *s) { return s ? s->int8_mask : -1; }

int iro_hip_dit_stack_set_runs(IroHipDiTStack *s, int runs) {
    if (!s) return -1;
    if (runs < 0 || runs > kMaxChains)
        return set_error(s->ctx, "dit_stack: runs %d outside 0..%d", runs, kMaxChains);
    IRO_HIP_TRY(s->ctx, hipStreamSynchronize(s->ctx->stream));
    s->chains = runs;
    s->graphs.drop();
    return 0;
}

size_t iro_hip_dit_stack_bytes(const IroHipDiTStack *s) {
    if (!s) return 0;
    size_t n = 0;
    for (int b = 0; b < s->blocks; ++b) {
        if (s->ada_set[b]) n += (size_t)6 * s->D * (s->D + sizeof(float) + sizeof(int32_t));
        if (!s->w_set[b]) continue;
        for (const auto *v : {&s->qkvg, &s->wo, &s->w13, &s->w2}) n += iro_hip_weight_bytes((*v)[b]);
    }
    return n;
}

// Pointers to the last step's scratch outputs: the final block's q, k, v,
// gate [M,D] and hidden [M,H], and the modulation rows of every block
// [B, blocks * ada_np] (block b at column b * ada_np, ada_np = 6D rounded
// up to 256).
int iro_hip_dit_stack_buffers(IroHipDiTStack *s, float **q, float **k, float **v, float **gate,
                              float **hidden, float **mod) {
    if (!s) return -1;
    if (q) *q = s->q;
    if (k) *k = s->k;
    if (v) *v = s->v;
    if (gate) *gate = s->g;
    if (hidden) *hidden = s->hidden;
    if (mod) *mod = s->mod;
    return 0;
}

void iro_hip_dit_stack_destroy(IroHipDiTStack *s) {
    if (!s) return;
    if (s->ctx) (void)hipStreamSynchronize(s->ctx->stream);
    stack_drop_graph(s);
    persist_free(s->persist);
    iro_hip_weight_destroy(s->ada_all);
    for (auto *v : {&s->qkvg, &s->wo, &s->w13, &s->w2})
        for (IroHipWeight *w : *v) iro_hip_weight_destroy(w);
    for (auto &f : s->f32w) f32_weights_free(f);
    for (int c = 0; c < s->nstreams; ++c) {
        (void)hipStreamDestroy(s->side[c]);
        (void)hipEventDestroy(s->join[c]);
    }
    if (s->fork) (void)hipEventDestroy(s->fork);
    for (void *p : s->chain_ws)
        if (p) (void)hipFree(p);
    stack_free_acts(s);
    delete s;
}

}  // extern "C"
