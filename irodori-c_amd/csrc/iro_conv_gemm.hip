// iro_conv_gemm.hip -- the int8 Conv1d with kernel 7 (dacvae.c:543-688) as
// one GEMM whose activation loader codes the input rows itself, so no
// im2col codes pass through HBM.
//
// The codes of output step t are x[t*stride - padding + tap*dilation, c]
// under t's own scale and zero point, set by the range of its whole 7*C
// window (dacvae.c:617-636).  conv_rows (iro_conv.hip) gives every input
// row's lo/hi; a block reduces them over the taps of its 64 output steps,
// which is exactly the window range (min and max only select), so the row
// parameters and the codes are the im2col kernels' bit for bit.  The second
// plane (dacvae.c:637-663, scale s/255, zero point 128) is coded from the
// same loaded values.
//
// Block: 256 threads, 64 output steps x 128*TJ output channels, four waves
// side by side along N, each a 64 x 32*TJ tile of v_mfma_i32_32x32x32_i8.
// k runs in chunks of 128 (C % 16 == 0, so each 16-column piece lies in one
// tap): per chunk every thread codes two 16-value pieces per plane into LDS
// in fragment order (signed operand form, a ^ 0x80), the inputs of the next
// chunk being loaded into registers while the MFMAs of this one run; one
// barrier per chunk.  Each wave streams its weight fragments from the packed
// buffer one chunk ahead.  Padding taps code the zero point (plane 2: 128);
// k at or past 7*C codes the signed zero, against zero weights.  Rows past
// T_out repeat row T_out - 1 and are never stored.
// Roofline: HBM, the input once (its taps re-read from L2) and the output
// once, against 2 * 7C * N ops per output step and plane.
#include "iro_gemm_core.h"
#include "iro_conv_row.h"

namespace iro {
namespace {

constexpr int kCvKC = 128;  // k bytes per chunk
constexpr int kCvBM = 64;   // output steps per block

template <int CONV, bool TWO, int TJ>
__global__ __launch_bounds__(256, 2) void conv7_gemm_kernel(KParams p, ConvRows cr) {
    constexpr int TI = 2, BM = kCvBM, PL = TWO ? 2 : 1, KC = kCvKC, KBC = KC / 32;
    constexpr int PLANE = BM * KC;         // LDS bytes per plane per chunk
    constexpr int PPT = PLANE / 16 / 256;  // pieces per thread per plane
    static_assert(BM == 32 * TI && PPT * 256 * 16 == PLANE, "piece geometry");
    __shared__ __attribute__((aligned(16))) uint8_t lds_a[2][PL * PLANE];
    __shared__ __attribute__((aligned(16))) RowLds<BM, TWO> rl;
    __shared__ float r_inv[BM], r_zpf[BM], r_s[BM], r_inv2[BM];

    int bx, by;
    if (!tile_of(blockIdx.x, p.tiles_m, p.tiles_n, p.tiles_per_xcd, p.row_major, bx, by)) return;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m0 = by * BM;
    const int nb0 = bx * 4 * TJ + wave * TJ;  // first packed 32-row weight block of this wave
    const int C = cr.C;

    // Row parameters of the block's output steps (dacvae.c:617-652).
    if (tid < BM) {
        int t = m0 + tid;
        t = t < p.M ? t : p.M - 1;
        const int base = t * cr.stride - cr.padding;
        float lo = 0.0f, hi = 0.0f;
#pragma unroll
        for (int tap = 0; tap < 7; ++tap) {
            const int it = base + tap * cr.dilation;
            if (it >= 0 && it < cr.T) {
                lo = sel_min(lo, cr.row_lo[it]);
                hi = sel_max(hi, cr.row_hi[it]);
            }
        }
        const RowQ q = row_params<CONV>(lo, hi);
        float sc2 = 0.0f, inv2 = 0.0f;
        if (TWO) conv_plane2_params<CONV>(q, lo, hi, sc2, inv2);
        rl.sx[0][tid] = q.s;
        rl.zx[0][tid] = q.zp;
        if (TWO) {
            rl.sx[TWO ? 1 : 0][tid] = sc2;
            rl.zx[TWO ? 1 : 0][tid] = 128;
        }
        r_inv[tid] = q.inv;
        r_zpf[tid] = q.zpf;
        r_s[tid] = q.s;
        r_inv2[tid] = inv2;
    }
    const ColParams<TJ> cp = load_cols<EPI_LINEAR, TJ>(p, nb0, lane, m0, BM);

    // Pieces of this thread: piece q = tid + 256 i of a plane's chunk is
    // fragment f = q / 64 = [k block q / 64 / TI][row block f % TI], lane
    // q % 64 of it: row (f % TI) * 32 + q % 32, k offset 16 ((q % 64) / 32).
    // Its tap and channel advance by 128 per chunk (C >= 64: at most two
    // wraps per chunk).
    int prow[PPT], pbase[PPT], ptap[PPT], pch[PPT];
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
        const int q = tid + 256 * i, f = q >> 6, ln = q & 63;
        prow[i] = (f % TI) * 32 + (ln & 31);
        int t = m0 + prow[i];
        t = t < p.M ? t : p.M - 1;
        pbase[i] = t * cr.stride - cr.padding;
        const int k = (f / TI) * 32 + (ln >> 5) * 16;
        ptap[i] = k / C;
        pch[i] = k - ptap[i] * C;
    }
    // Inputs of one chunk: per piece 16 floats, or a marker for padding
    // taps (kind 1) and k past 7C (kind 2).
    float4 xv[PPT][4];
    int kind[PPT];
    auto load_x = [&]() {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int it = pbase[i] + ptap[i] * cr.dilation;
            kind[i] = ptap[i] >= 7 ? 2 : (it >= 0 && it < cr.T ? 0 : 1);
            if (kind[i] == 0) {
                const float4 *src = reinterpret_cast<const float4 *>(cr.x + (size_t)it * C + pch[i]);
#pragma unroll
                for (int g = 0; g < 4; ++g) xv[i][g] = src[g];
            }
            // next chunk's tap and channel
            pch[i] += KC;
            if (pch[i] >= C) { pch[i] -= C; ++ptap[i]; }
            if (pch[i] >= C) { pch[i] -= C; ++ptap[i]; }
        }
    };
    auto code_x = [&](int buf) {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int r = prow[i];
            RowQ q;
            q.s = r_s[r];
            q.inv = r_inv[r];
            q.zpf = r_zpf[r];
            q.zp = rl.zx[0][r];
            v4i w1, w2;
            if (kind[i] == 0) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const float4 e = xv[i][g];
                    const uint32_t c1 = pack_codes4(quant_pre<CONV>(e.x, q), quant_pre<CONV>(e.y, q),
                                                    quant_pre<CONV>(e.z, q), quant_pre<CONV>(e.w, q));
                    w1[g] = (int)(c1 ^ 0x80808080u);
                    if (TWO) {
                        const float inv2 = r_inv2[r];
                        const float4 c4 = unpack_codes4(c1);
                        const uint32_t c2 = pack_codes4(plane2_pre<CONV>(e.x, c4.x, q, inv2),
                                                        plane2_pre<CONV>(e.y, c4.y, q, inv2),
                                                        plane2_pre<CONV>(e.z, c4.z, q, inv2),
                                                        plane2_pre<CONV>(e.w, c4.w, q, inv2));
                        w2[g] = (int)(c2 ^ 0x80808080u);
                    }
                }
            } else {
                // padding tap: the zero point (plane 2: 128); past 7C: signed 0
                const int z = kind[i] == 1 ? (int)((0x01010101u * (uint32_t)q.zp) ^ 0x80808080u) : 0;
                w1 = v4i{z, z, z, z};
                w2 = v4i{0, 0, 0, 0};
            }
            const int q16 = (tid + 256 * i) * 16;
            *reinterpret_cast<v4i *>(&lds_a[buf][q16]) = w1;
            if (TWO) *reinterpret_cast<v4i *>(&lds_a[buf][PLANE + q16]) = w2;
        }
    };

    const __amdgpu_buffer_rsrc_t wr = weight_rsrc(p);
    const int jstride = p.kb_count * 1024;  // bytes between 32-row weight blocks
    const int wbase = nb0 * jstride;
    const int nc = (p.K + KC - 1) / KC;
    auto load_b = [&](v4i (&dst)[KBC][TJ], int c) {
#pragma unroll
        for (int u = 0; u < KBC; ++u) {
            int kb = c * KBC + u;
            kb = kb < p.kb_count ? kb : p.kb_count - 1;
#pragma unroll
            for (int j = 0; j < TJ; ++j) dst[u][j] = load_frag(wr, lane * 16, wbase + j * jstride + kb * 1024);
        }
    };

    v16i acc[TI][TJ], acc2[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                acc[i][j][r] = 0;
                acc2[i][j][r] = 0;
            }

    v4i bcur[KBC][TJ], bnext[KBC][TJ];
    load_b(bcur, 0);
    load_x();
    __syncthreads();  // row parameters
    code_x(0);
    __syncthreads();
    for (int c = 0; c < nc; ++c) {
        const bool more = c + 1 < nc;
        if (more) {
            load_b(bnext, c + 1);
            load_x();
        }
        const uint8_t *abuf = lds_a[c & 1];
#pragma unroll
        for (int u = 0; u < KBC; ++u) {
            v4i a[PL][TI];
#pragma unroll
            for (int pl = 0; pl < PL; ++pl)
#pragma unroll
                for (int i = 0; i < TI; ++i)
                    a[pl][i] = *reinterpret_cast<const v4i *>(abuf + pl * PLANE +
                                                             ((u * TI + i) * 64 + lane) * 16);
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[0][i], bcur[u][j], acc[i][j], 0, 0, 0);
                    if (TWO)
                        acc2[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[PL - 1][i], bcur[u][j],
                                                                           acc2[i][j], 0, 0, 0);
                }
        }
        if (more) code_x((c + 1) & 1);
        __syncthreads();
#pragma unroll
        for (int u = 0; u < KBC; ++u)
#pragma unroll
            for (int j = 0; j < TJ; ++j) bcur[u][j] = bnext[u][j];
    }

    epilogue<CONV, EPI_LINEAR, TWO, TI, TJ, BM>(p, acc, acc2, cp, rl, nullptr, m0, nb0, lane);
}

}  // namespace

// Shapes the kernel takes.  It is chosen only up to 256 channels: each lane
// of an MFMA activation fragment holds its own row, so the loader's vector
// loads touch 32 rows each and its coding work is repeated per column tile;
// that beats writing and re-reading the im2col codes where they dominate
// (C = 96: 323 against 530 us per decoder Conv7, C = 192: 314 against 350
// us) and loses where the GEMM does (C = 384: 130 against 101 us, C = 768
// and the 512-channel Conv1d: about twice the time).
bool conv7_gemm_ok(const IroHipWeight *w, const ConvRows &cr) {
    return cr.C % 16 == 0 && cr.C >= 64 && cr.C <= 256 && (((uintptr_t)cr.x) & 15) == 0 &&
           w->Np % 128 == 0 && w->K == 7 * cr.C && w->layout == 0;
}

int launch_conv7_gemm(IroHipContext *ctx, const IroHipWeight *w, const ConvRows &cr, int T_out,
                      bool two, const float *bias, float *y) {
    if (!conv7_gemm_ok(w, cr)) return 1;
    GemmArgs a;
    a.M = T_out;
    a.K = w->K;
    a.bias = bias;
    a.y = y;
    a.ldy = w->N;
    KParams kp;
    if (fill_kparams(ctx, w, a, kp)) return -1;
    // 64 x 256 tiles for one plane; two planes keep 64 x 128 (their
    // accumulators would not fit twice).
    const int tj = !two && w->Np % 256 == 0 ? 2 : 1;
    kp.tiles_n = w->Np / (128 * tj);
    kp.tiles_m = (T_out + kCvBM - 1) / kCvBM;
    const int tiles = kp.tiles_n * kp.tiles_m;
    kp.tiles_per_xcd = (tiles + 7) / 8;
    // Row tiles run in order on each XCD: neighbouring output steps share
    // their input rows in its L2.
    kp.row_major = 1;
    const dim3 grid((unsigned)(8 * kp.tiles_per_xcd)), block(256);
    prof_begin(ctx);
#define IRO_CG(CV, TW, TJ)                                                                    \
    hipLaunchKernelGGL((conv7_gemm_kernel<CV, TW, TJ>), grid, block, 0, ctx->stream, kp, cr)
    const bool fast = ctx->convention == IRO_HIP_GCC_FASTMATH;
    if (fast) {
        if (two) IRO_CG(1, true, 1);
        else if (tj == 2) IRO_CG(1, false, 2);
        else IRO_CG(1, false, 1);
    } else {
        if (two) IRO_CG(0, true, 1);
        else if (tj == 2) IRO_CG(0, false, 2);
        else IRO_CG(0, false, 1);
    }
#undef IRO_CG
    IRO_HIP_CHECK_LAUNCH(ctx);
    // Algorithmic work: 2 * 7C * N per output step and plane; bytes: the
    // input once, the weight once, the output once.
    const double planes = two ? 2 : 1;
    prof_end(ctx, PK_CONV_GEMM, 2.0 * T_out * w->N * w->K * planes,
             4.0 * cr.T * cr.C + (double)w->N * w->K + 4.0 * T_out * w->N);
    return 0;
}

}  // namespace iro
