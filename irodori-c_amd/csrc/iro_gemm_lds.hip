// iro_gemm_lds.hip -- the int8 GEMM with both operands staged through LDS by
// direct global-to-LDS copies, many k blocks ahead.
//
// Why.  At the DiT shapes a GEMM tile's time is set by how many bytes it has
// in flight, not by its MFMAs: a timing copy of the register-streamed kernel
// with every MFMA removed runs as long as the real one.  Loads complete in
// issue order, so with weights streamed into a register ring of R k blocks
// every other load is effectively waited for R k blocks after it is issued,
// whatever the program's own waits say.  Here every operand load is a
// direct global-to-LDS copy whose completion the kernel counts itself
// (s_waitcnt vmcnt), and no load the compiler tracks sits in the main loop,
// so NST - 1 k blocks of activation and weight fragments stay in flight per
// workgroup (about 100-130 KiB, enough to cover L2 and MALL latency at the
// MFMA rate).
//
// Layout.  A workgroup of WM x WN waves computes a (WM*32*TI) x (WN*32*TJ)
// tile; wave (wm, wn) owns rows wm*32*TI .. and columns wn*32*TJ .. as TI x
// TJ tiles of v_mfma_i32_32x32x32_i8.  One pipeline stage is one k block
// (32 bytes of k): the tile's activation fragments (BM/32 per plane) and
// weight fragments (BN/32), each the 1 KiB MFMA operand a wave reads with
// one 16-byte LDS load per lane (the activation in the row/k order of the
// fragment, the weight exactly as it is pre-packed).  Waves issue the copies
// of a stage round-robin, a fixed number each (the rest copy the zero page
// into a sink), so every wave can wait for its own copies of stage kb with
// one vmcnt and a barrier then publishes all of them.
//
// Arithmetic and epilogues are those of iro_gemm_core.h: activation codes
// are signed (a ^ 0x80), the accumulators start at 0 and the epilogue adds
// 128 * rowsum, so the raw sums, and every output bit, equal the other
// kernels'.
#include "iro_gemm_core.h"

namespace iro {

namespace {

template <int VM>
__device__ __forceinline__ void lds_wait_vm() {
    static_assert(VM < 64, "vmcnt holds 6 bits");
    __builtin_amdgcn_s_waitcnt((VM & 15) | (7 << 4) | (15 << 8) | ((VM >> 4) << 14));
}

template <int CONV, int EPI, bool TWO, int WM, int WN, int TI, int TJ, int NST>
__global__ __launch_bounds__(64 * WM * WN, 1) void gemm_lds_kernel(KParams p) {
    constexpr int W = WM * WN, NT = 64 * W, PL = TWO ? 2 : 1;
    constexpr int BMW = 32 * TI, BM = WM * BMW, BN = WN * 32 * TJ;
    constexpr int RB = BM / 32;        // activation row blocks of the tile
    constexpr int FA = RB * PL;        // activation fragments per k block
    constexpr int FB = BN / 32;        // weight fragments per k block
    constexpr int F = FA + FB;
    constexpr int PW = (F + W - 1) / W;  // copies per wave per stage
    constexpr int STG = F * 1024;
    constexpr int VMW = (NST - 2) * PW;  // copies younger than a stage's own
    static_assert(NST >= 3 && VMW < 64, "pipeline depth");
    __shared__ __attribute__((aligned(16))) uint8_t lds[NST * STG];
    __shared__ __attribute__((aligned(16))) uint8_t sink[1024];  // never read
    __shared__ __attribute__((aligned(16))) RowLds<BMW, TWO> rl[WM];
    __shared__ uint64_t exptab[32];

    int bx, by;
    if (!tile_of(blockIdx.x, p.tiles_m, p.tiles_n, p.tiles_per_xcd, p.row_major, bx, by)) return;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int m0 = by * BM;
    const int n0b = bx * FB;  // first packed 32-column weight block of the tile

    // Row parameters per wave row group (the epilogue indexes them from the
    // group's first row).
    for (int t = tid; t < BM; t += NT) {
        const int g = t / BMW, r = t - g * BMW;
        int m = m0 + t;
        m = m < p.M ? m : p.M - 1;
        rl[g].sx[0][r] = p.sx1[m];
        rl[g].zx[0][r] = p.zx1[m];
        if (TWO) {
            rl[g].sx[TWO ? 1 : 0][r] = p.sx2[m];
            rl[g].zx[TWO ? 1 : 0][r] = p.zx2[m];
        }
        if (EPI == EPI_GATED) rl[g].goff[r] = (m / p.rows_per_branch) * p.ldg;
    }
    if (EPI == EPI_SWIGLU && tid < 32) exptab[tid] = kExp2Tab[tid];
    // A wave row group may lie wholly past M (the tile's last rows): it
    // stores nothing, and its gate rows are taken at row M-1 so that the
    // gated epilogue's parameter loads stay inside the gate array.
    const int m0w = m0 + wm * BMW;
    const bool rows_live = m0w < p.M;
    const int nb0 = n0b + wn * TJ;
    const ColParams<TJ> cp = load_cols<EPI, TJ>(p, nb0, lane, rows_live ? m0w : p.M - 1, BMW);

    // Copy i of this wave is fragment f = wave + W i of every stage:
    // activation plane f / RB, row block f % RB (lane L: row 32 rb + L % 32,
    // k bytes 16 (L / 32) .. +15 of the k block; rows past M repeat row
    // M-1, never stored), or weight block f - FA (lane L: its 16 bytes of
    // the packed fragment).  Per k block the source advances by 32 bytes
    // (activation) or 1 KiB (weight).
    const uint8_t *src[PW];
    int adv[PW];
#pragma unroll
    for (int i = 0; i < PW; ++i) {
        const int f = wave + W * i;
        if (f < FA && p.akbp > 0) {
            // fragment-layout codes: one contiguous 1 KiB per fragment (row
            // blocks past the last one repeat it; never stored)
            const int pl = f / RB, rb = f - pl * RB;
            int g = m0 / 32 + rb;
            const int glast = (p.M - 1) / 32;
            g = g < glast ? g : glast;
            src[i] = (pl ? p.a2 : p.a1) + ((size_t)g * p.akbp * 64 + lane) * 16;
            adv[i] = 1024;
        } else if (f < FA) {
            const int pl = f / RB, rb = f - pl * RB;
            int row = m0 + rb * 32 + (lane & 31);
            row = row < p.M ? row : p.M - 1;
            src[i] = (pl ? p.a2 : p.a1) + (size_t)row * p.lda + (lane >> 5) * 16;
            adv[i] = 32;
        } else if (f < F) {
            src[i] = reinterpret_cast<const uint8_t *>(p.bp) +
                     (size_t)(n0b + f - FA) * p.kb_count * 1024 + lane * 16;
            adv[i] = 1024;
        } else {
            src[i] = p.zero16;
            adv[i] = 0;
        }
    }
    const int nkb = p.K / 32;
    auto issue = [&](int kb) {
        uint8_t *base = lds + (kb % NST) * STG;
#pragma unroll
        for (int i = 0; i < PW; ++i) {
            const int f = wave + W * i;
            if (f < F && kb < nkb)
                dma16(src[i] + (size_t)kb * adv[i], base + f * 1024);
            else
                dma16(p.zero16, sink);
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

#pragma unroll
    for (int s = 0; s < NST - 1; ++s) issue(s);
    for (int kb = 0; kb < nkb; ++kb) {
        // This wave's copies of stage kb have landed once at most the NST-2
        // younger stages' copies are outstanding; the barrier publishes the
        // other waves' copies and frees the buffer of stage kb-1.
        lds_wait_vm<VMW>();
        __syncthreads();
        issue(kb + NST - 1);
        const uint8_t *st = lds + (kb % NST) * STG;
        v4i a[PL][TI], b[TJ];
#pragma unroll
        for (int pl = 0; pl < PL; ++pl)
#pragma unroll
            for (int i = 0; i < TI; ++i)
                a[pl][i] = *reinterpret_cast<const v4i *>(
                    st + ((pl * RB + wm * TI + i) * 64 + lane) * 16);
#pragma unroll
        for (int j = 0; j < TJ; ++j)
            b[j] = *reinterpret_cast<const v4i *>(st + ((FA + wn * TJ + j) * 64 + lane) * 16);
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[0][i], b[j], acc[i][j], 0, 0, 0);
                if (TWO)
                    acc2[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[PL - 1][i], b[j],
                                                                       acc2[i][j], 0, 0, 0);
            }
    }
    // The last stages' sink copies may still be in flight: no copy into this
    // block's LDS may outlive it.
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
    if (rows_live)
        epilogue<CONV, EPI, TWO, TI, TJ, BMW>(p, acc, acc2, cp, rl[wm], exptab, m0w, nb0, lane);
}

}  // namespace

// Shapes of the LDS-pipelined kernel (rows x columns per workgroup).
enum LdsCfg {
    LDS_192x256 = 1,  // 2 x 4 waves of 96 x 64 (one plane)
    LDS_96x128 = 2,   // 1 x 4 waves of 96 x 32 (one or two planes)
    LDS_128x256 = 3,  // 2 x 4 waves of 64 x 64 (one plane)
    LDS_96x256 = 4,   // 1 x 4 waves of 96 x 64 (one plane)
    LDS_64x128 = 5,   // 1 x 4 waves of 64 x 32 (one or two planes)
};

void lds_tile_shape(int cfg, int *bm, int *bn) {
    switch (cfg) {
        case LDS_192x256: *bm = 192; *bn = 256; return;
        case LDS_96x128: *bm = 96; *bn = 128; return;
        case LDS_128x256: *bm = 128; *bn = 256; return;
        case LDS_96x256: *bm = 96; *bn = 256; return;
        default: *bm = 64; *bn = 128; return;
    }
}

bool lds_cfg_ok(int cfg, bool two, int epi) {
    if (cfg < LDS_192x256 || cfg > LDS_64x128) return false;
    const bool wide = cfg == LDS_192x256 || cfg == LDS_128x256 || cfg == LDS_96x256;
    if (two && wide) return false;                      // two planes: 32-column waves
    if (epi == EPI_SWIGLU && !wide) return false;       // W1/W3 column pairs per wave
    return true;
}

template <int CONV, int EPI>
void launch_lds_e(const KParams &kp, bool two, int cfg, unsigned grid, hipStream_t st) {
#define IRO_LDS(TWO_, WM_, WN_, TI_, TJ_, NST_)                                               \
    hipLaunchKernelGGL((gemm_lds_kernel<CONV, EPI, TWO_, WM_, WN_, TI_, TJ_, NST_>), dim3(grid), \
                       dim3(64 * WM_ * WN_), 0, st, kp)
    if (cfg == LDS_192x256) {
        IRO_LDS(false, 2, 4, 3, 2, 10);  // 14 KiB stages
    } else if (cfg == LDS_128x256) {
        IRO_LDS(false, 2, 4, 2, 2, 11);  // 12 KiB stages
    } else if (cfg == LDS_96x256) {
        IRO_LDS(false, 1, 4, 3, 2, 13);  // 11 KiB stages
    } else if (cfg == LDS_96x128) {
        if constexpr (EPI != EPI_SWIGLU) {
            if (two)
                IRO_LDS(true, 1, 4, 3, 1, 14);  // 10 KiB stages
            else
                IRO_LDS(false, 1, 4, 3, 1, 20);  // 7 KiB stages
        }
    } else {
        if constexpr (EPI != EPI_SWIGLU) {
            if (two)
                IRO_LDS(true, 1, 4, 2, 1, 16);  // 8 KiB stages
            else
                IRO_LDS(false, 1, 4, 2, 1, 20);  // 6 KiB stages
        }
    }
#undef IRO_LDS
}

void launch_lds(const KParams &kp, int conv, int epi, bool two, int cfg, unsigned grid,
                hipStream_t st) {
    if (conv == IRO_HIP_GCC_FASTMATH) {
        switch (epi) {
            case EPI_LINEAR: launch_lds_e<1, EPI_LINEAR>(kp, two, cfg, grid, st); break;
            case EPI_QKVG: launch_lds_e<1, EPI_QKVG>(kp, two, cfg, grid, st); break;
            case EPI_SWIGLU: launch_lds_e<1, EPI_SWIGLU>(kp, two, cfg, grid, st); break;
            default: launch_lds_e<1, EPI_GATED>(kp, two, cfg, grid, st); break;
        }
    } else {
        switch (epi) {
            case EPI_LINEAR: launch_lds_e<0, EPI_LINEAR>(kp, two, cfg, grid, st); break;
            case EPI_QKVG: launch_lds_e<0, EPI_QKVG>(kp, two, cfg, grid, st); break;
            case EPI_SWIGLU: launch_lds_e<0, EPI_SWIGLU>(kp, two, cfg, grid, st); break;
            default: launch_lds_e<0, EPI_GATED>(kp, two, cfg, grid, st); break;
        }
    }
}

}  // namespace iro
