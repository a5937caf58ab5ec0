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
// The reduction runs over 32-channel blocks with the 7 taps inside (integer
// sums are exact in any order; the weight fragment of tap j, channel block
// cb is k block j * C/32 + cb of the packed [N, 7C] weight).  Per
// channel block the block loads its input window -- rows m0*stride -
// padding .. + 63*stride + 6*dilation, 32 channels, rows outside [0, T) as
// 0 -- once into LDS with coalesced loads (each input value is read once
// per block instead of once per tap), codes the 7 taps' activation
// fragments from it into LDS (signed operand form, a ^ 0x80; a padding row
// of zeros codes the zero point, and 128 in plane 2, exactly the padding
// codes), and runs the 7 k blocks of MFMAs, the next window's loads and the
// weight fragments in flight meanwhile.  Rows past T_out repeat row
// T_out - 1 and are never stored.
// Roofline: HBM, the input once (its windows overlap by 6*dilation rows
// from L2) and the output once, against 2 * 7C * N ops per output step and
// plane.
#include "iro_gemm_core.h"
#include "iro_conv_row.h"
#include "iro_quant_row.h"
#include "iro_snake.h"

namespace iro {
namespace {

constexpr int kCvBM = 64;     // output steps per block
constexpr int kCvWRows = 128;  // input window rows per block, at most
constexpr int kCvWPitch = 36;  // floats per LDS window row (32 + 4: spreads banks)

template <int CONV, bool TWO, int TJ>
__global__ __launch_bounds__(256, 2) void conv7_gemm_kernel(KParams p, ConvRows cr) {
    constexpr int TI = 2, BM = kCvBM, PL = TWO ? 2 : 1;
    constexpr int FR = 7 * TI;             // activation fragments per plane per channel block
    constexpr int APLANE = FR * 64 * 16;   // LDS bytes per plane
    constexpr int WLD = kCvWRows * 8 / 256;  // window float4 loads per thread, at most
    __shared__ __attribute__((aligned(16))) float xw[kCvWRows * kCvWPitch];
    __shared__ __attribute__((aligned(16))) uint8_t lds_a[PL * APLANE];
    __shared__ __attribute__((aligned(16))) RowLds<BM, TWO> rl;
    __shared__ float r_inv[BM], r_zpf[BM], r_s[BM], r_inv2[BM];

    int bx, by;
    if (!tile_of(blockIdx.x, p.tiles_m, p.tiles_n, p.tiles_per_xcd, p.row_major, bx, by)) return;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m0 = by * BM;
    const int nb0 = bx * 4 * TJ + wave * TJ;  // first packed 32-row weight block of this wave
    const int C = cr.C, cbs = C / 32;
    const int w0 = m0 * cr.stride - cr.padding;                // first window row
    const int wrows = 63 * cr.stride + 6 * cr.dilation + 1;   // <= kCvWRows

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

    // Window of channel block cb: float4 i = tid + 256 u is row i / 8,
    // channels 4 (i % 8) .. +3 of the block.
    float4 wv[WLD];
    auto load_window = [&](int cb) {
#pragma unroll
        for (int u = 0; u < WLD; ++u) {
            const int i = tid + 256 * u, r = i >> 3, gr = w0 + r;
            wv[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (r < wrows && gr >= 0 && gr < cr.T)
                wv[u] = *reinterpret_cast<const float4 *>(cr.x + (size_t)gr * C + cb * 32 +
                                                          4 * (i & 7));
        }
    };
    auto store_window = [&]() {
#pragma unroll
        for (int u = 0; u < WLD; ++u) {
            const int i = tid + 256 * u, r = i >> 3;
            if (r < wrows) *reinterpret_cast<float4 *>(&xw[r * kCvWPitch + 4 * (i & 7)]) = wv[u];
        }
    };
    // Fragment f = tap * TI + rb, lane ln: output row rb*32 + ln % 32,
    // channels 16 (ln / 32) .. +15 of window row row*stride + tap*dilation.
    auto code_window = [&]() {
        for (int pc = tid; pc < FR * 64; pc += 256) {
            const int f = pc >> 6, ln = pc & 63, tap = f / TI, rb = f - tap * TI;
            const int r = rb * 32 + (ln & 31);
            const float *src = &xw[(r * cr.stride + tap * cr.dilation) * kCvWPitch + (ln >> 5) * 16];
            RowQ q;
            q.s = r_s[r];
            q.inv = r_inv[r];
            q.zpf = r_zpf[r];
            q.zp = rl.zx[0][r];
            v4i w1, w2;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float4 e = *reinterpret_cast<const float4 *>(src + 4 * g);
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
            *reinterpret_cast<v4i *>(&lds_a[pc * 16]) = w1;
            if (TWO) *reinterpret_cast<v4i *>(&lds_a[APLANE + pc * 16]) = w2;
        }
    };

    const __amdgpu_buffer_rsrc_t wr = weight_rsrc(p);
    const int jstride = p.kb_count * 1024;  // bytes between 32-row weight blocks
    const int wbase = nb0 * jstride;
    v4i bf[7][TJ];
    auto load_b = [&](int cb) {
#pragma unroll
        for (int tap = 0; tap < 7; ++tap)
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                bf[tap][j] = load_frag(wr, lane * 16, wbase + j * jstride + (tap * cbs + cb) * 1024);
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

    load_window(0);
    for (int cb = 0; cb < cbs; ++cb) {
        load_b(cb);
        store_window();
        __syncthreads();  // the window (and, first time round, the row parameters)
        code_window();
        __syncthreads();
        if (cb + 1 < cbs) load_window(cb + 1);
#pragma unroll
        for (int tap = 0; tap < 7; ++tap) {
            v4i a[PL][TI];
#pragma unroll
            for (int pl = 0; pl < PL; ++pl)
#pragma unroll
                for (int i = 0; i < TI; ++i)
                    a[pl][i] = *reinterpret_cast<const v4i *>(&lds_a[pl * APLANE +
                                                                     ((tap * TI + i) * 64 + lane) * 16]);
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[0][i], bf[tap][j], acc[i][j], 0, 0, 0);
                    if (TWO)
                        acc2[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[PL - 1][i], bf[tap][j],
                                                                           acc2[i][j], 0, 0, 0);
                }
        }
        // The next round's window store and codes overwrite LDS the MFMAs
        // above read: every wave passes the barrier after its MFMAs.
        __syncthreads();
    }

    epilogue<CONV, EPI_LINEAR, TWO, TI, TJ, BM>(p, acc, acc2, cp, rl, nullptr, m0, nb0, lane);
}

// The 1x1 of a decoder residual unit (dacvae.c:967-1012) as one kernel:
// the in-place snake_bias of conv0's output (snake_bias_forward,
// dacvae.c:910-931, reciprocal form), the row quantization of the result
// (ops.c:321-348; two-term ops.c:427-442 with RES), the GEMM and
// output = skip + lin(q1) + bias (+ lin(q2)) -- so neither the snaked rows
// nor their codes reach HBM.  With C <= 192 a block of 32 * TI rows holds
// whole rows (LDS: the tile, the codes and the per-channel parameters within
// 64 KiB): phase 1 copies them into an LDS tile as flat float4 chunks (every
// lane busy) and snakes them there in place with per-channel bias, alpha
// and reciprocal from LDS; phase 2 quantizes each tile row with the
// eight-lane row quantizer of iro_quant_row.h (quant_row_g8), writing
// the codes into LDS in MFMA fragment order and the row parameters where the
// epilogue reads them; then each wave runs the C/32 k blocks of MFMAs
// against its weight fragments and the epilogue adds the skip rows.  One
// column tile covers all N (TJ = Np / 128).  Rows past M hold zeros and are
// never stored.

template <int CONV, bool TWO, int TJ, int TI>
__global__ __launch_bounds__(256, TI == 1 ? 4 : 2) void conv1x1_snake_kernel(KParams p, const float *__restrict__ hid,
                                                               const float *__restrict__ sbias,
                                                               const float *__restrict__ salpha,
                                                               unsigned k4_magic) {
    constexpr int BM = 32 * TI, PL = TWO ? 2 : 1;
    extern __shared__ __attribute__((aligned(16))) float rs_lds[];
    __shared__ uint32_t s_pio4[24];
    __shared__ __attribute__((aligned(16))) RowLds<BM, TWO> rl;
    const int C = p.K, KB = C / 32, pitch = C;
    float *s_b = rs_lds, *s_a = s_b + C, *s_i = s_a + C, *tile = s_i + C;
    uint8_t *codes = reinterpret_cast<uint8_t *>(tile + BM * pitch);  // PL planes of BM x C
    const int plane = BM * C;

    int bx, by;
    if (!tile_of(blockIdx.x, p.tiles_m, p.tiles_n, p.tiles_per_xcd, p.row_major, bx, by)) return;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m0 = by * BM;
    const int nb0 = bx * 4 * TJ + wave * TJ;

    stage_invpio4(s_pio4, tid);
    for (int c = tid; c < C; c += 256) {
        const float a = salpha[c];
        s_b[c] = sbias[c];
        s_a[c] = a;
        s_i[c] = snake_inv(a);
    }
    const ColParams<TJ> cp = load_cols<EPI_LINEAR, TJ>(p, nb0, lane, m0, BM);
    // Phase 1: float4 f = tid + 256 u of the block is row f / (C/4).
    // The raw rows go to the tile first, eight float4 loads per thread in
    // flight at a time, and are snaked there in place by a loop that is not
    // unrolled (one copy of the snake's code).  Rows past M stay zero.
    const int k4 = C >> 2, chunks = BM * k4;  // <= 64 * 64
    constexpr int G = 8;
    for (int base = 0; base < chunks; base += 256 * G) {
        float4 v4[G];
#pragma unroll
        for (int u = 0; u < G; ++u) {
            const int f = base + tid + 256 * u;
            v4[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (f < chunks && m0 + (int)__umulhi(2u * f, k4_magic) < p.M)
                v4[u] = *reinterpret_cast<const float4 *>(hid + (size_t)m0 * C + 4 * f);
        }
#pragma unroll
        for (int u = 0; u < G; ++u) {
            const int f = base + tid + 256 * u;
            if (f < chunks) *reinterpret_cast<float4 *>(tile + 4 * f) = v4[u];
        }
    }
    __syncthreads();  // the staged parameters and rows
    const int live = (p.M - m0 < BM ? p.M - m0 : BM) * k4;  // chunks of rows below M
#pragma unroll 1
    for (int f = tid; f < live; f += 256) {
        const int c4 = f - (int)__umulhi(2u * f, k4_magic) * k4;
        const float4 v = *reinterpret_cast<const float4 *>(tile + 4 * f);
        const float4 b = *reinterpret_cast<const float4 *>(s_b + 4 * c4);
        const float4 a = *reinterpret_cast<const float4 *>(s_a + 4 * c4);
        const float4 i = *reinterpret_cast<const float4 *>(s_i + 4 * c4);
        const float4 xv = make_float4(v.x + b.x, v.y + b.y, v.z + b.z, v.w + b.w);
        *reinterpret_cast<float4 *>(tile + 4 * f) = snake_value4<true, CONV == 1>(xv, a, i, s_pio4);
    }
    __syncthreads();
    // Phase 2: row quantization from the tile, codes in fragment order;
    // eight lanes per row (32 rows per pass), C / 32 float4 per lane.
    {
        const int sub = tid & 7, nch = C >> 5;
        for (int r = tid >> 3; r < BM; r += 32) {
            float4 v[8];
#pragma unroll
            for (int c = 0; c < 8; ++c)
                v[c] = c < nch ? *reinterpret_cast<const float4 *>(tile + r * pitch + (c * 8 + sub) * 4)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
            quant_row_g8<CONV, 8, TWO>(v, nch, r, sub, codes, -KB, rl.sx[0], rl.zx[0],
                                       TWO ? codes + plane : nullptr, rl.sx[TWO ? 1 : 0],
                                       rl.zx[TWO ? 1 : 0], 0x80808080u);
        }
    }
    __syncthreads();

    const __amdgpu_buffer_rsrc_t wr = weight_rsrc(p);
    const int jstride = p.kb_count * 1024;
    const int wbase = nb0 * jstride;
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
    for (int kb = 0; kb < KB; ++kb) {
        v4i b[TJ], a[PL][TI];
#pragma unroll
        for (int j = 0; j < TJ; ++j) b[j] = load_frag(wr, lane * 16, wbase + j * jstride + kb * 1024);
#pragma unroll
        for (int pl = 0; pl < PL; ++pl)
#pragma unroll
            for (int i = 0; i < TI; ++i)
                a[pl][i] = *reinterpret_cast<const v4i *>(codes + pl * plane + ((i * KB + kb) * 64 + lane) * 16);
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[0][i], b[j], acc[i][j], 0, 0, 0);
                if (TWO)
                    acc2[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[PL - 1][i], b[j], acc2[i][j], 0, 0, 0);
            }
    }
    epilogue<CONV, EPI_LINEAR, TWO, TI, TJ, BM>(p, acc, acc2, cp, rl, nullptr, m0, nb0, lane);
}

}  // namespace

int launch_conv1x1_snake(IroHipContext *ctx, const IroHipWeight *w, const float *hidden, int T,
                         const float *snake_bias, const float *snake_alpha, bool two,
                         const float *bias, const float *skip, float *output) {
    const int C = w->K;
    const int tj = w->Np / 128;
    if (C % 32 || C < 64 || C > 256 || w->layout != 0 || (tj != 1 && tj != 2) || (two && tj != 1) ||
        (((uintptr_t)hidden) & 15) || !snake_bias || !snake_alpha)
        return 1;
    // 32-row blocks: four waves per SIMD (128 registers) and four blocks
    // per CU in LDS (stage-3 two-plane 1x1 268 -> 252 us against 64-row
    // blocks, whose two-plane epilogue needs 166 registers).
    const int bm = 32;
    const size_t lds = sizeof(float) * ((size_t)3 * C + (size_t)bm * C) +
                       (size_t)bm * C * (two ? 2 : 1);
    if (lds > 65536) return 1;
    GemmArgs a;
    a.M = T;
    a.K = C;
    a.bias = bias;
    a.y = output;
    a.yin = skip;
    a.ldy = w->N;
    a.accumulate = 1;
    KParams kp;
    if (fill_kparams(ctx, w, a, kp)) return -1;
    kp.tiles_n = 1;
    kp.tiles_m = (T + bm - 1) / bm;
    kp.tiles_per_xcd = (kp.tiles_m + 7) / 8;
    kp.row_major = 1;
    const dim3 grid((unsigned)(8 * kp.tiles_per_xcd)), block(256);
    // floor(f / (C/4)) == umulhi(2 f, ceil(2^31 / (C/4))) for the chunk
    // indices f < 4096 used: the rounding adds less than 2^13 / 2^32 < 4 / C.
    const unsigned k4 = (unsigned)C / 4, magic = (unsigned)((0x80000000ull + k4 - 1) / k4);
    prof_begin(ctx);
#define IRO_RS(CV, TW, TJ)                                                                      \
    hipLaunchKernelGGL((conv1x1_snake_kernel<CV, TW, TJ, 1>), grid, block, lds, ctx->stream, kp, \
                       hidden, snake_bias, snake_alpha, magic)
    if (ctx->convention == IRO_HIP_GCC_FASTMATH) {
        if (two) IRO_RS(1, true, 1);
        else if (tj == 2) IRO_RS(1, false, 2);
        else IRO_RS(1, false, 1);
    } else {
        if (two) IRO_RS(0, true, 1);
        else if (tj == 2) IRO_RS(0, false, 2);
        else IRO_RS(0, false, 1);
    }
#undef IRO_RS
    IRO_HIP_CHECK_LAUNCH(ctx);
    // Algorithmic work: 2 * C * N per row and plane; bytes: the rows, the
    // skip rows and the output once, the weight once.
    const double planes = two ? 2 : 1;
    prof_end(ctx, PK_CONV_GEMM, 2.0 * T * w->N * C * planes,
             4.0 * T * C + 8.0 * T * w->N + (double)w->N * C);
    return 0;
}

// Shapes the kernel takes: C a multiple of 32 from 64 to 1024, a window of
// at most 128 rows (stride 1, dilation <= 10).
bool conv7_gemm_ok(const IroHipWeight *w, const ConvRows &cr) {
    return cr.C % 32 == 0 && cr.C >= 64 && cr.C <= 1024 && (((uintptr_t)cr.x) & 15) == 0 &&
           63LL * cr.stride + 6LL * cr.dilation + 1 <= kCvWRows && w->Np % 128 == 0 &&
           w->K == 7 * cr.C && w->layout == 0;
}

// Where it beats the im2col path (which writes the codes and reads them
// back): up to 256 channels always (C = 96, two planes: 286 against 579 us
// at T = 480000; C = 192: 224 against 373 us at T = 240000), 384 channels
// from 16384 steps (T = 30000: 91 against 105 us), wider rows on long
// inputs only (C = 768, T = 60000: 473 against 542 us), where the im2col
// traffic outweighs the coding work each column tile repeats; on short ones
// it loses (C = 768, T = 3000: 62 against 54 us; C = 512, T = 24000: 100
// against 94 us; C = 1024, T = 6000: 77 against 51 us).
bool conv7_gemm_pays(const ConvRows &cr, int T_out) {
    return cr.C <= 256 || (cr.C <= 384 && T_out >= 16384) || T_out >= 65536;
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
    // 64 x 128 tiles up to 256 channels (four blocks per CU), 64 x 256 above
    // (each column tile repeats the coding); two planes always 64 x 128.
    int tj = !two && w->Np % 256 == 0 && cr.C > 256 ? 2 : 1;
    if (ctx->conv_cols == 128 || two) tj = 1;
    if (ctx->conv_cols == 256 && !two && w->Np % 256 == 0) tj = 2;
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
