// iro_gemm.hip -- int8 x int8 -> int32 GEMM on gfx950 MFMA with the
// reference's dequantization epilogue fused in.
//
// C[m,n] = sum_k A[m,k] * W[n,k], A = u8 activation codes (row-major),
// W = s8 weight codes pre-packed in 1 KiB MFMA fragments (IroHipWeight).
// gfx950 int8 MFMA is signed-only, so A is fed as (a ^ 0x80) = a - 128 and
// the raw u8 x s8 sum is recovered exactly in int32 as
// acc + 128 * rowsum[n], rowsum = sum over k of W[n,k]  (|acc| < 2^31 for
// K < 66k).
//
// Tile kernel: 256 threads = 4 wavefronts side by side along N.  Block tile
// BM x BN = 32*TI x 128*TJ, wave tile 32*TI x 32*TJ of
// v_mfma_i32_32x32x32_i8.  The activation tile is shared by the four waves
// and staged through double-buffered LDS in fragment order (lane L reads
// 16 bytes at L*16: conflict-free ds_read_b128).  Each weight fragment is
// used by exactly one wave, so waves read their fragments straight from the
// pre-packed buffer into registers (one contiguous 1 KiB per wave load),
// one k-step ahead; weights never touch LDS.  Per k-step (BK = 64) a wave
// issues 4*TI*TJ MFMAs against 2*TI LDS reads.
//
// Addresses never leave the operands: rows past M repeat row M-1 and k past
// the activation's extent repeats its last 16 bytes; the packed weight is
// zero for every k >= K, so those products vanish, and rows past M are
// never stored.  The main loop therefore has no branches around its loads.
//
// Skinny kernel (M <= 32, e.g. the modulation linear on the conditioning
// rows): one block per 64 weight rows, the four waves split K, their int32
// partial sums meet in LDS (integer addition: exact in any order) and wave 0
// runs the epilogue.  It is bound by the weight read.
//
// The two-term activation (ops.c:427-442 + dit.c:477-485) runs both planes
// against the same weight fragment: two accumulators, one pass over W.
//
// Epilogues (all per element, identical op order to the reference):
//   EPI_LINEAR  ops.c:468-490 four branches (+ optional raw int32 `work`)
//   EPI_QKVG    dit.c:786-792 four projections, split store
//   EPI_SWIGLU  dit.c:945-956 W1,W3 then silu(w1)*w3 (ops.c:781-784)
//   EPI_GATED   dit.c:1013-1020 / 1032-1039 x += gate[b] * y
#include "iro_gemm_core.h"

namespace iro {

namespace {

// Exhaustive self-check of the SiLU gate's pieces over the 2^28 float
// inputs with bit patterns base .. base + 2^28 - 1 (one per thread): the
// expf digest term (bits(x) * 0x9E3779B97F4A7C15) ^ (bits(e) *
// 0xC2B2AE3D27D4EB4F), NaN results as 0x7FC00000, summed into out[0]; and
// into out[1] the inputs a whose silu_div(a, 1 + expf(-a)) differs from the
// IEEE quotient (NaN == NaN), or, where silu_q_common takes a, whose
// silu_q_common differs from it.
__global__ __launch_bounds__(256) void silu_selfcheck_kernel(unsigned long long *out, unsigned base) {
    __shared__ uint64_t tab[32];
    __shared__ unsigned long long part[2][4];
    if (threadIdx.x < 32) tab[threadIdx.x] = kExp2Tab[threadIdx.x];
    __syncthreads();
    const unsigned u = base + blockIdx.x * 256u + threadIdx.x;
    const float x = __uint_as_float(u);
    const float e = expf_glibc(x, tab);
    const unsigned ue = e != e ? 0x7FC00000u : __float_as_uint(e);
    unsigned long long h = ((unsigned long long)u * 0x9E3779B97F4A7C15ull) ^
                           ((unsigned long long)ue * 0xC2B2AE3D27D4EB4Full);
    const float b = 1.0f + expf_glibc(-x, tab);
    const float q0 = x / b, q1 = silu_div(x, b);
    bool ok;
    const float q2 = silu_q_common(x, tab, ok);
    unsigned long long bad = (__float_as_uint(q0) != __float_as_uint(q1) && !(q0 != q0 && q1 != q1)) ||
                             (ok && __float_as_uint(q0) != __float_as_uint(q2));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        h += __shfl_xor(h, off, 64);
        bad += __shfl_xor(bad, off, 64);
    }
    if ((threadIdx.x & 63) == 0) {
        part[0][threadIdx.x >> 6] = h;
        part[1][threadIdx.x >> 6] = bad;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        atomicAdd(&out[0], part[0][0] + part[0][1] + part[0][2] + part[0][3]);
        atomicAdd(&out[1], part[1][0] + part[1][1] + part[1][2] + part[1][3]);
    }
}

// Main loop: the activation tile is staged through LDS in chunks of KC
// bytes of k (double-buffered: chunk c+1 is fetched into registers while
// chunk c is consumed, one barrier per chunk), and each wave streams its
// own weight fragments through a ring of R register slots, R k-blocks of
// 32 ahead of their use.
template <int CONV, int EPI, bool TWO, int TI, int TJ>
__device__ __forceinline__ void gemm_tile_body(const KParams &p) {
    constexpr int BM = 32 * TI;
    constexpr int PL = TWO ? 2 : 1;
    constexpr int CP = 8;                               // 16-byte pieces per thread per chunk
    constexpr int KC = CP * 256 * 16 / (BM * PL);       // chunk of k, bytes per row per plane
    constexpr int KBC = KC / 32;                        // k blocks per chunk
    constexpr int PLANE = BM * KC;                      // LDS bytes per plane per chunk
    constexpr int R = 8 / TJ <= KBC ? 8 / TJ : KBC;     // weight ring depth in k blocks
    static_assert(KC % 32 == 0 && KBC % R == 0 && R % 2 == 0 && KBC >= 2, "chunk must hold whole rings");
    // Two-plane 64 x 256 tiles run one block per CU (their accumulators take
    // 128 registers), so nothing hides the activation staging but the MFMAs
    // of the same wave: those stage two chunks ahead, one piece per k step.
    constexpr bool DEEP = TWO && TI == 2 && TJ == 2;
    __shared__ __attribute__((aligned(16))) uint8_t lds_a[2][PL * PLANE];
    __shared__ __attribute__((aligned(16))) RowLds<BM, TWO> rl;
    __shared__ uint64_t exptab[32];

    int bx, by;
    if (!tile_of(blockIdx.x, p.tiles_m, p.tiles_n, p.tiles_per_xcd, p.row_major, bx, by)) return;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int m0 = by * BM;
    const int nb0 = bx * 4 * TJ + wave * TJ;  // first packed 32-row weight block of this wave

    stage_rows<EPI, TWO, BM>(p, rl, m0, tid);
    if (EPI == EPI_SWIGLU && tid < 32) exptab[tid] = kExp2Tab[tid];
    const ColParams<TJ> cp = load_cols<EPI, TJ>(p, nb0, lane, m0, BM);

    // Activation pieces of this thread: piece q = tid + 256*i of a chunk is
    // plane q / (PLANE/16), then fragment f = (q % (PLANE/16)) / 64 =
    // [k block kbl][row block rb] and lane ln = q % 64 of that fragment.
    const uint8_t *pa[CP];
    int kof[CP];
#pragma unroll
    for (int i = 0; i < CP; ++i) {
        const int q = tid + 256 * i;
        const int pl = q / (PLANE / 16);
        const int qq = q % (PLANE / 16);
        const int f = qq >> 6, ln = qq & 63;
        const int kbl = f / TI, rb = f % TI;
        int gr = m0 + rb * 32 + (ln & 31);
        gr = gr < p.M ? gr : p.M - 1;
        kof[i] = kbl * 32 + (ln >> 5) * 16;
        pa[i] = (pl == 0 ? p.a1 : p.a2) + (size_t)gr * p.lda;
    }
    const __amdgpu_buffer_rsrc_t wr = weight_rsrc(p);
    const int jstride = p.kb_count * 1024;     // bytes between 32-row weight blocks
    const int wbase = nb0 * jstride;           // this wave's first block
    const int nkb = (p.K + 31) / 32;  // k blocks holding activation data
    const int nc = (p.K + KC - 1) / KC;

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

    // Staging registers of the activation chunks: DEEP keeps two chunks in
    // flight (chunk c+2 is loaded while chunk c runs), one otherwise.
    constexpr int NRA = DEEP ? 2 : 1;
    v4i ra[NRA][CP];
    v4i rb[R][TJ];
    const v4i flip = {p.aflip, p.aflip, p.aflip, p.aflip};
    const v4i zero4 = {0, 0, 0, 0};

    // One piece of chunk c: its global load and its LDS store.
    auto load_piece = [&](v4i (&dst)[CP], int c, int i) {
        int k = c * KC + kof[i];
        k = k < p.K - 16 ? k : p.K - 16;  // past the extent: any in-bounds bytes
        dst[i] = *reinterpret_cast<const v4i *>(pa[i] + k);
    };
    auto store_piece = [&](const v4i (&src)[CP], int buf, int c, int i) {
        *reinterpret_cast<v4i *>(&lds_a[buf][(tid + 256 * i) * 16]) =
            c * KC + kof[i] < p.K ? (src[i] ^ flip) : zero4;
    };
    // Staging slot of chunk c is c % NRA; callers pass it as a constant
    // (the chunk loop is unrolled by two) so the registers stay registers.
    auto load_chunk = [&](v4i (&dst)[CP], int c) {
#pragma unroll
        for (int i = 0; i < CP; ++i) {
            int k = c * KC + kof[i];
            k = k < p.K - 16 ? k : p.K - 16;  // past the extent: any in-bounds bytes
            dst[i] = *reinterpret_cast<const v4i *>(pa[i] + k);
        }
    };
    // Codes enter LDS as a - 128; bytes at k >= K enter as 0, so every MFMA
    // of a chunk can run unconditionally (zero times any weight is zero).
    auto store_chunk = [&](const v4i (&src)[CP], int buf, int c) {
#pragma unroll
        for (int i = 0; i < CP; ++i)
            *reinterpret_cast<v4i *>(&lds_a[buf][(tid + 256 * i) * 16]) =
                c * KC + kof[i] < p.K ? (src[i] ^ flip) : zero4;
    };
    auto load_b = [&](int slot_unused, v4i (&dst)[TJ], int kb) {
        (void)slot_unused;
        kb = kb < nkb ? kb : nkb - 1;  // past the end: a repeat, multiplied by zero codes
#pragma unroll
        for (int j = 0; j < TJ; ++j) dst[j] = load_frag(wr, lane * 16, wbase + j * jstride + kb * 1024);
    };
    auto read_a = [&](v4i (&a)[PL][TI], const uint8_t *abuf, int kbl) {
#pragma unroll
        for (int pl = 0; pl < PL; ++pl)
#pragma unroll
            for (int i = 0; i < TI; ++i)
                a[pl][i] = *reinterpret_cast<const v4i *>(
                    abuf + pl * PLANE + ((kbl * TI + i) * 64 + lane) * 16);
    };
    auto mma = [&](const v4i (&a)[PL][TI], const v4i (&b)[TJ]) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[0][i], b[j], acc[i][j], 0, 0, 0);
                if (TWO)
                    acc2[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[PL - 1][i], b[j],
                                                                       acc2[i][j], 0, 0, 0);
            }
    };

    // Prologue: chunk 0 (and with DEEP chunk 1) and the first R weight k
    // blocks in flight together.
    load_chunk(ra[0], 0);
#pragma unroll
    for (int u = 0; u < R; ++u) load_b(u, rb[u], u);
    if (DEEP) load_chunk(ra[NRA - 1], 1 < nc ? 1 : 0);
    store_chunk(ra[0], 0, 0);
    __syncthreads();
    // Each chunk is one straight run of KBC k steps (fully unrolled, no
    // branches): step u reads the activation fragments of step u+1 from
    // LDS, issues its MFMAs on slot u % R, and refills that slot with the
    // weights of step u + R.  The next chunk's activation loads go out after
    // the first ring turn: loads complete in issue order, so weight
    // fragments issued after them are consumed a full turn later.  In the
    // last chunk they reload in-bounds bytes into the idle buffer.
    // DEEP: chunk c+1 (in registers since chunk c-1) goes to LDS and chunk
    // c+2 is loaded piece by piece, one piece per k step of chunk c, so the
    // staging issues among the MFMAs; the chunk ends with the barrier alone.
    // The buffer chunk c+1 is written to was last read in chunk c-1, before
    // the barrier that ended it.
    static_assert(!DEEP || CP == KBC, "one staged piece per k step");
    auto run_chunk_deep = [&](int c, auto par) {
        constexpr int PAR = decltype(par)::value;  // c % 2
        const uint8_t *abuf = lds_a[PAR];
        const int g0 = c * KBC;
        const int cn = c + 2 < nc ? c + 2 : c;  // past the end: an in-bounds reload
        v4i a0[PL][TI], a1[PL][TI];
        read_a(a0, abuf, 0);
#pragma unroll
        for (int u = 0; u < KBC; u += 2) {
            read_a(a1, abuf, u + 1);
            fence_sched();
            mma(a0, rb[u % R]);
            load_b(u % R, rb[u % R], g0 + u + R);
            store_piece(ra[1 - PAR], 1 - PAR, c + 1, u);
            load_piece(ra[PAR], cn, u);
            fence_sched();
            if (u + 2 < KBC) read_a(a0, abuf, u + 2);
            fence_sched();
            mma(a1, rb[(u + 1) % R]);
            load_b((u + 1) % R, rb[(u + 1) % R], g0 + u + 1 + R);
            store_piece(ra[1 - PAR], 1 - PAR, c + 1, u + 1);
            load_piece(ra[PAR], cn, u + 1);
            fence_sched();
        }
        __syncthreads();
    };
    auto run_chunk = [&](int c, auto par) {
        if constexpr (DEEP) {
            run_chunk_deep(c, par);
            return;
        }
        constexpr int PAR = decltype(par)::value;  // c % 2
        const uint8_t *abuf = lds_a[PAR];
        const int g0 = c * KBC;
        v4i a0[PL][TI], a1[PL][TI];
        read_a(a0, abuf, 0);
#pragma unroll
        for (int u = 0; u < KBC; u += 2) {
            read_a(a1, abuf, u + 1);
            fence_sched();
            mma(a0, rb[u % R]);
            load_b(u % R, rb[u % R], g0 + u + R);
            fence_sched();
            if (u + 2 < KBC) read_a(a0, abuf, u + 2);
            fence_sched();
            mma(a1, rb[(u + 1) % R]);
            load_b((u + 1) % R, rb[(u + 1) % R], g0 + u + 1 + R);
            if (u + 2 == R) {
                // DEEP: chunk c+2 into the registers chunk c left (stored
                // before this chunk began); past the end a reload of an
                // in-bounds chunk into the same registers.
                const int cl = c + (DEEP ? 2 : 1);
                load_chunk(ra[DEEP ? PAR : 0], cl < nc ? cl : c);
            }
            fence_sched();
        }
        store_chunk(ra[DEEP ? 1 - PAR : 0], 1 - PAR, c + 1);
        __syncthreads();
    };
    for (int c = 0; c < nc; c += 2) {
        run_chunk(c, std::integral_constant<int, 0>{});
        if (c + 1 < nc) run_chunk(c + 1, std::integral_constant<int, 1>{});
    }

    epilogue<CONV, EPI, TWO, TI, TJ, BM>(p, acc, acc2, cp, rl, exptab, m0, nb0, lane);
}

template <int CONV, int EPI, bool TWO, int TI, int TJ>
__global__ __launch_bounds__(256) void gemm_tile_kernel(KParams p) {
    gemm_tile_body<CONV, EPI, TWO, TI, TJ>(p);
}

// The 32-row tile exists to put two blocks on every CU: hold its register
// budget to two waves per SIMD.
template <int CONV, int EPI, bool TWO, int TI, int TJ>
__global__ __launch_bounds__(256, 2) void gemm_tile_kernel_o2(KParams p) {
    gemm_tile_body<CONV, EPI, TWO, TI, TJ>(p);
}

// ---- SwiGLU hidden state quantized in the W1/W3 kernel ------------------
//
// Instead of storing the hidden state in fp32 for a row quantization
// launch (ops.c:321-348, two-term ops.c:427-442: the W2 input of
// dit.c:958-966), the W1/W3 kernel can quantize it itself.  A row's range
// needs all of its columns, and the columns of a 64-row band come from the
// band's groups_n blocks, so those blocks exchange per-row partial ranges
// through device memory: each block merges its partials with agent-scope
// atomic max on magnitudes (lo <= 0 <= hi, and non-negative floats order
// like their bit patterns), counts itself in and waits until the whole
// band has; min and max are exact in any order, so the merged range is the
// row's range and the codes are those of the row quantizer.  Agent-scope
// read-modify-writes are coherent across the XCDs' L2 caches, and every
// exchange goes through them.  The host launches this form only when the
// whole grid is resident at once, so every wait ends; a bounded spin still
// sets the device error word and gives up rather than hang.  The block
// that leaves its band last zeroes the band's state for the next launch.

// Wave-uniform min / max over each row of 16 lanes (DPP), in every lane.
__device__ __forceinline__ float row16_min(float v) {
    v = __builtin_fminf(v, dpp_mov<0xB1>(v));
    v = __builtin_fminf(v, dpp_mov<0x4E>(v));
    v = __builtin_fminf(v, dpp_mov<0x141>(v));
    return __builtin_fminf(v, dpp_mov<0x140>(v));
}
__device__ __forceinline__ float row16_max(float v) {
    v = __builtin_fmaxf(v, dpp_mov<0xB1>(v));
    v = __builtin_fmaxf(v, dpp_mov<0x4E>(v));
    v = __builtin_fmaxf(v, dpp_mov<0x141>(v));
    return __builtin_fmaxf(v, dpp_mov<0x140>(v));
}

// w holds the codes of rows e = 0..3 (byte e) of this lane's column;
// across each quad of lanes the 4 x 4 bytes are transposed, so lane
// 4q + k returns row k's codes of the quad's columns (byte c = column c of
// the quad).  Two butterfly stages: exchange with lane ^ 1, then lane ^ 2,
// v_perm_b32 picking the kept and received bytes.
__device__ __forceinline__ uint32_t quad_transpose(uint32_t w, int lane) {
    uint32_t p = (uint32_t)__builtin_amdgcn_mov_dpp((int)w, 0xB1, 0xF, 0xF, true);
    w = __builtin_amdgcn_perm(p, w, (lane & 1) ? 0x03070105u : 0x06020400u);
    p = (uint32_t)__builtin_amdgcn_mov_dpp((int)w, 0x4E, 0xF, 0xF, true);
    return __builtin_amdgcn_perm(p, w, (lane & 2) ? 0x03020706u : 0x05040100u);
}

// The SwiGLU epilogue's values (dit.c:945-956 as EPI_SWIGLU computes them
// from raw sums that already include 128 * rowsum) kept in registers: the
// wave's one W1/W3 column-block pair, h[i][r] at row
// m0 + 32 i + 8 (r / 4) + 4 (lane / 32) + r % 4.  Rows past M and columns
// past the hidden width hold 0, which lies inside every row range and
// leaves every range and code of the valid rows unchanged.
template <int CONV, int TI, int BM>
__device__ __forceinline__ void swiglu_hold(const KParams &p, const v16i (&acc)[TI][2],
                                            const ColParams<2> &cp, const RowLds<BM, false> &rl,
                                            const uint64_t *exptab, int m0, int nb0, int lane,
                                            float (&h)[TI][16]) {
    const int half = lane >> 5;
    const bool hok = (nb0 >> 1) * 32 + (lane & 31) < p.hidden_n;
#pragma unroll
    for (int i = 0; i < TI; ++i) {
        float sx[16];
        int zx[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int rb = i * 32 + g * 8 + half * 4;
            const float4 s4 = *reinterpret_cast<const float4 *>(&rl.sx[0][rb]);
            const int4 z4 = *reinterpret_cast<const int4 *>(&rl.zx[0][rb]);
            sx[g * 4 + 0] = s4.x; sx[g * 4 + 1] = s4.y; sx[g * 4 + 2] = s4.z; sx[g * 4 + 3] = s4.w;
            zx[g * 4 + 0] = z4.x; zx[g * 4 + 1] = z4.y; zx[g * 4 + 2] = z4.z; zx[g * 4 + 3] = z4.w;
        }
        float y[2][16];
#pragma unroll
        for (int r = 0; r < 16; ++r)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float t = (float)(acc[i][j][r] - __mul24(zx[r], cp.cs[j]));
                y[j][r] = t * (sx[r] * cp.sw[j]);
            }
        float v[16];
        silu_mul16(y[0], y[1], exptab, v);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const bool ok = hok && m0 + i * 32 + (r >> 2) * 8 + (r & 3) + half * 4 < p.M;
            h[i][r] = ok ? v[r] : 0.0f;
        }
    }
}

// This block's partial ranges of every row of the band (both held slabs),
// merged over the wave's 32 columns per row with DPP and over the waves
// with LDS atomics into s_lo / s_hi (magnitude bits).
template <int TI>
__device__ __forceinline__ void band_partials(const float (&h)[2][TI][16], unsigned *s_lo,
                                              unsigned *s_hi, int lane) {
    const int half = lane >> 5;
    const bool lead = (lane & 15) == 0;
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float lo =
                row16_min(__builtin_fminf(__builtin_fminf(h[0][i][r], h[1][i][r]), 0.0f));
            const float hi =
                row16_max(__builtin_fmaxf(__builtin_fmaxf(h[0][i][r], h[1][i][r]), 0.0f));
            if (lead) {
                const int row = i * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
                atomicMax(&s_lo[row], __float_as_uint(lo) & 0x7fffffffu);
                atomicMax(&s_hi[row], __float_as_uint(hi) & 0x7fffffffu);
            }
        }
}

// Thread 0: count this block into the band and wait for the rest (bounded;
// error bit 8 past the limit, and no further waiting once it is set).
__device__ __forceinline__ void band_arrive_wait(unsigned *ctr, unsigned nblk, int *err,
                                                 int spin_limit) {
    unsigned seen = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
    for (int n = 0; seen < nblk; ++n) {
        if (n >= spin_limit) {
            __hip_atomic_fetch_or(err, 8, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        if ((n & 63) == 63 &&
            (__hip_atomic_fetch_or(err, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 8))
            break;
        __builtin_amdgcn_s_sleep(1);
        seen = __hip_atomic_fetch_or(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// One range phase of the band: publish this block's partials, wait for the
// band, and leave the rows' parameters in s_rq (and, from the band's first
// block, in s / z).  All threads of the block take part.
template <int CONV, int BM>
__device__ __forceinline__ void band_phase(const KParams &p, unsigned *cnt, unsigned *rng,
                                           const unsigned (&s_lo)[BM], const unsigned (&s_hi)[BM],
                                           float4 (&s_rq)[BM], float *s, int32_t *z, int m0,
                                           bool first, int tid) {
    __syncthreads();
    if (tid < 2 * BM) {
        const int row = tid % BM, which = tid / BM;
        const unsigned v = which ? s_hi[row] : s_lo[row];
        if (v && m0 + row < p.M)
            (void)__hip_atomic_fetch_max(&rng[4 * row + which], v, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    }
    // every merge of this block has been performed before it counts itself
    __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (15 << 8));
    __syncthreads();
    if (tid == 0) band_arrive_wait(cnt, (unsigned)p.groups_n, p.err, p.spin_limit);
    __syncthreads();
    if (tid < BM) {
        const unsigned ulo = __hip_atomic_fetch_or(&rng[4 * tid], 0u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
        const unsigned uhi = __hip_atomic_fetch_or(&rng[4 * tid + 1], 0u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
        const RowQ r = row_params<CONV>(-__uint_as_float(ulo), __uint_as_float(uhi));
        s_rq[tid] = make_float4(r.s, r.inv, r.zpf, __int_as_float(r.zp));
        if (first && m0 + tid < p.M) {
            s[m0 + tid] = r.s;
            z[m0 + tid] = r.zp;
        }
    }
    __syncthreads();
}

// Codes of the held values with the rows' parameters in s_rq, stored as
// signed codes at (row, column) of q; with RES the values become the
// remainders x - s (q - zp) (ops.c:437-439) for the second plane.
template <int CONV, int TI, int BM, bool RES>
__device__ __forceinline__ void band_codes(const KParams &p, float (&h)[2][TI][16],
                                           const float4 (&s_rq)[BM], uint8_t *q, int m0,
                                           const int (&hcol)[2], const bool (&colok)[2],
                                           int lane) {
    const int half = lane >> 5, k = lane & 3;
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            RowQ rq[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float4 f = s_rq[i * 32 + g * 8 + half * 4 + e];
                rq[e].s = f.x;
                rq[e].inv = f.y;
                rq[e].zpf = f.z;
                rq[e].zp = __float_as_int(f.w);
            }
            const int row = m0 + i * 32 + g * 8 + half * 4 + k;
#pragma unroll
            for (int sl = 0; sl < 2; ++sl) {
                float *v = &h[sl][i][g * 4];
                const uint32_t w = pack_codes4(quant_pre<CONV>(v[0], rq[0]),
                                               quant_pre<CONV>(v[1], rq[1]),
                                               quant_pre<CONV>(v[2], rq[2]),
                                               quant_pre<CONV>(v[3], rq[3]));
                if (RES) {
                    const float4 c = unpack_codes4(w);
                    v[0] = residual_value<CONV>(v[0], c.x, rq[0]);
                    v[1] = residual_value<CONV>(v[1], c.y, rq[1]);
                    v[2] = residual_value<CONV>(v[2], c.z, rq[2]);
                    v[3] = residual_value<CONV>(v[3], c.w, rq[3]);
                }
                const uint32_t t = quad_transpose(w, lane) ^ 0x80808080u;
                if (colok[sl] && row < p.M)
                    *reinterpret_cast<uint32_t *>(q + (size_t)row * p.ldhq + hcol[sl] +
                                                  4 * ((lane & 31) >> 2)) = t;
            }
        }
}

// Whole-tile kernel (one activation plane, K <= 1024, codes stored signed):
// the block's entire 64-row activation tile, 64 x K bytes, is copied into
// LDS by direct global-to-LDS loads (global_load_lds_dwordx4: lane L of a
// wave writes 16 bytes at the wave's LDS base + 16 L, which is the fragment
// order), so it needs no staging registers.  The copy runs two ring turns
// ahead of the MFMAs of the first slab: the pieces of turn t+2 are issued at
// the end of turn t, and turn t waits only for its own pieces (loads
// complete in issue order, so "at most R*TJ + P loads outstanding" means
// this wave's pieces of turn t have landed) and one barrier.  The block
// then sweeps `spb` consecutive weight column slabs against the stationary
// tile, barrier-free: each wave streams its weight fragments through an
// R-deep register ring, and the stream runs on across slabs, so the next
// slab's first R k blocks are in flight while this slab's epilogue runs.
// k past K is copied from a zero page.  The accumulators start at
// 128 * rowsum[n] (the signed-operand correction), so they end as the
// reference's raw u8 x s8 sums.  BQ: the SwiGLU hidden state is held in
// registers over the block's (at most two) slabs and quantized by the
// band exchange above instead of stored.
template <int CONV, int EPI, int TJ, int R, int TI, bool BQ = false>
__global__ __launch_bounds__(256, (TI == 2 && (EPI == EPI_QKVG || EPI == EPI_SWIGLU)) ? 2 : 1) void gemm_wt_kernel(KParams p) {
    static_assert(TI == 2 || TI == 4, "64- or 128-row tiles");
    static_assert(!BQ || (EPI == EPI_SWIGLU && TI == 2 && TJ == 2), "band quantization: W1/W3, 64 x 256");
    constexpr int BM = 32 * TI, KMAX = 1024;
    constexpr int P = R * TI / 4;  // activation pieces per thread per ring turn
    // Sweeping several slabs pays for the projections with the largest N
    // (QKVG, W1/W3); the others run one slab per block, which keeps their
    // epilogues' registers out of a loop.
    constexpr bool MULTI = EPI == EPI_QKVG || EPI == EPI_SWIGLU;
    __shared__ __attribute__((aligned(16))) uint8_t lds_a[BM * KMAX];
    __shared__ __attribute__((aligned(16))) uint8_t lds_sink[1024];  // never read
    __shared__ __attribute__((aligned(16))) RowLds<BM, false> rl;
    __shared__ uint64_t exptab[32];
    __shared__ unsigned s_rng[BQ ? 4 : 1][BQ ? BM : 1];  // |lo|, hi of each range phase
    __shared__ float4 s_rq[BQ ? BM : 1];                  // s, inv, zp (float), zp (int bits)
    __shared__ int s_last;

    // Work item = (row tile, group of spb slabs), dealt to the XCDs in the
    // order that splits the larger operand (see tile_of).
    int gx, by;
    if (!tile_of(blockIdx.x, p.tiles_m, p.groups_n, p.tiles_per_xcd, p.row_major, gx, by)) return;
    const int bx0 = gx * p.spb;
    const int nslab = !MULTI ? 1 : (p.tiles_n - bx0 < p.spb ? p.tiles_n - bx0 : p.spb);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int m0 = by * BM;

    stage_rows<EPI, false, BM>(p, rl, m0, tid);
    if (EPI == EPI_SWIGLU && tid < 32) exptab[tid] = kExp2Tab[tid];
    if constexpr (BQ) s_rng[tid / BM][tid % BM] = 0;  // 4 * BM == 256 threads
    // BQ: hs[1] holds the current slab's values, hs[0] the previous slab's
    float hs[BQ ? 2 : 1][BQ ? TI : 1][16];
    if constexpr (BQ) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) hs[1][i][r] = 0.0f;
    }

    const int nkb = (p.K + 31) / 32;             // k blocks holding activation data
    const int nkr = (nkb + R - 1) / R * R;       // whole ring turns (<= KMAX / 32)
    const int nturn = nkr / R;
    // Piece q = tid + 256 i of the tile: fragment f = q / 64 = wave + 4 i =
    // (k block, row block) = (f / TI, f % TI), lane q % 64.  For this thread
    // the row block is wave % TI and k advances by 128 / TI per piece, so
    // pieces t*P .. t*P+P-1 hold ring turn t's k blocks.  Turns past the
    // last one load the zero page into a sink, which keeps the count of
    // loads behind every turn's pieces the same.
    int arow_i = m0 + (wave % TI) * 32 + (lane & 31);
    arow_i = arow_i < p.M ? arow_i : p.M - 1;
    const uint8_t *arow = p.a1 + (size_t)arow_i * p.lda;
    const int k0 = (wave / TI) * 32 + (lane >> 5) * 16;
    auto copy_turn = [&](int t) {
#pragma unroll
        for (int q = 0; q < P; ++q) {
            const int i = t * P + q;
            const int k = k0 + (128 / TI) * i;
            const bool real = t < nturn;
            const uint8_t *src = real && k < p.K ? arow + k : p.zero16;
            uint8_t *dst = real ? lds_a + (size_t)(tid - lane + 256 * i) * 16 : lds_sink;
            dma16(src, dst);
        }
    };
    const __amdgpu_buffer_rsrc_t wr = weight_rsrc(p);
    const int jstride = p.kb_count * 1024;      // bytes between 32-row weight blocks
    const int slab_stride = 4 * TJ * jstride;   // bytes between column slabs
    const int pb0 = (bx0 * 4 * TJ + wave * TJ) * jstride;  // this wave's blocks in slab 0

    v16i acc[TI][TJ], acc2[TI][TJ];
    v4i rb[R][TJ];
    // Weight stream: k block kk of the current slab, or, for kk >= nkr, k
    // block kk - nkr of the next slab (the last slab repeats itself); k
    // blocks are clamped to nkb - 1 (repeats meet zero codes or are never
    // consumed).
    auto load_b = [&](v4i (&dst)[TJ], int cur, int nxt, int kk) {
        const bool next = kk >= nkr;
        int kb = next ? kk - nkr : kk;
        kb = kb < nkb ? kb : nkb - 1;
        const int src = (next ? nxt : cur) + kb * 1024;
#pragma unroll
        for (int j = 0; j < TJ; ++j) dst[j] = load_frag(wr, lane * 16, src + j * jstride);
    };
    auto read_a = [&](v4i (&a)[TI], int kb) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
            a[i] = *reinterpret_cast<const v4i *>(lds_a + ((kb * TI + i) * 64 + lane) * 16);
    };
    auto mma = [&](const v4i (&a)[TI], const v4i (&b)[TJ]) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
    };

    // Issue order: pieces of turn 0, the first R weight k blocks, pieces of
    // turn 1; every later turn t issues R*TJ weight loads and then the
    // pieces of turn t+2.  Behind the pieces of any turn t there are thus at
    // least R*TJ + P loads when turn t begins.
    copy_turn(0);
#pragma unroll
    for (int u = 0; u < R; ++u) load_b(rb[u], pb0, pb0, u);
    copy_turn(1);
    constexpr int VM = R * TJ + P;
    static_assert(VM < 64, "vmcnt holds 6 bits");

    for (int sl = 0; sl < nslab; ++sl) {
        const int pcur = pb0 + sl * slab_stride;
        const int pnxt = sl + 1 < nslab ? pcur + slab_stride : pcur;
        const int nb0 = (bx0 + sl) * 4 * TJ + wave * TJ;
        const ColParams<TJ> cp = load_cols<EPI, TJ>(p, nb0, lane, m0, BM);
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    acc[i][j][r] = 128 * cp.rs[j];
                    acc2[i][j][r] = 0;
                }
        // In the first slab each turn waits for its own pieces, then a
        // barrier publishes the other waves' pieces (and, at turn 0, the row
        // parameters); later slabs find the whole tile in LDS.
        v4i a0[TI], a1[TI];
        for (int t = 0; t < nturn; ++t) {
            const int g = t * R;
            if (sl == 0) {
                __builtin_amdgcn_s_waitcnt((VM & 15) | (7 << 4) | (15 << 8) | ((VM >> 4) << 14));
                __syncthreads();
            }
            // After a barrier the turn's first fragments are read here;
            // otherwise the previous turn read them ahead.
            if (sl == 0 || t == 0) read_a(a0, g);
#pragma unroll
            for (int u = 0; u < R; u += 2) {
                read_a(a1, g + u + 1);
                fence_sched();
                mma(a0, rb[u]);
                load_b(rb[u], pcur, pnxt, g + u + R);
                fence_sched();
                if (u + 2 < R)
                    read_a(a0, g + u + 2);
                else if (sl > 0)
                    read_a(a0, g + R < nkr ? g + R : nkr - 1);
                fence_sched();
                mma(a1, rb[u + 1]);
                load_b(rb[u + 1], pcur, pnxt, g + u + 1 + R);
                fence_sched();
            }
            if (sl == 0) copy_turn(t + 2);
        }
        if constexpr (BQ) {
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) hs[0][i][r] = hs[1][i][r];
            swiglu_hold<CONV, TI, BM>(p, acc, cp, rl, exptab, m0, nb0, lane, hs[1]);
        } else {
            epilogue<CONV, EPI, false, TI, TJ, BM, true>(p, acc, acc2, cp, rl, exptab, m0, nb0,
                                                         lane);
        }
    }
    if constexpr (BQ) {
        // hs[1] is slab nslab - 1, hs[0] slab 0 when there were two (else
        // zeros); wave column block of slab s: (bx0 + s) * 4 + wave.
        const int hcol[2] = {(bx0 * 4 + wave) * 32, ((bx0 + nslab - 1) * 4 + wave) * 32};
        const bool colok[2] = {nslab == 2 && hcol[0] < p.hidden_n, hcol[1] < p.hidden_n};
        unsigned *cnt = p.band_cnt + 4 * by;
        unsigned *rng = p.band_rng + 4 * (size_t)m0;
        const bool first = gx == 0;
        band_partials<TI>(hs, s_rng[0], s_rng[1], lane);
        band_phase<CONV, BM>(p, cnt, rng, s_rng[0], s_rng[1], s_rq, p.hs1, p.hz1, m0, first, tid);
        if (p.hq2) {
            band_codes<CONV, TI, BM, true>(p, hs, s_rq, p.hq1, m0, hcol, colok, lane);
            band_partials<TI>(hs, s_rng[2], s_rng[3], lane);
            band_phase<CONV, BM>(p, cnt + 1, rng + 2, s_rng[2], s_rng[3], s_rq, p.hs2, p.hz2, m0,
                                 first, tid);
            band_codes<CONV, TI, BM, false>(p, hs, s_rq, p.hq2, m0, hcol, colok, lane);
        } else {
            band_codes<CONV, TI, BM, false>(p, hs, s_rq, p.hq1, m0, hcol, colok, lane);
        }
        // Every block of the band has read the merged ranges once it has
        // departed: the last one zeroes the band's state.
        if (tid == 0)
            s_last = __hip_atomic_fetch_add(cnt + 2, 1u, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT) + 1 == (unsigned)p.groups_n;
        __syncthreads();
        if (s_last) {
            (void)__hip_atomic_fetch_and(&rng[tid], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (tid < 3)
                (void)__hip_atomic_fetch_and(&cnt[tid], 0u, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // No copy into this block's LDS may still be in flight when it exits.
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
}

// M <= 32: block = 64 weight rows (two packed blocks), four waves split the
// k blocks, int32 partials summed in LDS, wave 0 runs the epilogue.  A wave
// loads U = 8 k blocks before its MFMAs, so at K = 1024 its whole share is
// one round trip (measured ~1 % faster over the DiT stack than U = 4, whose
// 1024 -> 73728 modulation GEMM streams 75 MB of weights).
template <int CONV, int EPI, bool TWO>
__global__ __launch_bounds__(256) void gemm_skinny_kernel(KParams p) {
    constexpr int TJ = 2, PL = TWO ? 2 : 1, U = 8;
    __shared__ int red[3][PL][TJ][16][64];
    __shared__ __attribute__((aligned(16))) RowLds<32, TWO> rl;
    __shared__ uint64_t exptab[32];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int nb0 = blockIdx.x * TJ;
    stage_rows<EPI, TWO, 32>(p, rl, 0, tid);
    if (EPI == EPI_SWIGLU && tid < 32) exptab[tid] = kExp2Tab[tid];

    const int kbn = (p.K + 31) / 32;           // k blocks holding activation data
    const int per = (kbn + 3) / 4;
    const int kb_lo = wave * per;
    const int kb_hi = kb_lo + per < kbn ? kb_lo + per : kbn;

    int row = lane & 31;
    row = row < p.M ? row : p.M - 1;
    const int kk = (lane >> 5) * 16;
    const uint8_t *pa1 = p.a1 + (size_t)row * p.lda + kk;
    const uint8_t *pa2 = TWO ? p.a2 + (size_t)row * p.lda + kk : nullptr;
    const int8_t *pbw = p.bp + (size_t)nb0 * p.kb_count * 1024 + lane * 16;
    const size_t jstride = (size_t)p.kb_count * 1024;
    const int lim = p.K - 16 - kk;
    const v4i flip = {p.aflip, p.aflip, p.aflip, p.aflip};

    v16i acc[1][TJ], acc2[1][TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            acc[0][j][r] = 0;
            acc2[0][j][r] = 0;
        }
    for (int kb = kb_lo; kb < kb_hi; kb += U) {
        v4i a[U], a2[U], b[U][TJ];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = kb + u < kb_hi ? kb + u : kb_lo;  // repeats stay in bounds
            int koff = k * 32;
            koff = koff < lim ? koff : lim;
            a[u] = *reinterpret_cast<const v4i *>(pa1 + koff);
            if (TWO) a2[u] = *reinterpret_cast<const v4i *>(pa2 + koff);
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                b[u][j] = *reinterpret_cast<const v4i *>(pbw + j * jstride + (size_t)k * 1024);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (kb + u >= kb_hi) break;
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                acc[0][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[u] ^ flip, b[u][j], acc[0][j],
                                                                  0, 0, 0);
                if (TWO)
                    acc2[0][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a2[u] ^ flip, b[u][j],
                                                                       acc2[0][j], 0, 0, 0);
            }
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                red[wave - 1][0][j][r][lane] = acc[0][j][r];
                if (TWO) red[wave - 1][PL - 1][j][r][lane] = acc2[0][j][r];
            }
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 0; w < 3; ++w)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                acc[0][j][r] += red[w][0][j][r][lane];
                if (TWO) acc2[0][j][r] += red[w][PL - 1][j][r][lane];
            }
    const ColParams<TJ> cp = load_cols<EPI, TJ>(p, nb0, lane, 0, 32);
    epilogue<CONV, EPI, TWO, 1, TJ, 32>(p, acc, acc2, cp, rl, exptab, 0, nb0, lane);
}

// ---- launch ------------------------------------------------------------------

struct TileCfg {
    int ti, tj;
};

template <int CONV, int EPI, bool TWO>
void launch_tile(const KParams &kp, TileCfg t, unsigned grid, hipStream_t st) {
#define IRO_TILE(TI_, TJ_)                                                                  \
    hipLaunchKernelGGL((gemm_tile_kernel<CONV, EPI, TWO, TI_, TJ_>), dim3(grid), dim3(256), 0, \
                       st, kp)
    // Two planes of a 128 x 256 tile would hold 256 accumulator registers
    // per lane and spill: that shape runs as 128 x 128.
    if (t.ti == 1)
        hipLaunchKernelGGL((gemm_tile_kernel_o2<CONV, EPI, TWO, 1, 2>), dim3(grid), dim3(256), 0,
                           st, kp);
    else if (t.ti == 2 && t.tj == 1) IRO_TILE(2, 1);
    else if (t.ti == 2 && t.tj == 2) IRO_TILE(2, 2);
    else if (t.ti == 4 && (t.tj == 1 || TWO)) IRO_TILE(4, 1);
    else IRO_TILE(4, (TWO ? 1 : 2));
#undef IRO_TILE
}

enum Mode { MODE_TILE = 0, MODE_SKINNY = 1, MODE_WHOLE = 2 };

template <int CONV, int EPI>
void launch_wt(const KParams &kp, int ti, int tj, int ring, unsigned grid, hipStream_t st) {
    if constexpr (EPI == EPI_SWIGLU) {
        if (kp.hq1) {  // the caller checked ti == 2, tj == 2, ring 4
            hipLaunchKernelGGL((gemm_wt_kernel<CONV, EPI, 2, 4, 2, true>), dim3(grid), dim3(256),
                               0, st, kp);
            return;
        }
    }
    if (ti == 4) {
        if (tj == 1)
            hipLaunchKernelGGL((gemm_wt_kernel<CONV, EPI, 1, 8, 4>), dim3(grid), dim3(256), 0, st,
                               kp);
        else
            hipLaunchKernelGGL((gemm_wt_kernel<CONV, EPI, 2, 4, 4>), dim3(grid), dim3(256), 0, st,
                               kp);
    } else if (tj == 1)
        hipLaunchKernelGGL((gemm_wt_kernel<CONV, EPI, 1, 8, 2>), dim3(grid), dim3(256), 0, st, kp);
    else if (ring == 8)
        hipLaunchKernelGGL((gemm_wt_kernel<CONV, EPI, 2, 8, 2>), dim3(grid), dim3(256), 0, st, kp);
    else
        hipLaunchKernelGGL((gemm_wt_kernel<CONV, EPI, 2, 4, 2>), dim3(grid), dim3(256), 0, st, kp);
}

template <int CONV, int EPI>
void launch_e(const KParams &kp, bool two, Mode mode, TileCfg t, int ring, unsigned grid,
              hipStream_t st) {
    if (mode == MODE_SKINNY) {
        if (two)
            hipLaunchKernelGGL((gemm_skinny_kernel<CONV, EPI, true>), dim3(grid), dim3(256), 0, st,
                               kp);
        else
            hipLaunchKernelGGL((gemm_skinny_kernel<CONV, EPI, false>), dim3(grid), dim3(256), 0,
                               st, kp);
    } else if (mode == MODE_WHOLE) {
        launch_wt<CONV, EPI>(kp, t.ti, t.tj, ring, grid, st);
    } else if (two) {
        launch_tile<CONV, EPI, true>(kp, t, grid, st);
    } else {
        launch_tile<CONV, EPI, false>(kp, t, grid, st);
    }
}

template <int CONV>
void launch_c(const KParams &kp, Epi epi, bool two, Mode mode, TileCfg t, int ring, unsigned grid,
              hipStream_t st) {
    switch (epi) {
        case EPI_LINEAR: launch_e<CONV, EPI_LINEAR>(kp, two, mode, t, ring, grid, st); break;
        case EPI_QKVG: launch_e<CONV, EPI_QKVG>(kp, two, mode, t, ring, grid, st); break;
        case EPI_SWIGLU: launch_e<CONV, EPI_SWIGLU>(kp, two, mode, t, ring, grid, st); break;
        case EPI_GATED: launch_e<CONV, EPI_GATED>(kp, two, mode, t, ring, grid, st); break;
    }
}

// Whether the band-quantizing W1/W3 kernel can take a launch of `grid`
// blocks whose shape fits it (`shape`): no concurrent chain of launches
// shares the GPU (a context workspace override marks one) and the GPU holds
// every block at once, so no block waits for one that cannot start.  Then
// the band state is sized (allocated zeroed, outside graph capture) and
// its pointers set: returns 0.  Returns 1 to decline, -1 on error.
int band_quant_setup(IroHipContext *ctx, KParams &kp, bool shape, unsigned grid) {
    if (!shape || !ctx->band_quant || ctx->ws_override) return 1;
    const int conv = ctx->convention == IRO_HIP_GCC_FASTMATH ? 1 : 0;
    if (!ctx->band_occ[conv]) {
        int n = 0;
        const hipError_t e =
            conv ? hipOccupancyMaxActiveBlocksPerMultiprocessor(
                       &n, reinterpret_cast<const void *>(
                               &gemm_wt_kernel<1, EPI_SWIGLU, 2, 4, 2, true>), 256, 0)
                 : hipOccupancyMaxActiveBlocksPerMultiprocessor(
                       &n, reinterpret_cast<const void *>(
                               &gemm_wt_kernel<0, EPI_SWIGLU, 2, 4, 2, true>), 256, 0);
        if (e != hipSuccess) return set_error(ctx, "gemm: occupancy query failed");
        ctx->band_occ[conv] = n > 0 ? n : -1;
    }
    const int cus = ctx->cus > 0 ? ctx->cus : 256;
    if (ctx->band_occ[conv] < 0 || (long long)grid > (long long)ctx->band_occ[conv] * cus)
        return 1;
    // [tiles_m][4] counters, then [64 tiles_m][4] row ranges
    const size_t need = sizeof(unsigned) * 4 * (size_t)kp.tiles_m * 65;
    if (need > ctx->band_state_bytes) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(ctx->stream, &cs) != hipSuccess ||
            cs != hipStreamCaptureStatusNone)
            return 1;  // never allocate under capture: the eager run sized it
        IRO_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        if (ctx->band_state) (void)hipFree(ctx->band_state);
        ctx->band_state = nullptr;
        ctx->band_state_bytes = 0;
        const size_t bytes = round_up(need, 4096);
        IRO_HIP_TRY(ctx, hipMalloc(&ctx->band_state, bytes));
        if (launch_fill(ctx, ctx->band_state, 0, bytes)) return -1;
        ctx->band_state_bytes = bytes;
    }
    kp.band_cnt = ctx->band_state;
    kp.band_rng = ctx->band_state + 4 * (size_t)kp.tiles_m;
    return 0;
}

// Tile choice (measured on MI355X at the DiT shapes): 64-row tiles keep
// two blocks resident per CU; 256 columns per block halve the activation
// re-reads of 128, so they win whenever they still give every CU a tile.
// Two planes of a 64 x 256 tile need 128 accumulator registers per lane
// (one block per CU); 32-row tiles (ti = 1) double the tile count at 64
// registers, measured no faster at the W2 shape.  The SwiGLU epilogue
// needs an even number of 32-column blocks per wave.
TileCfg choose_tile(int M, int N, int Np, int K, int cus, bool two, Epi epi, int forced) {
    if (forced) {
        TileCfg t{forced / 10, forced % 10};
        if (epi == EPI_SWIGLU && t.tj % 2) t.tj = 2;
        if (t.ti == 1) t.tj = 2;
        if (two && t.ti * t.tj > 4) t.tj = 1;
        if (epi == EPI_SWIGLU && two && t.ti * t.tj > 4) t.ti = 2;
        return t;
    }
    const long long tiles22 = (long long)((M + 63) / 64) * (Np / 256);
    if (epi == EPI_SWIGLU) return TileCfg{2, 2};
    // Few rows (a plain sampler step, M = 750): 64 x 256 tiles would leave
    // most CUs idle; 32-row tiles double the count (measured at M = 750:
    // W2 two-term 22.6 us against 32.1, Wo 12.4 against 13.8).
    if (tiles22 * 2 < cus) return TileCfg{1, 2};
    if (two) return TileCfg{2, 2};
    // Many short-k tiles (the decoder's upsample GEMMs: 240000 x 384 and
    // 30000 x 3072 with k = 192 and 384): a 64-row tile has too little MFMA
    // work for its copy and epilogue latency; 128 x 128 tiles of the chunked
    // kernel measured 0.08 ms faster per decode.
    if (K <= 512 && tiles22 >= 8LL * cus) return TileCfg{4, 1};
    // Short k on a weight with 128 or more rows of padding (the decoder's
    // stage-1 1x1: 30000 x 384 padded to 512, k = 384): 128 x 128 tiles of
    // the chunked kernel measured 46.7 us against 58.9 us for the 64 x 256
    // whole-tile kernel (quantization included).
    if (K <= 512 && Np - N >= 128 && (long long)((M + 127) / 128) * (Np / 128) >= 2LL * cus)
        return TileCfg{4, 1};
    return tiles22 >= cus ? TileCfg{2, 2} : TileCfg{2, 1};
}

}  // namespace

// Exhaustive digests of the device's sqrtf and 1 / x (the correctly
// rounded operations the adaLN apply relies on) over the 2^28 inputs from
// base: out[0] += (bits(x) * 0x9E3779B97F4A7C15) ^ (bits(sqrtf(x)) *
// 0xC2B2AE3D27D4EB4F), out[1] the same for 1 / x; NaN results as 0x7FC00000.
__global__ __launch_bounds__(256) void fp32_selfcheck_kernel(unsigned long long *out, unsigned base) {
    __shared__ unsigned long long part[2][4];
    const unsigned u = base + blockIdx.x * 256u + threadIdx.x;
    const float x = __uint_as_float(u);
    const float r = __builtin_sqrtf(x), q = 1.0f / x;
    const unsigned ur = r != r ? 0x7FC00000u : __float_as_uint(r);
    const unsigned uq = q != q ? 0x7FC00000u : __float_as_uint(q);
    unsigned long long hs = ((unsigned long long)u * 0x9E3779B97F4A7C15ull) ^
                            ((unsigned long long)ur * 0xC2B2AE3D27D4EB4Full);
    unsigned long long hq = ((unsigned long long)u * 0x9E3779B97F4A7C15ull) ^
                            ((unsigned long long)uq * 0xC2B2AE3D27D4EB4Full);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        hs += __shfl_xor(hs, off, 64);
        hq += __shfl_xor(hq, off, 64);
    }
    if ((threadIdx.x & 63) == 0) {
        part[0][threadIdx.x >> 6] = hs;
        part[1][threadIdx.x >> 6] = hq;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        atomicAdd(&out[0], part[0][0] + part[0][1] + part[0][2] + part[0][3]);
        atomicAdd(&out[1], part[1][0] + part[1][1] + part[1][2] + part[1][3]);
    }
}

int launch_fp32_selfcheck(IroHipContext *ctx, unsigned long long *out) {
    for (unsigned long long base = 0; base < (1ull << 32); base += (1ull << 28)) {
        hipLaunchKernelGGL(fp32_selfcheck_kernel, dim3(1u << 20), dim3(256), 0, ctx->stream, out,
                           (unsigned)base);
        IRO_HIP_CHECK_LAUNCH(ctx);
    }
    return 0;
}

// All 2^32 inputs in 16 launches of 2^20 blocks; out[2] must start zeroed.
int launch_silu_selfcheck(IroHipContext *ctx, unsigned long long *out) {
    for (unsigned long long base = 0; base < (1ull << 32); base += (1ull << 28)) {
        hipLaunchKernelGGL(silu_selfcheck_kernel, dim3(1u << 20), dim3(256), 0, ctx->stream, out,
                           (unsigned)base);
        IRO_HIP_CHECK_LAUNCH(ctx);
    }
    return 0;
}

void gemm_prof_end(IroHipContext *ctx, const GemmArgs &a, const IroHipWeight *w, Epi epi,
                   bool two);

int ctx_cus(const IroHipContext *ctx) { return ctx->cus > 0 ? ctx->cus : 256; }

int gemm_lds_cfg(const IroHipContext *ctx, Epi epi, bool two, int M, int K, int N) {
    if (M <= 32 || ctx->gemm_lds < 0 || K % 32) return 0;
    // Default: the QKVG projection (measured at 2250 x 1024 -> 4096: 23.2 us
    // against 25.8 us for the register-streamed whole-tile kernel; the
    // W1/W3, Wo and W2 shapes ran slower through it), and long, wide
    // one-plane linears such as the kernel-7 Conv1d's GEMM (24000 rows,
    // K = 3584, N = 512: 66.5 us against 71.3 us for the tile kernel; at
    // 6000 rows, K = 7168, N = 256 it was slower, 60 against 34 us).
    if (ctx->gemm_lds == 0 && epi != EPI_QKVG) {
        if (epi == EPI_LINEAR && !two && M >= 16384 && K >= 2048 && N >= 512 &&
            lds_cfg_ok(LDS_192x256_CFG, two, epi))
            return LDS_192x256_CFG;
        // Wide one-plane linears of a few thousand rows (the decoder's
        // stage-1 upsample: 3000 x 7680, K = 768): 77.8 us against 115 us
        // with the whole-tile kernel (its quantization and gather included).
        if (epi == EPI_LINEAR && !two && M <= 8192 && K >= 512 && K <= 1024 && N >= 6144 &&
            (long long)((M + 191) / 192) * (N / 256) >= ctx_cus(ctx) &&
            lds_cfg_ok(LDS_192x256_CFG, two, epi))
            return LDS_192x256_CFG;
        return 0;
    }
    int cfg = ctx->gemm_lds > 0 ? ctx->gemm_lds : LDS_192x256_CFG;
    // Few rows: 96 x 128 tiles keep every CU busy (measured at M = 750,
    // N = 4096: 15.4 us against 22.0 for 192 x 256).  Past K = 1024 the
    // tile kernel is faster there (M = 750, K = 1280, N = 5120: 17.4 us
    // against 27.3 for 96 x 128 and 21-24 for the larger shapes).
    if (ctx->gemm_lds == 0) {
        const int cus = ctx->cus > 0 ? ctx->cus : 256;
        // the QKVG output is 4K wide: K / 64 column tiles of 256
        if ((long long)((M + 191) / 192) * (K / 64) * 2 < cus) {
            if (K > 1024) return 0;
            cfg = LDS_96x128_CFG;
        }
    }
    return lds_cfg_ok(cfg, two, epi) ? cfg : 0;
}

// The launch parameters every GEMM kernel takes from a weight and its
// arguments (tiles and grid are the caller's).
int fill_kparams(IroHipContext *ctx, const IroHipWeight *w, const GemmArgs &a, KParams &kp) {
    kp.a1 = a.a1;
    kp.a2 = a.a2;
    kp.lda = a.lda;
    kp.bp = w->packed;
    kp.kb_count = w->Kp / 32;
    kp.M = a.M;
    kp.N = w->N;
    kp.K = a.K;
    kp.sx1 = a.sx1;
    kp.sx2 = a.sx2;
    kp.zx1 = a.zx1;
    kp.zx2 = a.zx2;
    kp.sw = w->scale;
    kp.colsum = w->colsum;
    kp.rowsum = w->rowsum;
    kp.bias = a.bias;
    kp.y = a.y;
    kp.yin = a.yin;
    kp.ldy = a.ldy;
    kp.work = a.work;
    kp.ldw = a.ldw;
    kp.accumulate = a.accumulate;
    kp.seg0 = a.seg[0];
    kp.seg1 = a.seg[1];
    kp.seg2 = a.seg[2];
    kp.seg3 = a.seg[3];
    kp.seg_n = a.seg_n;
    kp.hidden = a.hidden;
    kp.ldh = a.ldh;
    kp.hidden_n = w->layout == 1 ? w->part_N[0] : 0;
    kp.xres = a.xres;
    kp.gate = a.gate;
    kp.ldg = a.ldg > 0 ? a.ldg : a.ldx;
    kp.ldx = a.ldx;
    kp.rows_per_branch = a.rows_per_branch > 0 ? a.rows_per_branch : 1;
    kp.aflip = a.a_signed ? 0 : (int)0x80808080;
    kp.zero16 = static_cast<const uint8_t *>(ctx->zero16);
    if ((long long)w->Np * w->Kp >= (1LL << 31))
        return set_error(ctx, "gemm: packed weight of %d x %d bytes exceeds 2 GiB", w->Np, w->Kp);
    kp.wbytes = w->Np * w->Kp;
    kp.hq1 = a.hq1;
    kp.hq2 = a.hq2;
    kp.ldhq = a.ldhq;
    kp.hs1 = a.hs1;
    kp.hs2 = a.hs2;
    kp.hz1 = a.hz1;
    kp.hz2 = a.hz2;
    kp.band_cnt = kp.band_rng = nullptr;
    kp.err = ctx->dev_err;
    kp.spin_limit = 1 << 20;
    return 0;
}

int launch_gemm(IroHipContext *ctx, const IroHipWeight *w, const GemmArgs &a, Epi epi) {
    if (a.M <= 0) return 0;
    if (a.K <= 0 || a.K % 16 || a.K > w->Kp || a.K < w->K || a.K > 65536 || a.lda < a.K ||
        a.lda % 16 ||
        (((uintptr_t)a.a1) & 15) || (a.a2 && (((uintptr_t)a.a2) & 15)) || w->Np % 128 ||
        (w->Np % 256 && (epi == EPI_SWIGLU || epi == EPI_QKVG)))
        return set_error(ctx, "gemm: unsupported operand shape (K=%d lda=%d Kp=%d Np=%d)", a.K,
                         a.lda, w->Kp, w->Np);
    if (epi == EPI_SWIGLU && (w->layout != 1 || w->part_N[0] % 32))
        return set_error(ctx, "gemm: SwiGLU epilogue needs an interleaved W1/W3 weight");
    if (epi != EPI_SWIGLU && w->layout != 0)
        return set_error(ctx, "gemm: an interleaved weight needs the SwiGLU epilogue");
    if (epi == EPI_QKVG && (a.seg_n <= 0 || w->N > 4 * a.seg_n))
        return set_error(ctx, "gemm: QKVG epilogue needs N <= 4 * segment width");
    KParams kp;
    if (fill_kparams(ctx, w, a, kp)) return -1;
    const bool two = a.a2 != nullptr;
    const bool skinny = a.M <= 32;
    const bool bq = a.hq1 != nullptr;
    if (bq && (epi != EPI_SWIGLU || !a.hs1 || !a.hz1 || (a.hq2 && (!a.hs2 || !a.hz2)) ||
               a.ldhq < w->part_N[0] || a.ldhq % 4 || (((uintptr_t)a.hq1) & 3) ||
               (((uintptr_t)a.hq2) & 3)))
        return set_error(ctx, "gemm: invalid hidden-state code buffers");
    // Signed codes with whole k blocks take the LDS-pipelined kernel.
    int lcfg = a.a_signed ? gemm_lds_cfg(ctx, epi, two, a.M, a.K, w->N) : 0;
    if (lcfg) {
        int bm = 0, bn = 0;
        lds_tile_shape(lcfg, &bm, &bn);
        if (w->Np % bn) lcfg = 0;  // a narrow weight: the 128-column tiles below
    }
    kp.akbp = a.a_kbp;
    if (a.a_kbp > 0 && (!lcfg || a.a_kbp * 32 != a.K))
        return set_error(ctx, "gemm: fragment-layout codes need the LDS-pipelined kernel");
    if (lcfg && bq) return 1;
    if (lcfg) {
        int bm = 0, bn = 0;
        lds_tile_shape(lcfg, &bm, &bn);
        kp.tiles_n = w->Np / bn;
        kp.tiles_m = (a.M + bm - 1) / bm;
        const int tiles = kp.tiles_n * kp.tiles_m;
        kp.tiles_per_xcd = (tiles + 7) / 8;
        const double abytes = (double)a.M * a.K * (two ? 2 : 1), wbytes = (double)w->Np * a.K;
        kp.row_major = ctx->tile_order >= 0 ? ctx->tile_order : (abytes > wbytes ? 1 : 0);
        prof_begin(ctx);
        launch_lds(kp, ctx->convention, epi, two, lcfg, (unsigned)(8 * kp.tiles_per_xcd),
                   ctx->stream);
        IRO_HIP_CHECK_LAUNCH(ctx);
        gemm_prof_end(ctx, a, w, epi, two);
        return 0;
    }
    TileCfg t{0, 0};
    Mode mode = MODE_TILE;
    int ring = ctx->gemm_ring ? ctx->gemm_ring : 4;
    unsigned grid;
    if (skinny) {
        mode = MODE_SKINNY;
        grid = (unsigned)(w->Np / 64);
        kp.tiles_n = grid;
        kp.tiles_m = 1;
        kp.tiles_per_xcd = 0;
        kp.row_major = 0;
    } else {
        t = choose_tile(a.M, w->N, w->Np, a.K, ctx->cus > 0 ? ctx->cus : 256, two, epi, ctx->gemm_tile);
        if (two && t.ti * t.tj > 4) t.tj = 1;  // as launch_tile runs it
        if (w->Np % 256) {  // a narrow weight (128 padded rows): 128-column tiles
            t.tj = 1;
            if (t.ti == 1) t.ti = 2;
        }
        // Signed single-plane codes with K <= 1024 fit a whole 64-row tile
        // in LDS: the barrier-free whole-tile kernel.
        if (a.a_signed && !two && a.K <= 1024 && t.ti == 2) {
            mode = MODE_WHOLE;
            // 128-row tiles (one block per CU, the tile in 128 KiB of LDS)
            // halve the weight stream per output against 64-row ones.
            if (ctx->gemm_wt_rows == 128) t.ti = 4;
        }
        kp.tiles_n = w->Np / (128 * t.tj);
        kp.tiles_m = (a.M + 32 * t.ti - 1) / (32 * t.ti);
        const int tiles = kp.tiles_n * kp.tiles_m;
        kp.tiles_per_xcd = (tiles + 7) / 8;
        // Each XCD reads its share of one operand once and all of the other:
        // keep the larger operand split.
        const double abytes = (double)a.M * a.K * (two ? 2 : 1), wbytes = (double)w->Np * a.K;
        kp.row_major = ctx->tile_order >= 0 ? ctx->tile_order : (abytes > wbytes ? 1 : 0);
        grid = (unsigned)(8 * kp.tiles_per_xcd);
        if (mode == MODE_WHOLE) {
            // Slabs per block: W1/W3 takes the fewest that still leave
            // about one block per CU per resident slot pair, so the
            // stationary tile serves as many slabs as the grid allows (its
            // SiLU epilogue then overlaps the weight stream of the next
            // slab).  QKVG runs one slab per block: its store-bound epilogue
            // gains more from the extra blocks (measured 26.9 us against
            // 29.5 us with two slabs at M = 2250, N = 4096, K = 1024).
            int spb = (epi == EPI_QKVG || epi == EPI_SWIGLU) ? ctx->gemm_spb : 1;
            if (spb <= 0 && epi == EPI_QKVG) spb = 1;
            if (spb <= 0 && t.ti == 4) {
                // one resident block per CU: the fewest slabs per block
                // that give every item a CU
                const int cus = ctx->cus > 0 ? ctx->cus : 256;
                spb = (int)(((long long)kp.tiles_m * kp.tiles_n + cus - 1) / cus);
            }
            if (spb <= 0) {
                const int cus = ctx->cus > 0 ? ctx->cus : 256;
                spb = 1;
                while (spb < kp.tiles_n && (long long)kp.tiles_m * ((kp.tiles_n + 2 * spb - 1) / (2 * spb)) >= cus)
                    spb *= 2;
            }
            kp.spb = spb;
            kp.groups_n = (kp.tiles_n + spb - 1) / spb;
            // Row bands per XCD: the blocks of an XCD then share their
            // stationary activation tiles in its L2, which shortens the
            // latency-bound tile copy; the weight stream hides its latency
            // in the ring (measured faster than slab order at the DiT
            // shapes although it moves more bytes).
            // At few rows (a plain step, M = 750) the weight is the larger
            // operand by far: column slabs per XCD keep each XCD's share of
            // it in its L2 (measured 0.96 against 1.01 ms per 12-block step).
            kp.row_major = ctx->tile_order >= 0 ? ctx->tile_order : (a.M <= 1024 ? 0 : 1);
            const int items = kp.groups_n * kp.tiles_m;
            kp.tiles_per_xcd = (items + 7) / 8;
            grid = (unsigned)(8 * kp.tiles_per_xcd);
        }
    }
    if (bq) {
        const int rc = band_quant_setup(ctx, kp, mode == MODE_WHOLE && t.ti == 2 && t.tj == 2 &&
                                                     ring == 4 && kp.spb <= 2, grid);
        if (rc) return rc;
    }
    prof_begin(ctx);
    if (ctx->convention == IRO_HIP_GCC_FASTMATH)
        launch_c<1>(kp, epi, two, mode, t, ring, grid, ctx->stream);
    else
        launch_c<0>(kp, epi, two, mode, t, ring, grid, ctx->stream);
    IRO_HIP_CHECK_LAUNCH(ctx);
    gemm_prof_end(ctx, a, w, epi, two);
    return 0;
}

// Algorithmic work of one GEMM launch for the profiler: 2*M*N*K per plane;
// bytes = codes + weights + outputs.
void gemm_prof_end(IroHipContext *ctx, const GemmArgs &a, const IroHipWeight *w, Epi epi,
                   bool two) {
    const double M = a.M, N = w->N, K = w->K, planes = two ? 2 : 1;
    double out_bytes = 4 * M * N;
    ProfKind kind = two ? PK_GEMM_LINEAR_2T : PK_GEMM_LINEAR;
    if (epi == EPI_LINEAR) {
        out_bytes *= 1 + (a.accumulate ? 1 : 0) + (a.work ? 1 : 0);
    } else if (epi == EPI_QKVG) {
        kind = two ? PK_GEMM_QKVG_2T : PK_GEMM_QKVG;
    } else if (epi == EPI_SWIGLU && a.hq1) {
        // W1/W3 quantizing its hidden state: codes of each plane, row
        // parameters
        kind = PK_GEMM_SWIGLU_Q;
        out_bytes = (M * N / 2 + 8 * M) * (a.hq2 ? 2 : 1);
    } else if (epi == EPI_SWIGLU) {
        kind = two ? PK_GEMM_SWIGLU_2T : PK_GEMM_SWIGLU;
        out_bytes /= 2;
    } else {
        kind = two ? PK_GEMM_GATED_2T : PK_GEMM_GATED;
        out_bytes *= 2;
    }
    prof_end(ctx, kind, 2 * M * N * K * planes, M * K * planes + N * K + out_bytes);
}

}  // namespace iro
