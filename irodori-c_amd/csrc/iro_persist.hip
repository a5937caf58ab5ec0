// iro_persist.hip -- the int8 linear stack of one Euler step (the dit_block
// sequence of dit.c:983-1040 over every block, its int8 parts) as one
// persistent kernel, after the modulation GEMM.
//
// Why one kernel.  Every kernel of the stack is short (a few to 30 us) and
// its tile prologue (activation copy), epilogue (dequantization, fp32
// stores) and ramp run in lockstep across the grid; the quantizations are
// separate launches bound by their fixed cost.  Here workgroups take work
// items from a queue, so one workgroup's copies and stores overlap another's
// MFMAs, quantizations run as items between the GEMMs that produce and
// consume them, and the step pays one launch.
//
// XCD-local rows.  The stack is row-wise: a row's QKVG, Wo, W1/W3 and W2 in
// every block depend only on that row.  The rows are cut into bands of 96
// (three 32-row MFMA blocks) and each of the eight XCDs owns a contiguous
// run of bands; a workgroup reads its XCD from the hardware (XCC_ID) and
// only takes items of its XCD's rows.  Every hand-off between items -- fp32
// rows to a quantization item, codes to a GEMM item, x between the gated
// residuals -- therefore stays inside one XCD, whose L2 is the point of
// coherence for all of its CUs: a producer waits for its stores to reach L2
// (s_waitcnt vmcnt(0)) and then counts the item done with an atomic; a
// consumer polls that count with an atomic, then invalidates its CU's L1
// (buffer_inv sc1) before reading.  Nothing crosses the XCDs' L2 caches,
// which are not coherent with one another.
//
// Measured at the model's shape (12 blocks, 3 x 750 rows): 2.76 ms per step
// against 1.48 ms for one kernel per GEMM, so it is off by default.  Each
// band's chain of 8 stages x 12 blocks is serial, and the items on it are
// bound by memory latency (a timing copy without any MFMA runs as long), so
// the chain, not the arithmetic, sets the step time.
//
// Items of one block, per band: QX (quantize x, 6 items of 16 rows) ->
// QKVG (16 column slabs of 256) -> QV (quantize V) -> Wo (4 slabs, x +=
// gate_a * y) -> QX2 -> W1/W3 + SiLU (2H/256 slabs) -> QH (two-term,
// 12 items of 8 rows) -> W2 (8 slabs of 128, two planes, x += gate_m * y),
// then the next block's QX.  Each item waits until the previous stage of its
// band has finished, which makes the chain of a band linear (every buffer
// is rewritten only after all of its readers finished).  Items are handed
// out in block, stage, band order; a workgroup only ever waits for items
// with smaller tickets, which running workgroups hold, so the queue cannot
// deadlock.  Every wait is bounded: past the limit it sets the device error
// word and gives up, and once that word is set no item waits at all, so the
// grid always drains.
//
// Arithmetic: the same quantizer (iro_quant_row.h) and epilogues
// (iro_gemm_core.h) as the per-kernel path, so the result is bit-identical
// to it and to the reference's block sequence.
#include "iro_gemm_core.h"
#include "iro_quant_row.h"

#include <new>
#include <vector>

namespace iro {

namespace {

constexpr int kTI = 3;           // 32-row MFMA blocks per band
constexpr int kBand = 32 * kTI;  // rows per band
constexpr int kChunkBytes = 24 * 1024;  // one A chunk: 24 fragments of 1 KiB
constexpr int kNBuf = 3;                // A chunks in flight
constexpr int kQxRows = 16, kQhRows = 8;  // rows per quantization item
constexpr int kMaxXcd = 8;

enum PStage { PS_QX = 0, PS_QKVG, PS_QV, PS_WO, PS_QX2, PS_W13, PS_QH, PS_W2, PS_N };

// One block's packed weight as the kernel reads it.
struct PWeight {
    const int8_t *bp;
    const float *sw;
    const int32_t *colsum, *rowsum;
    int N, Kp, wbytes, part_n;
};

struct PParams {
    int M, D, H, S, blocks, two_w2;
    int band_lo[kMaxXcd + 1];  // XCD k owns bands [band_lo[k], band_lo[k+1])
    int n_items[PS_N];         // items per band of each stage
    int per_band;              // sum of n_items
    float *x, *q, *k, *v, *g, *hidden;
    const float *mod;
    int ldm, ada_np;
    uint8_t *c[5];             // codes: x, v, x2, hidden plane 1, hidden plane 2
    float *s[5];
    int32_t *z[5];
    const PWeight *w;          // [blocks][4]: QKVG, Wo, W1/W3, W2
    int *tickets;              // [kMaxXcd]
    int *done;                 // [PS_N][nbands], cumulative over the blocks
    int nbands;
    int *err;
    const uint8_t *zero16;
    int spin_limit;
};

__device__ __forceinline__ int xcc_id() {
    // HW_REG_XCC_ID (20), bits [3:0]
    return __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20);
}

__device__ __forceinline__ void waitcnt_vm0() {
    __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (15 << 8));
}

template <int VM>
__device__ __forceinline__ void waitcnt_vm() {
    static_assert(VM < 64, "vmcnt holds 6 bits");
    __builtin_amdgcn_s_waitcnt((VM & 15) | (7 << 4) | (15 << 8) | ((VM >> 4) << 14));
}

// Lane 0 of wave 0 waits until *ctr >= target (an atomic read, so the value
// is the one every CU of the XCD sees), then the whole workgroup drops its
// CU's L1 lines so that its loads see what the producers stored in L2.
__device__ __forceinline__ void acquire(const PParams &pp, int *ctr, int target, int tid) {
    if (tid == 0 && target > 0) {
        int n = 0;
        while (__hip_atomic_fetch_add(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) <
               target) {
            if (__hip_atomic_load(pp.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
            if (++n > pp.spin_limit) {
                __hip_atomic_fetch_or(pp.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    __syncthreads();
    // Device-scope invalidate: a workgroup-scope one (sc0) leaves the CU's
    // L1 alone outside thread-group-split mode, where the L1 already is the
    // workgroup's point of coherence.
    asm volatile("buffer_inv sc1" ::: "memory");
}

// Every wave's stores have reached L2; then the item is counted.
__device__ __forceinline__ void release(int *ctr, int tid) {
    waitcnt_vm0();
    __syncthreads();
    if (tid == 0) __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Rows [r0, r1) of src [M, K] (ld ldx) quantized into signed codes, one
// wave per row.
template <int CONV, int CH, bool RES>
__device__ __forceinline__ void quant_item(const float *src, int K, int r0, int r1, uint8_t *q1,
                                           float *s1, int32_t *z1, uint8_t *q2, float *s2,
                                           int32_t *z2, int tid) {
    const int lane = tid & 63, wave = tid >> 6;
    for (int row = r0 + wave; row < r1; row += 4) {
        float4 v[CH];
        load_row<CH, false>(src + (size_t)row * K, K, lane, v);
        quant_row<CONV, CH, RES, false>(v, row, K, lane, q1, K, s1, z1, nullptr, q2, s2, z2,
                                        0x80808080u);
    }
}

// One 96 x 128*TJ output tile of a GEMM item: the activation codes of the
// band pass through LDS in chunks of KC bytes of k (three buffers; chunk
// c+2 is copied by direct global-to-LDS loads while chunk c runs), each
// wave streams its TJ weight column blocks through a register ring R k
// blocks ahead, and the epilogue of the per-kernel path finishes the tile.
template <int CONV, int EPI, bool TWO, int TJ>
__device__ __forceinline__ void gemm_item(const KParams &p, int m0, int slab, uint8_t *lds,
                                          uint8_t *sink, void *rl_raw, const uint64_t *exptab,
                                          int tid) {
    constexpr int TI = kTI, BM = kBand, PL = TWO ? 2 : 1;
    constexpr int KC = TWO ? 128 : 256;
    constexpr int KBC = KC / 32;
    constexpr int FPL = KBC * TI;  // fragments per plane per chunk
    constexpr int FR = FPL * PL;
    constexpr int P = FR / 4;      // direct copies per wave per chunk
    constexpr int R = 4;           // weight ring depth (k blocks)
    static_assert(FR * 1024 == kChunkBytes && FR % 4 == 0 && KBC % R == 0, "chunk layout");
    constexpr int VM0 = R * TJ + P, VM1 = KBC * TJ + P, VM2 = 2 * KBC * TJ + P;
    RowLds<BM, TWO> &rl = *reinterpret_cast<RowLds<BM, TWO> *>(rl_raw);
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nb0 = slab * 4 * TJ + wave * TJ;  // first packed 32-row weight block of the wave

    stage_rows<EPI, TWO, BM>(p, rl, m0, tid);
    const ColParams<TJ> cp = load_cols<EPI, TJ>(p, nb0, lane, m0, BM);

    // Copy i of this wave in a chunk is fragment f = wave + 4 i: plane f /
    // FPL, k block (f % FPL) / TI, row block f % TI; lane L copies row
    // 32 rb + L % 32, k bytes 32 kbl + 16 (L / 32) .. +15 (rows past M repeat
    // row M-1; they are never stored).
    const uint8_t *src[P];
    int dst[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const int f = wave + 4 * i;
        const int pl = f / FPL, ff = f % FPL;
        const int kbl = ff / TI, rb = ff % TI;
        int row = m0 + rb * 32 + (lane & 31);
        row = row < p.M ? row : p.M - 1;
        src[i] = (pl ? p.a2 : p.a1) + (size_t)row * p.lda + kbl * 32 + (lane >> 5) * 16;
        dst[i] = f * 1024;
    }
    const int nc = p.K / KC;
    const int nkb = p.K / 32;
    // Chunks past the last one copy the zero page into a sink, so every
    // chunk issues the same number of loads and the waits below count right.
    auto copy_chunk = [&](int c) {
        if (c < nc) {
            uint8_t *base = lds + (c % kNBuf) * kChunkBytes;
#pragma unroll
            for (int i = 0; i < P; ++i) dma16(src[i] + c * KC, base + dst[i]);
        } else {
#pragma unroll
            for (int i = 0; i < P; ++i) dma16(p.zero16, sink);
        }
    };
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
    v4i rb[R][TJ];
    auto load_b = [&](v4i (&d)[TJ], int kb) {
        kb = kb < nkb ? kb : nkb - 1;  // past the end: a repeat, never consumed
#pragma unroll
        for (int j = 0; j < TJ; ++j) d[j] = load_frag(wr, lane * 16, wbase + j * jstride + kb * 1024);
    };
    auto read_a = [&](v4i (&a)[PL][TI], const uint8_t *abuf, int kbl) {
#pragma unroll
        for (int pl = 0; pl < PL; ++pl)
#pragma unroll
            for (int i = 0; i < TI; ++i)
                a[pl][i] = *reinterpret_cast<const v4i *>(
                    abuf + ((pl * FPL + kbl * TI + i) * 64 + lane) * 16);
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

    // Issue order: chunk 0, the first R weight k blocks, chunk 1; chunk c
    // then copies chunk c+2 after its barrier and refills the ring once per
    // k step.  So behind chunk c's copies there are R*TJ + P loads when
    // chunk 0 starts, KBC*TJ + P at chunk 1 and 2*KBC*TJ + P later.
    copy_chunk(0);
#pragma unroll
    for (int u = 0; u < R; ++u) load_b(rb[u], u);
    copy_chunk(1);
    for (int c = 0; c < nc; ++c) {
        if (c == 0)
            waitcnt_vm<VM0>();
        else if (c == 1)
            waitcnt_vm<VM1>();
        else
            waitcnt_vm<VM2>();
        __syncthreads();
        // The buffer chunk c+2 lands in held chunk c-1, which every wave
        // finished before the barrier.
        copy_chunk(c + 2);
        const uint8_t *abuf = lds + (c % kNBuf) * kChunkBytes;
        const int g0 = c * KBC;
        v4i a0[PL][TI], a1[PL][TI];
        read_a(a0, abuf, 0);
#pragma unroll
        for (int u = 0; u < KBC; u += 2) {
            read_a(a1, abuf, u + 1);
            fence_sched();
            mma(a0, rb[u % R]);
            load_b(rb[u % R], g0 + u + R);
            fence_sched();
            if (u + 2 < KBC) read_a(a0, abuf, u + 2);
            fence_sched();
            mma(a1, rb[(u + 1) % R]);
            load_b(rb[(u + 1) % R], g0 + u + 1 + R);
            fence_sched();
        }
    }
    waitcnt_vm0();  // the ring's last (unused) refills and the sink copies
    epilogue<CONV, EPI, TWO, TI, TJ, BM>(p, acc, acc2, cp, rl, exptab, m0, nb0, lane);
}

__device__ __forceinline__ KParams gemm_params(const PParams &pp, const PWeight &w,
                                               const uint8_t *a1, const uint8_t *a2,
                                               const float *s1, const float *s2,
                                               const int32_t *z1, const int32_t *z2, int K) {
    KParams p{};
    p.a1 = a1;
    p.a2 = a2;
    p.lda = K;
    p.bp = w.bp;
    p.kb_count = w.Kp / 32;
    p.M = pp.M;
    p.N = w.N;
    p.K = K;
    p.sx1 = s1;
    p.sx2 = s2;
    p.zx1 = z1;
    p.zx2 = z2;
    p.sw = w.sw;
    p.colsum = w.colsum;
    p.rowsum = w.rowsum;
    p.rows_per_branch = pp.S;
    p.zero16 = pp.zero16;
    p.wbytes = w.wbytes;
    return p;
}

template <int CONV, int CHX, int CHH>
__global__ __launch_bounds__(256, 2) void persist_stack_kernel(PParams pp) {
    __shared__ __attribute__((aligned(16))) uint8_t lds_a[kNBuf * kChunkBytes];
    __shared__ __attribute__((aligned(16))) uint8_t lds_sink[1024];  // never read
    __shared__ __attribute__((aligned(16))) uint8_t rl_raw[sizeof(RowLds<kBand, true>)];
    __shared__ uint64_t exptab[32];
    __shared__ int s_ticket;
    const int tid = threadIdx.x;
    if (tid < 32) exptab[tid] = kExp2Tab[tid];
    const int xcc = xcc_id();
    if (xcc >= kMaxXcd) {
        if (tid == 0) __hip_atomic_fetch_or(pp.err, 4, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    const int blo = pp.band_lo[xcc];
    const int nbk = pp.band_lo[xcc + 1] - blo;
    const int per_block = nbk * pp.per_band;
    const int total = per_block * pp.blocks;
    const int D = pp.D, H = pp.H;
    for (;;) {
        __syncthreads();  // the previous item's LDS and s_ticket are free
        if (tid == 0) s_ticket = __hip_atomic_fetch_add(&pp.tickets[xcc], 1, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        const int t = s_ticket;
        if (t >= total) break;
        // ticket -> (block, stage, band, sub-item): block-major, then stage,
        // then band, then the stage's items of the band
        const int blk = t / per_block;
        int r = t - blk * per_block;
        int st = 0;
        while (r >= nbk * pp.n_items[st]) {
            r -= nbk * pp.n_items[st];
            ++st;
        }
        const int bl = r / pp.n_items[st];
        const int sub = r - bl * pp.n_items[st];
        const int band = blo + bl;
        const int m0 = band * kBand;
        int *done = pp.done + st * pp.nbands + band;
        // the previous stage of this band (the previous block's W2 for QX)
        if (st == PS_QX) {
            if (blk > 0)
                acquire(pp, pp.done + PS_W2 * pp.nbands + band, pp.n_items[PS_W2] * blk, tid);
        } else {
            acquire(pp, pp.done + (st - 1) * pp.nbands + band, pp.n_items[st - 1] * (blk + 1),
                    tid);
        }
        const PWeight *wb = pp.w + blk * 4;
        const float *mod = pp.mod + (size_t)blk * pp.ada_np;
        switch (st) {
            case PS_QX:
            case PS_QV:
            case PS_QX2: {
                const int ci = st == PS_QX ? 0 : (st == PS_QV ? 1 : 2);
                const float *src = st == PS_QV ? pp.v : pp.x;
                const int r0 = m0 + sub * kQxRows;
                const int r1 = min(r0 + kQxRows, pp.M);
                quant_item<CONV, CHX, false>(src, D, r0, r1, pp.c[ci], pp.s[ci], pp.z[ci],
                                             nullptr, nullptr, nullptr, tid);
                break;
            }
            case PS_QH: {
                const int r0 = m0 + sub * kQhRows;
                const int r1 = min(r0 + kQhRows, pp.M);
                if (pp.two_w2)
                    quant_item<CONV, CHH, true>(pp.hidden, H, r0, r1, pp.c[3], pp.s[3], pp.z[3],
                                                pp.c[4], pp.s[4], pp.z[4], tid);
                else
                    quant_item<CONV, CHH, false>(pp.hidden, H, r0, r1, pp.c[3], pp.s[3], pp.z[3],
                                                 nullptr, nullptr, nullptr, tid);
                break;
            }
            case PS_QKVG: {
                KParams p = gemm_params(pp, wb[0], pp.c[0], nullptr, pp.s[0], nullptr, pp.z[0],
                                        nullptr, D);
                p.seg0 = pp.q;
                p.seg1 = pp.k;
                p.seg2 = pp.v;
                p.seg3 = pp.g;
                p.seg_n = wb[0].part_n;
                gemm_item<CONV, EPI_QKVG, false, 2>(p, m0, sub, lds_a, lds_sink, rl_raw, exptab,
                                                    tid);
                break;
            }
            case PS_WO: {
                KParams p = gemm_params(pp, wb[1], pp.c[1], nullptr, pp.s[1], nullptr, pp.z[1],
                                        nullptr, D);
                p.xres = pp.x;
                p.gate = mod + 2 * D;
                p.ldg = pp.ldm;
                p.ldx = D;
                gemm_item<CONV, EPI_GATED, false, 2>(p, m0, sub, lds_a, lds_sink, rl_raw, exptab,
                                                     tid);
                break;
            }
            case PS_W13: {
                KParams p = gemm_params(pp, wb[2], pp.c[2], nullptr, pp.s[2], nullptr, pp.z[2],
                                        nullptr, D);
                p.hidden = pp.hidden;
                p.ldh = H;
                p.hidden_n = wb[2].part_n;
                gemm_item<CONV, EPI_SWIGLU, false, 2>(p, m0, sub, lds_a, lds_sink, rl_raw, exptab,
                                                      tid);
                break;
            }
            default: {  // PS_W2
                KParams p = gemm_params(pp, wb[3], pp.c[3], pp.two_w2 ? pp.c[4] : nullptr,
                                        pp.s[3], pp.s[4], pp.z[3], pp.z[4], H);
                p.xres = pp.x;
                p.gate = mod + 5 * D;
                p.ldg = pp.ldm;
                p.ldx = D;
                if (pp.two_w2)
                    gemm_item<CONV, EPI_GATED, true, 1>(p, m0, sub, lds_a, lds_sink, rl_raw,
                                                        exptab, tid);
                else
                    gemm_item<CONV, EPI_GATED, false, 1>(p, m0, sub, lds_a, lds_sink, rl_raw,
                                                         exptab, tid);
                break;
            }
        }
        release(done, tid);
    }
}

// After the step: every band's last stage must have counted all of its
// items; otherwise some XCD's queue was not (fully) served and the error
// word says so.
__global__ __launch_bounds__(256) void persist_check_kernel(const int *done, int nbands, int want,
                                                            int *err) {
    for (int b = threadIdx.x; b < nbands; b += 256)
        if (done[PS_W2 * nbands + b] != want)
            __hip_atomic_fetch_or(err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

// ---- host side -----------------------------------------------------------------

struct PersistPlan {
    int M = 0, nbands = 0;
    uint8_t *codes = nullptr;  // one allocation for codes, scales, zero points, sync words
    size_t bytes = 0;
    PParams pp{};
    PWeight *wdev = nullptr;
    int wblocks = 0;
};

bool persist_supported(int D, int H, int residual_mask) {
    return D % 256 == 0 && D <= 1024 && H % 256 == 0 && H <= 3072 && (residual_mask & 7) == 0;
}

void persist_free(PersistPlan *pl) {
    if (!pl) return;
    if (pl->codes) (void)hipFree(pl->codes);
    if (pl->wdev) (void)hipFree(pl->wdev);
    delete pl;
}

// Buffers for M rows and the weight table of `blocks` blocks (weights[b*4 +
// i]: QKVG, Wo, W1/W3, W2).  Allocates; call outside graph capture.
int persist_prepare(IroHipContext *ctx, PersistPlan **plp, int M, int D, int H, int S, int blocks,
                    int two_w2, const IroHipWeight *const *weights, float *q, float *k, float *v,
                    float *g, float *hidden, const float *mod, int ldm, int ada_np) {
    PersistPlan *pl = *plp;
    if (!pl) {
        pl = new (std::nothrow) PersistPlan();
        if (!pl) return set_error(ctx, "persistent stack: out of host memory");
        *plp = pl;
    }
    const int nbands = (M + kBand - 1) / kBand;
    if (pl->M != M) {
        if (pl->codes) (void)hipFree(pl->codes);
        pl->codes = nullptr;
        const size_t md = round_up((size_t)M * D, 256), mh = round_up((size_t)M * H, 256);
        const size_t rows = round_up(4 * (size_t)M, 256);
        const size_t sync = round_up(sizeof(int) * (kMaxXcd + PS_N * (size_t)nbands + 1), 256);
        pl->bytes = 3 * md + 2 * mh + 10 * rows + sync;
        IRO_HIP_TRY(ctx, hipMalloc(&pl->codes, pl->bytes));
        uint8_t *b = pl->codes;
        for (int i = 0; i < 5; ++i) {
            pl->pp.c[i] = b;
            b += i < 3 ? md : mh;
        }
        for (int i = 0; i < 5; ++i) {
            pl->pp.s[i] = reinterpret_cast<float *>(b);
            b += rows;
            pl->pp.z[i] = reinterpret_cast<int32_t *>(b);
            b += rows;
        }
        pl->pp.tickets = reinterpret_cast<int *>(b);
        pl->pp.done = pl->pp.tickets + kMaxXcd;
        pl->M = M;
        pl->nbands = nbands;
    }
    if (pl->wblocks != blocks) {
        if (pl->wdev) (void)hipFree(pl->wdev);
        pl->wdev = nullptr;
        IRO_HIP_TRY(ctx, hipMalloc(&pl->wdev, sizeof(PWeight) * 4 * (size_t)blocks));
        pl->wblocks = blocks;
    }
    std::vector<PWeight> wt(4 * (size_t)blocks);
    for (int i = 0; i < 4 * blocks; ++i) {
        const IroHipWeight *w = weights[i];
        wt[i] = PWeight{w->packed, w->scale, w->colsum, w->rowsum ? w->rowsum : w->colsum,
                        w->N, w->Kp, w->Np * w->Kp, w->part_N[0]};
    }
    IRO_HIP_TRY(ctx, hipMemcpyAsync(pl->wdev, wt.data(), sizeof(PWeight) * wt.size(),
                                    hipMemcpyHostToDevice, ctx->stream));
    IRO_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    PParams &pp = pl->pp;
    pp.M = M;
    pp.D = D;
    pp.H = H;
    pp.S = S;
    pp.blocks = blocks;
    pp.two_w2 = two_w2;
    for (int k = 0; k <= kMaxXcd; ++k) pp.band_lo[k] = (int)((long long)nbands * k / kMaxXcd);
    pp.n_items[PS_QX] = kBand / kQxRows;
    pp.n_items[PS_QKVG] = 4 * D / 256;
    pp.n_items[PS_QV] = kBand / kQxRows;
    pp.n_items[PS_WO] = D / 256;
    pp.n_items[PS_QX2] = kBand / kQxRows;
    pp.n_items[PS_W13] = 2 * H / 256;
    pp.n_items[PS_QH] = kBand / kQhRows;
    pp.n_items[PS_W2] = D / 128;
    pp.per_band = 0;
    for (int s = 0; s < PS_N; ++s) pp.per_band += pp.n_items[s];
    pp.q = q;
    pp.k = k;
    pp.v = v;
    pp.g = g;
    pp.hidden = hidden;
    pp.mod = mod;
    pp.ldm = ldm;
    pp.ada_np = ada_np;
    pp.w = pl->wdev;
    pp.nbands = nbands;
    pp.err = ctx->dev_err;
    pp.zero16 = static_cast<const uint8_t *>(ctx->zero16);
    pp.spin_limit = 1 << 22;
    return 0;
}

// The step's queue: zero the tickets and counters (a fill kernel, so the
// launch can be captured), the persistent kernel on two workgroups per CU,
// then the completion check.
int persist_launch(IroHipContext *ctx, PersistPlan *pl, float *x) {
    PParams pp = pl->pp;
    pp.x = x;
    const size_t sync = sizeof(int) * (kMaxXcd + PS_N * (size_t)pl->nbands);
    if (launch_fill(ctx, pp.tickets, 0, sync)) return -1;
    const unsigned grid = (unsigned)(2 * (ctx->cus > 0 ? ctx->cus : 256));
    prof_begin(ctx);
    if (ctx->convention == IRO_HIP_GCC_FASTMATH)
        hipLaunchKernelGGL((persist_stack_kernel<1, 4, 12>), dim3(grid), dim3(256), 0,
                           ctx->stream, pp);
    else
        hipLaunchKernelGGL((persist_stack_kernel<0, 4, 12>), dim3(grid), dim3(256), 0,
                           ctx->stream, pp);
    IRO_HIP_CHECK_LAUNCH(ctx);
    const double M = pp.M, D = pp.D, H = pp.H;
    const double ops = pp.blocks * (2 * M * D * 4 * D + 2 * M * D * D + 2 * M * D * 2 * H +
                                    2 * M * H * D * (pp.two_w2 ? 2 : 1));
    prof_end(ctx, PK_PERSIST_STACK, ops, 0.0);
    hipLaunchKernelGGL(persist_check_kernel, dim3(1), dim3(256), 0, ctx->stream, pp.done,
                       pl->nbands, pp.n_items[PS_W2] * pp.blocks, pp.err);
    IRO_HIP_CHECK_LAUNCH(ctx);
    return 0;
}

}  // namespace iro
