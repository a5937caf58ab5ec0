// iro_gemm_core.h -- device pieces shared by the int8 GEMM kernels
// (iro_gemm.hip) and the persistent DiT stack kernel (iro_persist.hip):
// the kernel parameter block, the reference's dequantization epilogues
// (ops.c:468-490, dit.c:786-792, 945-956, 1013-1020), the SiLU gate, row and
// column parameter staging, direct global-to-LDS copies and the weight
// fragment loads.  Everything here is inline device code in an anonymous
// namespace: each including file gets its own copy.
#pragma once

#include "iro_expf.h"
#include "iro_internal.h"
#include "iro_round.h"

#include <type_traits>

namespace iro {

// Parameters of one GEMM launch (all kernels, all epilogues).
struct KParams {
    const uint8_t *a1, *a2;
    int lda;
    const int8_t *bp;
    int kb_count;  // Kp / 32
    int M, N, K;
    const float *sx1, *sx2;
    const int32_t *zx1, *zx2;
    const float *sw;
    const int32_t *colsum;
    const int32_t *rowsum;
    const float *bias;
    float *y;
    const float *yin;  // accumulate: the prior output rows, nullptr = y itself
    int ldy;
    int32_t *work;
    int ldw;
    int accumulate;
    float *seg0, *seg1, *seg2, *seg3;
    int seg_n;
    float *hidden;
    int ldh;
    int hidden_n;
    float *xres;
    const float *gate;
    int ldg;
    int ldx;
    int rows_per_branch;
    int tiles_n, tiles_m;  // tiles of the tile kernel along N and M
    int tiles_per_xcd;     // ceil(tiles / 8)
    int row_major;         // tile order, see tile_of
    int aflip;             // XOR applied to stored codes: 0x80808080 for u8 codes, 0 if signed
    int spb, groups_n;     // whole-tile kernel: column slabs per block, slab groups per row
    const uint8_t *zero16; // 256 zero bytes
    int wbytes;            // bytes of the packed weight (< 2^31)
    int akbp;              // > 0: A codes in the MFMA fragment layout, akbp k blocks per row block
    // SwiGLU epilogue that quantizes the hidden state itself (hq1 set):
    // signed codes [M, ldhq] of each plane, row scales and zero points, and
    // the band exchange state (per band: arrivals of the two range phases
    // and departures; per row: |lo|, hi of each phase as float bits).
    uint8_t *hq1, *hq2;
    int ldhq;
    float *hs1, *hs2;
    int32_t *hz1, *hz2;
    unsigned *band_cnt, *band_rng;
    int *err;
    int spin_limit;
};

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

using I0 = std::integral_constant<int, 0>;
using I1 = std::integral_constant<int, 1>;




// ops.c:468-490: y = t*c [+ b] or y += t*c [+ b] with the build's rounding.
template <int CONV>
__device__ __forceinline__ float lin_out(float t, float c, float b, bool has_bias, bool acc,
                                         float yold) {
    if (CONV == 1) {
        if (acc && has_bias) return __builtin_fmaf(t, c, yold + b);
        if (acc) return __builtin_fmaf(t, c, yold);
        if (has_bias) return __builtin_fmaf(t, c, b);
        return t * c;
    }
    if (acc && has_bias) return yold + (t * c + b);
    if (acc) return yold + t * c;
    if (has_bias) return t * c + b;
    return t * c;
}

// Second plane accumulated without bias (accumulate = 1 branch).
template <int CONV>
__device__ __forceinline__ float add_term(float y, float t, float c) {
    return CONV == 1 ? __builtin_fmaf(t, c, y) : y + t * c;
}

// a / b, correctly rounded, for b = 1 + expf(-a) (so b >= 1): reciprocal,
// one Newton step, the quotient and one remainder correction (Markstein)
// give the IEEE quotient when b < 2^64 and 2^-100 <= |a| < 2^126, checked
// against the IEEE division for every float a on the GPU; zeros return a
// (= a / b); the remaining lanes (a < -44, denormal or non-finite a) take
// the IEEE division.
__device__ __forceinline__ float silu_div(float a, float b) {
    const float aa = __builtin_fabsf(a);
    const bool fast = b < 0x1p64f && aa < 0x1p126f && (aa >= 0x1p-100f || a == 0.0f);
    const float y = __builtin_amdgcn_rcpf(b);
    const float y1 = __builtin_fmaf(__builtin_fmaf(-b, y, 1.0f), y, y);
    const float q0 = a * y1;
    float q = __builtin_fmaf(__builtin_fmaf(-b, q0, a), y1, q0);
    q = a == 0.0f ? a : q;
    if (__builtin_expect(!fast, 0)) q = a / b;
    return q;
}

// ops.c:781-784 as the strict build computes it: x / (1 + expf(-x)) * g.
__device__ __forceinline__ float silu_mul(float a, float g, const uint64_t *tab) {
    const float e = expf_glibc(-a, tab);
    return silu_div(a, 1.0f + e) * g;
}

// The quotient a / (1 + expf(-a)) on the gate's common inputs (ok):
// -44 < a, |a| < 2^126, and |a| >= 2^-100 or a == 0.  There expf(-a) <
// 2^64 cannot overflow, and where glibc's expf underflows to 0 (a > 103.97)
// the table value of the clamped input is below 2^-24, so 1 + e is the
// same without expf's special-case selects, and silu_div's fast quotient
// applies (b < 2^64).  Inputs with ok false must take silu_mul.  Checked
// against the IEEE quotient for every float a by iro_hip_selfcheck_silu.
__device__ __forceinline__ float silu_q_common(float a, const uint64_t *tab, bool &ok) {
    const float aa = __builtin_fabsf(a);
    ok = a > -44.0f && aa < 0x1p126f && (aa >= 0x1p-100f || a == 0.0f);
    const float b = 1.0f + expf_glibc_table(-a, tab);
    const float y = __builtin_amdgcn_rcpf(b);
    const float y1 = __builtin_fmaf(__builtin_fmaf(-b, y, 1.0f), y, y);
    const float q0 = a * y1;
    const float q = __builtin_fmaf(__builtin_fmaf(-b, q0, a), y1, q0);
    return a == 0.0f ? a : q;
}

// silu_mul over 16 values: the common path for all of them, then one
// (rarely taken) branch that redoes the others with silu_mul.
__device__ __forceinline__ void silu_mul16(const float (&a)[16], const float (&g)[16],
                                           const uint64_t *tab, float (&h)[16]) {
    uint32_t rare = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        bool ok;
        h[r] = silu_q_common(a[r], tab, ok) * g[r];
        rare |= ok ? 0u : 1u << r;
    }
    if (__builtin_expect(rare != 0, 0)) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if ((rare >> r) & 1u) h[r] = silu_mul(a[r], g[r], tab);
    }
}

// Per-row parameters of a block's rows, staged in LDS: scale and zero
// point of each plane and the gate row offset of the gated epilogue.
template <int BM, bool TWO>
struct RowLds {
    float sx[TWO ? 2 : 1][BM];
    int zx[TWO ? 2 : 1][BM];
    int goff[BM];
};

template <int EPI, bool TWO, int BM>
__device__ __forceinline__ void stage_rows(const KParams &p, RowLds<BM, TWO> &r, int m0, int tid) {
    if (tid < BM) {
        int m = m0 + tid;
        m = m < p.M ? m : p.M - 1;
        r.sx[0][tid] = p.sx1[m];
        r.zx[0][tid] = p.zx1[m];
        if (TWO) {
            r.sx[TWO ? 1 : 0][tid] = p.sx2[m];
            r.zx[TWO ? 1 : 0][tid] = p.zx2[m];
        }
        if (EPI == EPI_GATED) r.goff[tid] = (m / p.rows_per_branch) * p.ldg;
    }
}

// Per-column parameters of the TJ 32-column blocks of one wave (packed
// column order), loaded before the main loop so their latency is hidden.
template <int TJ>
struct ColParams {
    int cs[TJ], rs[TJ];
    float sw[TJ], b[TJ];
    float glo[TJ], ghi[TJ];  // gated epilogue: gate of the tile's first and last branch
};

// Gate rows of the gated epilogue (dit.c:1013-1020): row m uses gate row
// m / rows_per_branch.  A tile whose rows fall in at most two branches
// takes both gate values per column up front and selects per row.
__device__ __forceinline__ int gate_branch_lo(const KParams &p, int m0) {
    return m0 / p.rows_per_branch;
}
__device__ __forceinline__ int gate_branch_hi(const KParams &p, int m0, int bm) {
    const int last = (m0 + bm < p.M ? m0 + bm : p.M) - 1;
    return last / p.rows_per_branch;
}

template <int EPI, int TJ>
__device__ __forceinline__ ColParams<TJ> load_cols(const KParams &p, int nb0, int lane, int m0,
                                                   int bm) {
    ColParams<TJ> c;
    const int blo = EPI == EPI_GATED ? gate_branch_lo(p, m0) : 0;
    const int bhi = EPI == EPI_GATED ? gate_branch_hi(p, m0, bm) : 0;
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const int pc = (nb0 + j) * 32 + (lane & 31);  // packed: padded to Np, in bounds
        c.cs[j] = p.colsum[pc];
        c.rs[j] = p.rowsum[pc];
        c.sw[j] = p.sw[pc];
        c.b[j] = (EPI == EPI_LINEAR && p.bias && pc < p.N) ? p.bias[pc] : 0.0f;
        if (EPI == EPI_GATED) {
            const int gc = pc < p.N ? pc : p.N - 1;  // padded columns are never stored
            c.glo[j] = p.gate[blo * p.ldg + gc];
            c.ghi[j] = p.gate[bhi * p.ldg + gc];
        } else {
            c.glo[j] = c.ghi[j] = 0.0f;
        }
    }
    return c;
}

// Epilogue of one wave's TI x TJ accumulator tiles.  The QKVG planes and
// the SwiGLU hidden state, the two largest output streams, are stored
// nontemporally (measured 1-2 % faster over the stack: the store bursts of
// all blocks drain sooner when they do not displace cached lines).  32x32 accumulator
// layout: lane L, register r holds row 8*(r/4) + 4*(L/32) + r%4 and column
// L%32 of the tile.  Row (m0 + i*32 + 8*g + e) is wave-uniform, so every
// store address is a scalar row base plus one per-lane offset fixed per
// column block.  FULL tiles (all rows < M, all columns < N, and for the
// gated epilogue at most two gate branches) store without predicates; the
// others clamp their loads to row M-1, predicate stores and gather the gate
// per element.
template <int CONV, int EPI, bool TWO, int TI, int TJ, int BM, bool FULL, bool RAW>
__device__ __forceinline__ void epilogue_body(const KParams &p, const v16i (&acc)[TI][TJ],
                                              const v16i (&acc2)[TI][TJ],
                                              const ColParams<TJ> &cp, const RowLds<BM, TWO> &rl,
                                              const uint64_t *exptab, int m0, int nb0, int lane) {
    const bool has_bias = EPI == EPI_LINEAR && p.bias != nullptr;
    const int half = lane >> 5;
    int pc[TJ], c128[TJ];
    unsigned off[TJ];  // element offset of (row m0-relative half*4, column) from a row base
    float *segp[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        pc[j] = (nb0 + j) * 32 + (lane & 31);
        c128[j] = RAW ? 0 : 128 * cp.rs[j];
        if (EPI == EPI_QKVG) {
            const int sg = pc[j] / p.seg_n;
            segp[j] = sg == 0 ? p.seg0 : (sg == 1 ? p.seg1 : (sg == 2 ? p.seg2 : p.seg3));
            segp[j] += pc[j] - sg * p.seg_n + (size_t)half * 4 * p.seg_n;
        } else if (EPI == EPI_LINEAR) {
            off[j] = (unsigned)(half * 4 * p.ldy + pc[j]);
        } else if (EPI == EPI_GATED) {
            off[j] = (unsigned)(half * 4 * p.ldx + pc[j]);
        }
    }
    unsigned offh[TJ / 2 > 0 ? TJ / 2 : 1];
    if (EPI == EPI_SWIGLU) {
#pragma unroll
        for (int j = 0; j + 1 < TJ; j += 2)
            offh[j / 2] = (unsigned)(half * 4 * p.ldh + ((nb0 + j) >> 1) * 32 + (lane & 31));
    }
    // Gated residual: every old x of the wave tile is loaded before the
    // first store (the stores may alias later loads for the compiler, which
    // would otherwise serialize one load round trip per 32x32 block).  Full
    // tiles span at most two gate branches: rows below gbnd take glo.
    // Tiles of three 32-row blocks load each block's old x just before it
    // (all of them at once would hold another 96 registers per lane).
    constexpr bool XALL = TI <= 2;
    constexpr int GI = EPI == EPI_GATED ? (XALL ? TI : 1) : 1, GJ = EPI == EPI_GATED ? TJ : 1;
    float xold[GI][GJ][16];
    const int gbnd = EPI == EPI_GATED ? (gate_branch_lo(p, m0) + 1) * p.rows_per_branch : 0;
    auto load_xold = [&](int gi, int i) {
#pragma unroll
        for (int j = 0; j < GJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                int m = m0 + i * 32 + (r >> 2) * 8 + (r & 3);
                if (!FULL) m = m + half * 4 < p.M ? m : p.M - 1 - half * 4;
                xold[gi][j][r] = (FULL || pc[j] < p.N)
                                     ? p.xres[(long long)m * p.ldx + off[j]] : 0.0f;
            }
    };
    if (EPI == EPI_GATED && XALL) {
#pragma unroll
        for (int i = 0; i < GI; ++i) load_xold(i, i);
    }
#pragma unroll
    for (int i = 0; i < TI; ++i) {
        if (EPI == EPI_GATED && !XALL) load_xold(0, i);
        float sx[16], sx2[16];
        int zx[16], zx2[16], goff[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int rb = i * 32 + g * 8 + half * 4;
            const float4 s4 = *reinterpret_cast<const float4 *>(&rl.sx[0][rb]);
            const int4 z4 = *reinterpret_cast<const int4 *>(&rl.zx[0][rb]);
            sx[g * 4 + 0] = s4.x; sx[g * 4 + 1] = s4.y; sx[g * 4 + 2] = s4.z; sx[g * 4 + 3] = s4.w;
            zx[g * 4 + 0] = z4.x; zx[g * 4 + 1] = z4.y; zx[g * 4 + 2] = z4.z; zx[g * 4 + 3] = z4.w;
            if (TWO) {
                const float4 t4 = *reinterpret_cast<const float4 *>(&rl.sx[TWO ? 1 : 0][rb]);
                const int4 w4 = *reinterpret_cast<const int4 *>(&rl.zx[TWO ? 1 : 0][rb]);
                sx2[g * 4 + 0] = t4.x; sx2[g * 4 + 1] = t4.y; sx2[g * 4 + 2] = t4.z; sx2[g * 4 + 3] = t4.w;
                zx2[g * 4 + 0] = w4.x; zx2[g * 4 + 1] = w4.y; zx2[g * 4 + 2] = w4.z; zx2[g * 4 + 3] = w4.w;
            }
            if (EPI == EPI_GATED && !FULL) {
                const int4 o4 = *reinterpret_cast<const int4 *>(&rl.goff[rb]);
                goff[g * 4 + 0] = o4.x; goff[g * 4 + 1] = o4.y; goff[g * 4 + 2] = o4.z; goff[g * 4 + 3] = o4.w;
            }
        }
        // Row of register r is rowu(r) + half*4; rowu is wave-uniform.
        auto rowu = [&](int r) { return m0 + i * 32 + (r >> 2) * 8 + (r & 3); };
        auto row_ok = [&](int r) { return FULL || rowu(r) + half * 4 < p.M; };
        // Uniform row base used for loads: in partial tiles it is pulled back
        // so the lane's row base + half*4 is at most M-1 (it may be negative
        // when M < 5; base + per-lane offset is then still a valid row).
        auto row_ld = [&](int r) {
            int m = rowu(r);
            if (!FULL) m = m + half * 4 < p.M ? m : p.M - 1 - half * 4;
            return m;
        };
        float yv[TJ][16];
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const bool col_ok = FULL || pc[j] < p.N;
            float old[16], gv[16];
            if (EPI == EPI_LINEAR && p.accumulate) {
                const float *yo = p.yin ? p.yin : p.y;
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    old[r] = col_ok ? yo[(long long)row_ld(r) * p.ldy + off[j]] : 0.0f;
            }
            if (EPI == EPI_GATED) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    old[r] = xold[EPI == EPI_GATED && XALL ? i : 0][EPI == EPI_GATED ? j : 0][r];
                    if (FULL)
                        gv[r] = rowu(r) + half * 4 < gbnd ? cp.glo[j] : cp.ghi[j];
                    else
                        gv[r] = col_ok ? p.gate[goff[r] + pc[j]] : 0.0f;
                }
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int raw = acc[i][j][r] + c128[j];
                const float t = (float)(raw - __mul24(zx[r], cp.cs[j]));
                const float c = sx[r] * cp.sw[j];
                float y;
                if (EPI == EPI_LINEAR)
                    y = lin_out<CONV>(t, c, cp.b[j], has_bias, p.accumulate != 0,
                                      p.accumulate ? old[r] : 0.0f);
                else
                    y = t * c;
                if (TWO) {
                    const int raw2 = acc2[i][j][r] + c128[j];
                    const float t2 = (float)(raw2 - __mul24(zx2[r], cp.cs[j]));
                    const float c2 = sx2[r] * cp.sw[j];
                    y = add_term<CONV>(y, t2, c2);
                }
                yv[j][r] = y;
                const bool ok = row_ok(r) && col_ok;
                const size_t ru = (size_t)rowu(r);
                if (EPI == EPI_LINEAR) {
                    if (ok) {
                        p.y[ru * p.ldy + off[j]] = y;
                        if (p.work) p.work[(ru + half * 4) * p.ldw + pc[j]] = raw;
                    }
                } else if (EPI == EPI_QKVG) {
                    if (ok) __builtin_nontemporal_store(y, &segp[j][ru * p.seg_n]);
                } else if (EPI == EPI_GATED) {
                    if (ok)
                        p.xres[ru * p.ldx + off[j]] =
                            CONV == 1 ? __builtin_fmaf(gv[r], y, old[r]) : old[r] + gv[r] * y;
                }
            }
        }
        if (EPI == EPI_SWIGLU) {
            // Interleaved W1/W3: column block nb0+j (j even) is W1 block
            // (nb0+j)/2, block nb0+j+1 the matching W3 block.
#pragma unroll
            for (int j = 0; j + 1 < TJ; j += 2) {
                const bool hok = FULL || ((nb0 + j) >> 1) * 32 + (lane & 31) < p.hidden_n;
                float hv[16];
                silu_mul16(yv[j], yv[j + 1], exptab, hv);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    if (row_ok(r) && hok)
                        __builtin_nontemporal_store(hv[r], &p.hidden[(size_t)rowu(r) * p.ldh + offh[j / 2]]);
                }
            }
        }
    }
}

template <int CONV, int EPI, bool TWO, int TI, int TJ, int BM, bool RAW = false>
__device__ __forceinline__ void epilogue(const KParams &p, const v16i (&acc)[TI][TJ],
                                         const v16i (&acc2)[TI][TJ], const ColParams<TJ> &cp,
                                         const RowLds<BM, TWO> &rl, const uint64_t *exptab,
                                         int m0, int nb0, int lane) {
    const int ncols = EPI == EPI_SWIGLU ? 2 * p.hidden_n : p.N;
    bool full = m0 + BM <= p.M && (nb0 + TJ) * 32 <= ncols;
    if (EPI == EPI_GATED) full = full && gate_branch_hi(p, m0, BM) - gate_branch_lo(p, m0) <= 1;
    if (full)
        epilogue_body<CONV, EPI, TWO, TI, TJ, BM, true, RAW>(p, acc, acc2, cp, rl, exptab, m0,
                                                             nb0, lane);
    else
        epilogue_body<CONV, EPI, TWO, TI, TJ, BM, false, RAW>(p, acc, acc2, cp, rl, exptab, m0,
                                                              nb0, lane);
}

// Direct global-to-LDS copy of 16 bytes per lane (global_load_lds_dwordx4:
// lane L writes at the wave-uniform LDS address + 16 L).  Written as inline
// assembly so that the compiler's wait-count insertion, which cannot tell
// which LDS bytes a copy writes, does not drain every outstanding load
// before each later LDS read; callers wait for the copies themselves.
__device__ __forceinline__ void dma16(const uint8_t *src, uint8_t *lds) {
    const uint32_t a = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)lds);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(src), "s"(a)
                 : "memory", "m0");
}

// Scheduling fence between the parts of a main-loop k step.  Each step
// issues the LDS reads of the next step's activation fragments, then (after
// a fence) its own MFMAs and the weight loads that refill the ring.  Without
// the fences the scheduler sinks the LDS reads below the MFMAs (and shares
// their registers with the current step's), which exposes the LDS latency
// once per k step, and sinks the loads below later MFMAs, which drains the
// ring.
__device__ __forceinline__ void fence_sched() { __builtin_amdgcn_sched_barrier(0); }

// Weight fragments are read through a buffer resource: the base and every
// wave-uniform offset (column block, k block) live in scalar registers and
// the one per-lane offset (lane * 16) in a vector register, so refilling the
// weight ring costs no vector ALU work.  The packed weight is below 2 GiB
// (launch_gemm checks), so 32-bit offsets reach all of it.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t weight_rsrc(const KParams &p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(p.bp), 0, p.wbytes, 0x00020000);
}
__device__ __forceinline__ v4i load_frag(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}

// Tile -> (column slab, row tile).  Workgroups are dealt to the eight XCDs
// round-robin (workgroup w runs on XCD w % 8), so workgroup w takes tile
// (w % 8) * per + w / 8 of a fixed order: each XCD works through one
// contiguous run of it.  Column-slab-major order (row_major = 0) gives each
// XCD a few weight slabs that stay in its L2 while all row tiles pass; it
// suits GEMMs whose weight outweighs the activation.  Row-tile-major order
// gives each XCD a band of activation rows read once, against all slabs.
__device__ __forceinline__ bool tile_of(int w, int tiles_m, int tiles_n, int per, int row_major,
                                        int &bx, int &by) {
    const int t = (w & 7) * per + (w >> 3);
    if (t >= tiles_m * tiles_n) return false;
    if (row_major) {
        by = t / tiles_n;
        bx = t - by * tiles_n;
    } else {
        bx = t / tiles_m;
        by = t - bx * tiles_m;
    }
    return true;
}


}  // namespace

// iro_gemm.hip: the launch parameters common to every GEMM kernel.
int fill_kparams(IroHipContext *ctx, const IroHipWeight *w, const GemmArgs &a, KParams &kp);

// iro_gemm_lds.hip: the LDS-pipelined kernel.  Shapes: 1 192x256, 2 96x128,
// 3 128x256, 4 96x256, 5 64x128 (rows x columns per workgroup).
constexpr int LDS_192x256_CFG = 1, LDS_96x128_CFG = 2;
void lds_tile_shape(int cfg, int *bm, int *bn);
bool lds_cfg_ok(int cfg, bool two, int epi);
void launch_lds(const KParams &kp, int conv, int epi, bool two, int cfg, unsigned grid,
                hipStream_t st);

}  // namespace iro
