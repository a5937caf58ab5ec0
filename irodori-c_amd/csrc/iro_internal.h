// iro_internal.h -- types shared by the gfx950 kernels and the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <vector>

#include "iro_hip.h"

namespace iro {
// Kernel kinds the event profiler accumulates (names in iro_capi.hip).
enum ProfKind {
    PK_QUANT = 0,
    PK_QUANT_RESIDUAL,
    PK_GEMM_LINEAR,
    PK_GEMM_LINEAR_2T,
    PK_GEMM_QKVG,
    PK_GEMM_QKVG_2T,
    PK_GEMM_SWIGLU,
    PK_GEMM_SWIGLU_2T,
    PK_GEMM_GATED,
    PK_GEMM_GATED_2T,
    PK_CONV_ROWS,
    PK_CONV_IM2COL,
    PK_CONVT_GATHER,
    PK_PERSIST_STACK,
    PK_SNAKE,
    PK_GEMM_SWIGLU_Q,
    PK_CONV_GEMM,
    PK_OTHER,
    PK_COUNT
};
struct ProfState;
}  // namespace iro

// Context: one device, one stream, one rounding convention, one growable
// device workspace for the activations the fused entry points stage
// (quantized codes, row scales, the SwiGLU hidden state, im2col rows),
// and an optional per-kernel event profiler.
struct IroHipContext {
    int device = 0;
    int convention = IRO_HIP_STRICT;
    hipStream_t stream = nullptr;
    char err[512] = {0};
    int has_err = 0;
    void *ws = nullptr;
    size_t ws_bytes = 0;
    unsigned ws_epoch = 0;  // bumped whenever ws is reallocated
    // a second workspace for calls composed of other calls (the codec
    // residual unit and decoder): their intermediates live here while the
    // inner calls use ws
    void *ws_outer = nullptr;
    size_t ws_outer_bytes = 0;
    // while set, the inner workspace of the calls being issued (a chain of
    // launches on its own stream, sized beforehand; never grown)
    void *ws_override = nullptr;
    size_t ws_override_bytes = 0;
    char backend[256] = {0};
    int cus = 0;        // compute units of the device
    void *zero16 = nullptr;  // 256 zero bytes: the source of padding k pieces
    int gemm_tile = 0;  // 0: tile shape chosen per GEMM; else 10*TI + TJ
    int tile_order = -1;  // -1: per GEMM; 0 column-slab-major; 1 row-major
    int gemm_ring = 0;    // weight ring depth of the whole-tile kernel (0: default)
    int gemm_spb = 0;     // column slabs per whole-tile block (0: chosen per GEMM)
    int gemm_lds = 0;     // LDS-pipelined GEMM: 0 shape chosen per GEMM, -1 off, > 0 forced shape
    int gemm_wt_rows = 0; // rows per whole-tile block: 0 chosen per GEMM, 64 or 128
    int conv_mode = 2;    // kernel-7 convolutions: 2 the GEMM codes its own rows where
                          // that pays, 3 wherever it can, 1 a one-pass im2col, 0 the
                          // two-pass im2col
    int conv_cols = 0;    // output channels per block of that GEMM: 0 chosen, 128, 256
    int band_quant = 0;   // W1/W3 kernel quantizes the SwiGLU hidden state itself (opt-in)
    // band exchange state of that kernel: zero between launches
    unsigned *band_state = nullptr;
    size_t band_state_bytes = 0;
    int band_occ[2] = {0, 0};  // resident blocks per CU of its two conventions' kernels
    iro::ProfState *prof = nullptr;  // non-null while profiling is on
    float *rope = nullptr;  // rotation table: per position cos[32] then sin[32]
    int rope_S = 0;         // positions held by rope
    int *dev_err = nullptr;  // device error word: kernels OR in a code, iro_hip_sync reports it
    void *noalloc_scratch = nullptr;  // this device's address of the no-alloc scratch
    size_t noalloc_scratch_bytes = 0;
};

// The joined-key layout of one utterance's attention context: per batch b,
// the kept context rows in order (dit.c:815-843).
struct IroHipAttnContext {
    IroHipContext *ctx = nullptr;
    int B = 0, C = 0, context_batch = 0;
    int max_valid = 0;           // largest number of kept context rows of any batch
    int *rows = nullptr;         // [B][C]: source row of joined key S + i (device)
    int *nvalid = nullptr;       // [B]: kept context rows (device)
    std::vector<int> nvalid_h;   // the same, on the host
};

// A quantized weight, pre-packed for the MFMA B operand.
//
// Packed layout: [Np/32][Kp/32] fragments of 1 KiB.  Fragment (nb, kb)
// holds rows nb*32 .. +31 (in packed order) and k = kb*32 .. +31; lane L of
// a wave owns bytes [L*16, L*16+16): row nb*32 + (L & 31), k = kb*32 +
// (L >> 5)*16 .. +15.  A wave therefore loads one fragment with one
// 16-byte read per lane, and a GEMM tile of BN x BK is BN/32 contiguous
// runs of BK/32 fragments.  Rows beyond N and k beyond K are zero.
//
// Packed row order: layout 0 keeps the logical order (parts concatenated);
// layout 1 interleaves two equal parts in 32-row blocks (packed block 2t
// is part 0 block t, 2t+1 is part 1 block t), so an output tile of 64
// columns holds matching W1 and W3 columns.  scale/colsum are stored in
// packed order.
struct IroHipWeight {
    IroHipContext *ctx = nullptr;
    int N = 0, K = 0;    // logical
    int Np = 0, Kp = 0;  // padded to kNPad / kKPad
    int layout = 0;
    int nparts = 1;
    int part_N[8] = {0};
    int8_t *packed = nullptr;
    float *scale = nullptr;
    int32_t *colsum = nullptr;  // as given (used by the epilogue)
    int32_t *rowsum = nullptr;  // true sum of the packed codes of each row;
                                // equals colsum unless a caller supplied an
                                // inconsistent one (ops.c:391 selfcheck does)
    int convention = -1;        // rounding convention the codes were made
                                // under; -1 when the caller supplied them
};

namespace iro {

constexpr int kNPad = 256;  // packed rows padded to a multiple of this
// Packed rows of a weight of N rows: narrow single-part weights (N <= 128,
// the decoder's 96-channel convolutions) pad to 128 rows, which the
// 128-column tiles cover; all others to kNPad.
inline int packed_rows(int N, int layout, int nparts) {
    return (N <= 128 && layout == 0 && nparts == 1)
               ? 128
               : (int)(((size_t)N + kNPad - 1) / kNPad * kNPad);
}
constexpr int kKPad = 128;  // packed k padded to a multiple of this

int set_error(IroHipContext *ctx, const char *fmt, ...);
int noalloc_scratch_init(IroHipContext *ctx);  // iro_dit.hip

#define IRO_HIP_TRY(ctx, expr)                                                        \
    do {                                                                              \
        hipError_t e_ = (expr);                                                       \
        if (e_ != hipSuccess)                                                         \
            return ::iro::set_error((ctx), "%s:%d %s: %s", __FILE__, __LINE__, #expr, \
                                    hipGetErrorString(e_));                           \
    } while (0)

#define IRO_HIP_CHECK_LAUNCH(ctx) IRO_HIP_TRY(ctx, hipGetLastError())

// Event pair around one launch when the context profiler is on; `ops` and
// `bytes` are the launch's algorithmic work (multiply-adds x2, HBM bytes).
void prof_begin(IroHipContext *ctx);
void prof_end(IroHipContext *ctx, ProfKind kind, double ops, double bytes);

// Bump allocation from the context workspace; grows it (after draining the
// stream) when a call needs more.  Offsets are 256-byte aligned.
struct Workspace {
    IroHipContext *ctx;
    int outer = 0;  // 1: the context's outer workspace
    size_t need = 0;
    size_t reserve(size_t bytes) {
        size_t off = need;
        need += (bytes + 255) & ~size_t(255);
        return off;
    }
    int commit();  // ensures ctx->ws holds `need` bytes
    template <class T>
    T *at(size_t off) const {
        return reinterpret_cast<T *>(
            static_cast<char *>(outer ? ctx->ws_outer : ctx->ws_override ? ctx->ws_override : ctx->ws) +
            off);
    }
};

// ---- kernel launchers (iro_quant.hip, iro_gemm.hip, iro_conv.hip) -------

// Input rows of a kernel-7 Conv1d for the GEMM that codes them itself
// (iro_conv_gemm.hip): x [T, C] and each row's lo/hi over channels.
struct ConvRows {
    const float *x;
    const float *row_lo, *row_hi;
    int T, C, stride, dilation, padding;
};
bool conv7_gemm_ok(const IroHipWeight *w, const ConvRows &cr);
bool conv7_gemm_pays(const ConvRows &cr, int T_out);
// A decoder residual unit's 1x1 with its in-place snake_bias and row
// quantization in one kernel (C % 32 == 0, 64 <= C <= 192, two planes up to
// 160); returns 1
// (nothing launched) for other shapes.
int launch_conv1x1_snake(IroHipContext *ctx, const IroHipWeight *w, const float *hidden, int T,
                         const float *snake_bias, const float *snake_alpha, bool two,
                         const float *bias, const float *skip, float *output);
// iro_codec.hip: snake (reciprocal form) of x into y with each row's lo/hi.
bool snake_rows_ok(const float *x, int C, const float *y);
int launch_snake_rows(IroHipContext *ctx, const float *x, int T, int C, const float *alpha,
                      float *y, float *row_lo, float *row_hi);
// iro_capi.hip: iro_hip_conv1d_int8, optionally with the snake of
// snake_alpha applied to the input rows first (into snake_out, [T, C]), as
// conv1d_int8_forward does with a snake (dacvae.c:599-603).
int conv1d_int8(IroHipContext *ctx, const float *input, int T, int C, const IroHipWeight *w,
                int kernel, int stride, int dilation, int padding, const float *bias,
                int residual, float *output, int *t_out, const float *snake_alpha,
                float *snake_out);
// iro_hip_convtranspose1d_int8 likewise: with snake_alpha the input rows'
// snake (iro_snake_forward, dacvae.c:830-857) runs inside the row
// quantizer where it takes the shape, else into snake_out first.
int convtranspose1d_int8(IroHipContext *ctx, const float *input, int T_in, int C_in,
                         const IroHipWeight *w, int C_out, int kernel, int stride, int padding,
                         int output_padding, const float *bias, int residual, float *output,
                         int *t_out, const float *snake_alpha, float *snake_out);
// Returns 1 (nothing launched) when conv7_gemm_ok refuses the shape.
int launch_conv7_gemm(IroHipContext *ctx, const IroHipWeight *w, const ConvRows &cr, int T_out,
                      bool two, const float *bias, float *y);

// Snake applied to each element before it is quantized: x + bias[c] (x as
// it is when bias is null), then the reciprocal-form snake with alpha[c]
// (the in-place snake_bias of a residual unit, or the snake before an
// upsample; at most 1536 channels).
struct SnakePre {
    const float *bias;
    const float *alpha;
};
// With `snake`, returns 1 (nothing launched) for shapes the fused path does
// not take; the caller then runs the snake as its own pass.
int launch_quant_rows(IroHipContext *ctx, const float *x, int M, int K, int ldx, uint8_t *q1,
                      int ldq, float *s1, int32_t *z1, float *res, uint8_t *q2, float *s2,
                      int32_t *z2, bool signed_codes = false, const SnakePre *snake = nullptr);
int launch_weight_quant(IroHipContext *ctx, const float *w, int N, int K, long long stride_n,
                        long long stride_k, int8_t *q, float *scale, int32_t *colsum);
int launch_pack(IroHipContext *ctx, const int8_t *q, const float *scale, const int32_t *colsum,
                const int32_t *rowsum, IroHipWeight *w);
int launch_fill(IroHipContext *ctx, void *dst, int value, size_t bytes);
int launch_codes_selfcheck(IroHipContext *ctx, unsigned long long *out);
// iro_engine.hip: x = silu(x) [* g] (ops.c:776-784) and x += gate[m / S] * branch.
int launch_silu(IroHipContext *ctx, float *x, const float *g, long long n);
int launch_gated_residual(IroHipContext *ctx, float *x, const float *gate, int ldg,
                          const float *branch, int M, int D, int S);

// A zeroed layout-0 weight of N x K, and a copy of a whole layout-0 weight
// into its rows row0 .. row0 + src->Np (row0 a multiple of 32): several
// weights that share one activation become one GEMM.
// The packed buffers of a weight of logical N x K (contents undefined).
int weight_alloc(IroHipContext *ctx, int N, int K, int layout, int nparts, const int *parts_N,
                 bool separate_rowsum, IroHipWeight **out);
int weight_rows_alloc(IroHipContext *ctx, int N, int K, IroHipWeight **out);
int weight_rows_copy(IroHipContext *ctx, IroHipWeight *dst, int row0, const IroHipWeight *src);

enum Epi { EPI_LINEAR = 0, EPI_QKVG = 1, EPI_SWIGLU = 2, EPI_GATED = 3 };

struct GemmArgs {
    const uint8_t *a1 = nullptr;  // u8 codes [M, lda] (plane 1)
    const uint8_t *a2 = nullptr;  // plane 2, nullptr for one plane
    int lda = 0;
    const float *sx1 = nullptr, *sx2 = nullptr;
    const int32_t *zx1 = nullptr, *zx2 = nullptr;
    int M = 0;
    int K = 0;  // k extent read from A (multiple of 16, <= w->Kp)
    const float *bias = nullptr;
    float *y = nullptr;  // EPI_LINEAR output [M, ldy]
    // accumulate: y = yin + ... with yin [M, ldy] the prior rows (the same
    // buffer as y, or one that does not overlap it); nullptr = y itself.
    const float *yin = nullptr;
    int ldy = 0;
    int32_t *work = nullptr;  // raw plane-1 sums [M, ldw], nullable
    int ldw = 0;
    int accumulate = 0;
    float *seg[4] = {nullptr, nullptr, nullptr, nullptr};  // EPI_QKVG
    int seg_n = 0;
    float *hidden = nullptr;  // EPI_SWIGLU [M, ldh]
    int ldh = 0;
    float *xres = nullptr;  // EPI_GATED [M, ldx]
    const float *gate = nullptr;  // [M / rows_per_branch, ldg]
    int ldg = 0;
    int ldx = 0;
    int rows_per_branch = 1;
    int a_signed = 0;  // codes already stored as a ^ 0x80 (quantize_into)
    int a_kbp = 0;     // > 0: codes in the MFMA fragment layout with a_kbp k blocks
                       // per 32-row block (LDS-pipelined kernel only)
    // EPI_SWIGLU only: when hq1 is set the kernel quantizes the hidden state
    // itself (one plane, two with hq2) into these row-major signed codes
    // instead of storing it; launch_gemm returns 1, launching nothing, when
    // the GEMM's shape does not allow that.
    uint8_t *hq1 = nullptr, *hq2 = nullptr;
    int ldhq = 0;
    float *hs1 = nullptr, *hs2 = nullptr;
    int32_t *hz1 = nullptr, *hz2 = nullptr;
};

int launch_gemm(IroHipContext *ctx, const IroHipWeight *w, const GemmArgs &a, Epi epi);
// The LDS-pipelined kernel's shape a GEMM of M rows and k extent K with
// signed codes would take, or 0 when it takes another kernel.
int gemm_lds_cfg(const IroHipContext *ctx, Epi epi, bool two, int M, int K, int N = 0);
int launch_silu_selfcheck(IroHipContext *ctx, unsigned long long *out);
int launch_fp32_selfcheck(IroHipContext *ctx, unsigned long long *out);

inline size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }

// Activation staging in the context workspace: codes in rows padded to 16
// bytes (the GEMM reads A in 16-byte chunks), or, for the LDS-pipelined
// kernel, in the MFMA fragment layout (ld < 0: -ld k blocks per 32-row
// block, rows padded to 32); row scales and zero points, and the second
// plane when the two-term residual quantization is on.
struct ActBufs {
    uint8_t *q1, *q2;
    float *s1, *s2;
    int32_t *z1, *z2;
    int ld;
};

inline size_t act_code_bytes(int M, int K, bool packed) {
    return packed ? round_up((size_t)M, 32) * (size_t)K : round_up((size_t)K, 16) * M;
}

inline void act_reserve(Workspace &ws, int M, int K, bool two, size_t off[6], bool packed = false) {
    const size_t cb = act_code_bytes(M, K, packed);
    off[0] = ws.reserve(cb);
    off[1] = ws.reserve(sizeof(float) * M);
    off[2] = ws.reserve(sizeof(int32_t) * M);
    off[3] = two ? ws.reserve(cb) : 0;
    off[4] = two ? ws.reserve(sizeof(float) * M) : 0;
    off[5] = two ? ws.reserve(sizeof(int32_t) * M) : 0;
}

inline ActBufs act_at(const Workspace &ws, int K, bool two, const size_t off[6],
                      bool packed = false) {
    ActBufs b;
    b.ld = packed ? -(K / 32) : (int)round_up((size_t)K, 16);
    b.q1 = ws.at<uint8_t>(off[0]);
    b.s1 = ws.at<float>(off[1]);
    b.z1 = ws.at<int32_t>(off[2]);
    b.q2 = two ? ws.at<uint8_t>(off[3]) : nullptr;
    b.s2 = two ? ws.at<float>(off[4]) : nullptr;
    b.z2 = two ? ws.at<int32_t>(off[5]) : nullptr;
    return b;
}

inline int quantize_into(IroHipContext *ctx, const float *x, int M, int K, int ldx,
                         const ActBufs &b) {
    return launch_quant_rows(ctx, x, M, K, ldx, b.q1, b.ld, b.s1, b.z1, nullptr, b.q2, b.s2,
                             b.z2, true);
}

inline GemmArgs gemm_args(const ActBufs &b, int M, int K) {
    GemmArgs a;
    a.a1 = b.q1;
    a.a2 = b.q2;
    a.lda = b.ld;
    a.sx1 = b.s1;
    a.zx1 = b.z1;
    a.sx2 = b.s2;
    a.zx2 = b.z2;
    a.M = M;
    a.K = (int)round_up((size_t)K, 16);
    a.a_signed = 1;
    if (b.ld < 0) {
        a.lda = K;
        a.a_kbp = -b.ld;
    }
    return a;
}

// The persistent stack kernel (iro_persist.hip).
struct PersistPlan;
bool persist_supported(int D, int H, int residual_mask);
int persist_prepare(IroHipContext *ctx, PersistPlan **plan, int M, int D, int H, int S, int blocks,
                    int two_w2, const IroHipWeight *const *weights, float *q, float *k, float *v,
                    float *g, float *hidden, const float *mod, int ldm, int ada_np);
int persist_launch(IroHipContext *ctx, PersistPlan *plan, float *x);
void persist_free(PersistPlan *plan);

int launch_conv_rows(IroHipContext *ctx, const float *x, int T, int C, float *lo, float *hi);
// Kernel 7, C % 4 == 0, C <= 1024: window ranges and codes in one pass.
bool conv_im2col7_ok(int C, int kernel, int ldc);
int launch_conv_im2col7(IroHipContext *ctx, const float *x, int T, int C, int T_out, int stride,
                        int dilation, int padding, uint8_t *cols1, uint8_t *cols2, int ldc,
                        float *s1, int32_t *z1, float *s2, int32_t *z2, bool signed_codes);
int launch_convt_gather(IroHipContext *ctx, const float *expanded, int T_in, int C_out,
                        int kernel, int stride, int padding, int T_out, const float *bias,
                        float *y);
int launch_conv_im2col(IroHipContext *ctx, const float *x, int T, int C, int T_out, int kernel,
                       int stride, int dilation, int padding, const float *row_lo,
                       const float *row_hi, uint8_t *cols1, uint8_t *cols2, int ldc, float *s1,
                       int32_t *z1, float *s2, int32_t *z2);

}  // namespace iro
