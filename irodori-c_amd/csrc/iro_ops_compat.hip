// iro_ops_compat.hip -- the reference's host-pointer int8 API (ops.h:18-78,
// ops.c:257-491) served by the MI355X kernels through a process-wide
// default context.  Declared in include/iro_int8_ops.h.
//
// Weights quantized here keep the reference's host arrays (callers and
// tests read data/scale/colsum) and a pre-packed device copy, found again
// by the address of `data` until iro_int8_weight_free.  A weight struct
// built by hand (as ops.c:391 does) is packed for the one call.
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <unordered_map>

#include "iro_int8_ops.h"
#include "iro_internal.h"

namespace {

std::mutex g_mu;
IroHipContext *g_ctx = nullptr;
int g_init_failed = 0;
int g_error = 0;

struct Entry {
    IroHipWeight *w;
    const float *scale;
    const int32_t *colsum;
    int N, K;
};
std::unordered_map<const int8_t *, Entry> g_weights;

int env_convention() {
    const char *e = getenv("IRO_HIP_CONVENTION");
    if (e && (!strcmp(e, "fastmath") || !strcmp(e, "fast") || !strcmp(e, "1")))
        return IRO_HIP_GCC_FASTMATH;
    return IRO_HIP_STRICT;
}

IroHipContext *ctx_locked() {
    if (!g_ctx && !g_init_failed) {
        if (iro_hip_create(0, env_convention(), &g_ctx) != 0) {
            g_ctx = nullptr;
            g_init_failed = 1;
        }
    }
    return g_ctx;
}

// Device scratch for one call, freed at scope exit.
struct DevBuf {
    IroHipContext *ctx;
    void *p = nullptr;
    explicit DevBuf(IroHipContext *c) : ctx(c) {}
    ~DevBuf() {
        if (p) iro_hip_free(ctx, p);
    }
    template <class T>
    T *get(size_t bytes) {
        if (iro_hip_alloc(ctx, bytes, &p)) return nullptr;
        return static_cast<T *>(p);
    }
};

int fail() {
    g_error = 1;
    return -1;
}

int quantize_common(IroInt8Weight *dst, const float *w, int N, int K, bool transposed) {
    if (!dst || !w || N <= 0 || K <= 0) return -1;
    memset(dst, 0, sizeof(*dst));
    std::lock_guard<std::mutex> lock(g_mu);
    IroHipContext *ctx = ctx_locked();
    if (!ctx) return fail();
    DevBuf src(ctx);
    float *wd = src.get<float>(sizeof(float) * (size_t)N * K);
    if (!wd || iro_hip_upload(ctx, wd, w, sizeof(float) * (size_t)N * K)) return fail();
    IroHipWeight *hw = nullptr;
    const int rc = transposed ? iro_hip_weight_create_transposed(ctx, wd, N, K, &hw)
                              : iro_hip_weight_create(ctx, wd, N, K, &hw);
    if (rc) return fail();
    dst->data = (int8_t *)malloc((size_t)N * K);
    dst->scale = (float *)malloc(sizeof(float) * (size_t)N);
    dst->colsum = (int32_t *)malloc(sizeof(int32_t) * (size_t)N);
    if (!dst->data || !dst->scale || !dst->colsum ||
        iro_hip_weight_export(ctx, hw, dst->data, dst->scale, dst->colsum)) {
        free(dst->data);
        free(dst->scale);
        free(dst->colsum);
        memset(dst, 0, sizeof(*dst));
        iro_hip_weight_destroy(hw);
        return fail();
    }
    dst->N = N;
    dst->K = K;
    g_weights[dst->data] = Entry{hw, dst->scale, dst->colsum, N, K};
    return 0;
}

}  // namespace

extern "C" {

int iro_int8_weight_quantize(IroInt8Weight *dst, const float *w, int N, int K) {
    return quantize_common(dst, w, N, K, false);
}

int iro_int8_weight_quantize_transposed(IroInt8Weight *dst, const float *w, int N, int K) {
    return quantize_common(dst, w, N, K, true);
}

void iro_int8_weight_free(IroInt8Weight *w) {
    if (!w) return;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        auto it = g_weights.find(w->data);
        if (it != g_weights.end()) {
            iro_hip_weight_destroy(it->second.w);
            g_weights.erase(it);
        }
    }
    free(w->data);
    free(w->scale);
    free(w->colsum);
    memset(w, 0, sizeof(*w));
}

size_t iro_int8_weight_bytes(const IroInt8Weight *w) {
    if (!w || !w->data) return 0;
    return (size_t)w->N * w->K + (size_t)w->N * (sizeof(float) + sizeof(int32_t));
}

void iro_int8_quantize_rows(const float *x, int M, int K, uint8_t *q, float *scale,
                            int32_t *zero) {
    if (M <= 0 || K <= 0) return;
    std::lock_guard<std::mutex> lock(g_mu);
    IroHipContext *ctx = ctx_locked();
    if (!ctx) {
        fail();
        return;
    }
    const size_t xb = sizeof(float) * (size_t)M * K, qb = (size_t)M * K;
    DevBuf buf(ctx);
    char *p = buf.get<char>(xb + qb + 8 * (size_t)M + 1024);
    if (!p) {
        fail();
        return;
    }
    float *xd = (float *)p;
    uint8_t *qd = (uint8_t *)(p + ((xb + 255) & ~size_t(255)));
    float *sd = (float *)((char *)qd + ((qb + 255) & ~size_t(255)));
    int32_t *zd = (int32_t *)((char *)sd + ((4 * (size_t)M + 255) & ~size_t(255)));
    if (iro_hip_upload(ctx, xd, x, xb) || iro_hip_quantize_rows(ctx, xd, M, K, qd, sd, zd) ||
        iro_hip_download(ctx, q, qd, qb) || iro_hip_download(ctx, scale, sd, 4 * (size_t)M) ||
        iro_hip_download(ctx, zero, zd, 4 * (size_t)M))
        fail();
}

void iro_int8_quantize_rows_residual(const float *x, int M, int K, uint8_t *q1, float *scale1,
                                     int32_t *zero1, float *residual, uint8_t *q2,
                                     float *scale2, int32_t *zero2) {
    if (M <= 0 || K <= 0) return;
    std::lock_guard<std::mutex> lock(g_mu);
    IroHipContext *ctx = ctx_locked();
    if (!ctx) {
        fail();
        return;
    }
    const size_t xb = sizeof(float) * (size_t)M * K, qb = (size_t)M * K;
    const size_t xa = (xb + 255) & ~size_t(255), qa = (qb + 255) & ~size_t(255);
    const size_t va = (4 * (size_t)M + 255) & ~size_t(255);
    DevBuf buf(ctx);
    char *p = buf.get<char>(2 * xa + 2 * qa + 4 * va);
    if (!p) {
        fail();
        return;
    }
    float *xd = (float *)p;
    float *rd = (float *)(p + xa);
    uint8_t *q1d = (uint8_t *)(p + 2 * xa);
    uint8_t *q2d = q1d + qa;
    float *s1d = (float *)(p + 2 * xa + 2 * qa);
    int32_t *z1d = (int32_t *)((char *)s1d + va);
    float *s2d = (float *)((char *)s1d + 2 * va);
    int32_t *z2d = (int32_t *)((char *)s1d + 3 * va);
    if (iro_hip_upload(ctx, xd, x, xb) ||
        iro_hip_quantize_rows_residual(ctx, xd, M, K, q1d, s1d, z1d, rd, q2d, s2d, z2d) ||
        iro_hip_download(ctx, q1, q1d, qb) || iro_hip_download(ctx, scale1, s1d, 4 * (size_t)M) ||
        iro_hip_download(ctx, zero1, z1d, 4 * (size_t)M) ||
        (residual && iro_hip_download(ctx, residual, rd, xb)) ||
        iro_hip_download(ctx, q2, q2d, qb) || iro_hip_download(ctx, scale2, s2d, 4 * (size_t)M) ||
        iro_hip_download(ctx, zero2, z2d, 4 * (size_t)M))
        fail();
}

void iro_int8_linear_ex(const uint8_t *q, const float *scale, const int32_t *zero,
                        const IroInt8Weight *w, const float *bias, float *y, int M,
                        int32_t *work, int accumulate) {
    if (!w || M <= 0) return;
    const int N = w->N, K = w->K;
    std::lock_guard<std::mutex> lock(g_mu);
    IroHipContext *ctx = ctx_locked();
    if (!ctx) {
        fail();
        return;
    }
    IroHipWeight *hw = nullptr;
    bool temp = false;
    auto it = g_weights.find(w->data);
    if (it != g_weights.end() && it->second.scale == w->scale && it->second.colsum == w->colsum &&
        it->second.N == N && it->second.K == K) {
        hw = it->second.w;
    } else {
        if (iro_hip_weight_from_host(ctx, w->data, w->scale, w->colsum, N, K, &hw)) {
            fail();
            return;
        }
        temp = true;
    }
    auto al = [](size_t b) { return (b + 255) & ~size_t(255); };
    const size_t qb = al((size_t)M * K), vb = al(4 * (size_t)M), yb = al(4 * (size_t)M * N),
                 bb = al(4 * (size_t)N);
    DevBuf buf(ctx);
    char *p = buf.get<char>(qb + 2 * vb + 2 * yb + bb);
    int rc = p ? 0 : -1;
    if (!rc) {
        uint8_t *qd = (uint8_t *)p;
        float *sd = (float *)(p + qb);
        int32_t *zd = (int32_t *)(p + qb + vb);
        float *yd = (float *)(p + qb + 2 * vb);
        int32_t *wd = (int32_t *)(p + qb + 2 * vb + yb);
        float *bd = bias ? (float *)(p + qb + 2 * vb + 2 * yb) : nullptr;
        rc = iro_hip_upload(ctx, qd, q, (size_t)M * K) ||
             iro_hip_upload(ctx, sd, scale, 4 * (size_t)M) ||
             iro_hip_upload(ctx, zd, zero, 4 * (size_t)M) ||
             (bias && iro_hip_upload(ctx, bd, bias, 4 * (size_t)N)) ||
             (accumulate && iro_hip_upload(ctx, yd, y, 4 * (size_t)M * N)) ||
             iro_hip_int8_linear_ex(ctx, qd, sd, zd, hw, bd, yd, M, work ? wd : nullptr,
                                    accumulate) ||
             iro_hip_download(ctx, y, yd, 4 * (size_t)M * N) ||
             (work && iro_hip_download(ctx, work, wd, 4 * (size_t)M * N));
    }
    if (temp) iro_hip_weight_destroy(hw);
    if (rc) fail();
}

void iro_int8_linear(const uint8_t *q, const float *scale, const int32_t *zero,
                     const IroInt8Weight *w, const float *bias, float *y, int M, int32_t *work) {
    iro_int8_linear_ex(q, scale, zero, w, bias, y, M, work, 0);
}

int iro_int8_fast_available(void) { return 1; }

const char *iro_int8_prepare_backend(void) {
    std::lock_guard<std::mutex> lock(g_mu);
    IroHipContext *ctx = ctx_locked();
    return ctx ? iro_hip_backend_name(ctx) : nullptr;
}

int iro_int8_selfcheck(void) {
    std::lock_guard<std::mutex> lock(g_mu);
    IroHipContext *ctx = ctx_locked();
    if (!ctx) return -1;
    return iro_hip_selfcheck(ctx) == 0 ? 0 : -1;
}

int iro_int8_last_error(void) { return g_error; }

}  // extern "C"
