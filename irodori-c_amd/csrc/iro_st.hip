// iro_st.hip -- the weight source: safetensors checkpoints read through a
// read-only mmap (the file format of safetensors.c:1-7: an 8-byte
// little-endian header length, a JSON header naming every tensor's dtype,
// shape and byte range, then the data), int8 weights built straight from
// their tensors, and the packed int8 weight as a file of its own so a
// restart can skip quantization.
//
// Host code only.  The checkpoint API needs no device: it can open and
// inspect files on a machine without a GPU.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "iro_internal.h"

// ---- checkpoint -------------------------------------------------------------

struct IroHipSafetensors {
    struct Tensor {
        std::string name;
        int dtype = 0;
        int ndims = 0;
        uint64_t shape[8] = {0};
        uint64_t begin = 0, nbytes = 0;
    };
    int fd = -1;
    uint8_t *map = nullptr;
    size_t map_size = 0;
    uint64_t data_start = 0;
    std::vector<Tensor> tensors;
    std::vector<std::pair<std::string, std::string>> meta;
};

namespace {

thread_local char st_err[512];

int st_fail(const char *fmt, const char *a = "", unsigned long long v = 0) {
    std::snprintf(st_err, sizeof(st_err), fmt, a, v);
    return -1;
}

// dtype names in IroDType order (irodori.h:15-26) and their item sizes.
const char *const kDtypeName[] = {"F32", "F16", "BF16", "I64", "I32", "I16", "I8", "U8", "BOOL"};
const int kDtypeSize[] = {4, 2, 2, 8, 4, 2, 1, 1, 1};

// A JSON reader for the header's grammar: the root object maps names to
// tensor objects ({"dtype": string, "shape": [int...], "data_offsets":
// [int, int]}, other members ignored) and "__metadata__" to an object of
// strings.  Strings are kept as the raw bytes between their quotes (escape
// sequences are checked, not decoded), as safetensors.c's tokenizer keeps
// them, so a metadata value is its JSON text.
struct Json {
    const char *s;
    size_t n, i = 0;
    void ws() {
        while (i < n && (s[i] == ' ' || s[i] == '\t' || s[i] == '\n' || s[i] == '\r')) ++i;
    }
    bool eat(char c) {
        ws();
        if (i < n && s[i] == c) {
            ++i;
            return true;
        }
        return false;
    }
    // Escapes are validated as JSON defines them (\" \\ \/ \b \f \n \r \t
    // and \u with four hex digits) and kept undecoded.
    bool str(std::string &out) {
        ws();
        if (i >= n || s[i] != '"') return false;
        const size_t b = ++i;
        while (i < n && s[i] != '"') {
            if (s[i] == '\\') {
                if (++i >= n) return false;
                const char e = s[i];
                if (e == 'u') {
                    for (int k = 1; k <= 4; ++k) {
                        const char h = i + k < n ? s[i + k] : 0;
                        if (!((h >= '0' && h <= '9') || (h >= 'a' && h <= 'f') ||
                              (h >= 'A' && h <= 'F')))
                            return false;
                    }
                    i += 4;
                } else if (!std::strchr("\"\\/bfnrt", e) || !e) {
                    return false;
                }
            }
            ++i;
        }
        if (i >= n) return false;
        out.assign(s + b, i - b);
        ++i;
        return true;
    }
    bool integer(long long &v) {
        ws();
        const size_t b = i;
        if (i < n && s[i] == '-') ++i;
        if (i >= n || s[i] < '0' || s[i] > '9') return false;
        unsigned long long u = 0;
        while (i < n && s[i] >= '0' && s[i] <= '9') {
            if (u > (~0ull - 9) / 10) return false;
            u = u * 10 + (unsigned)(s[i++] - '0');
        }
        if (u > (unsigned long long)INT64_MAX) return false;
        v = s[b] == '-' ? -(long long)u : (long long)u;
        return true;
    }
    // Any value, skipped (depth-limited).
    bool skip(int depth = 0) {
        ws();
        if (i >= n || depth > 64) return false;
        const char c = s[i];
        if (c == '"') {
            std::string t;
            return str(t);
        }
        if (c == '{' || c == '[') {
            const char close = c == '{' ? '}' : ']';
            ++i;
            if (eat(close)) return true;
            for (;;) {
                if (c == '{') {
                    std::string k;
                    if (!str(k) || !eat(':')) return false;
                }
                if (!skip(depth + 1)) return false;
                if (eat(close)) return true;
                if (!eat(',')) return false;
            }
        }
        // number, true, false, null
        const size_t b = i;
        while (i < n && s[i] != ',' && s[i] != '}' && s[i] != ']' && s[i] != ' ' &&
               s[i] != '\n' && s[i] != '\r' && s[i] != '\t')
            ++i;
        return i > b;
    }
    bool int_array(std::vector<long long> &out, size_t max) {
        if (!eat('[')) return false;
        if (eat(']')) return true;
        for (;;) {
            long long v;
            if (out.size() >= max || !integer(v)) return false;
            out.push_back(v);
            if (eat(']')) return true;
            if (!eat(',')) return false;
        }
    }
};

int dtype_code(const std::string &t) {
    for (int d = 0; d < 9; ++d)
        if (t == kDtypeName[d]) return d;
    return -1;
}

// One tensor entry; false if malformed.
bool parse_tensor(Json &j, IroHipSafetensors::Tensor &t, uint64_t data_bytes) {
    if (!j.eat('{')) return false;
    bool have_dtype = false, have_shape = false, have_off = false;
    std::vector<long long> shape, off;
    if (!j.eat('}')) {
        for (;;) {
            std::string key;
            if (!j.str(key) || !j.eat(':')) return false;
            if (key == "dtype") {
                std::string v;
                if (!j.str(v) || (t.dtype = dtype_code(v)) < 0) return false;
                have_dtype = true;
            } else if (key == "shape") {
                if (!j.int_array(shape, 8)) return false;
                have_shape = true;
            } else if (key == "data_offsets") {
                if (!j.int_array(off, 2) || off.size() != 2) return false;
                have_off = true;
            } else if (!j.skip()) {
                return false;
            }
            if (j.eat('}')) break;
            if (!j.eat(',')) return false;
        }
    }
    if (!have_dtype || !have_shape || !have_off) return false;
    t.ndims = (int)shape.size();
    unsigned long long numel = 1;
    for (int d = 0; d < t.ndims; ++d) {
        if (shape[d] < 0) return false;
        t.shape[d] = (uint64_t)shape[d];
        if (shape[d] == 0) {
            numel = 0;
        } else if (numel) {
            if (numel > ~0ull / (unsigned long long)shape[d]) return false;
            numel *= (unsigned long long)shape[d];
        }
    }
    if (off[0] < 0 || off[1] < off[0] || (uint64_t)off[1] > data_bytes) return false;
    t.begin = (uint64_t)off[0];
    t.nbytes = (uint64_t)(off[1] - off[0]);
    const unsigned long long isz = (unsigned long long)kDtypeSize[t.dtype];
    return numel <= ~0ull / isz && numel * isz == t.nbytes;
}

bool parse_meta(Json &j, IroHipSafetensors &st) {
    if (!j.eat('{')) return false;
    if (j.eat('}')) return true;
    for (;;) {
        std::string k, v;
        if (!j.str(k) || !j.eat(':') || !j.str(v)) return false;
        st.meta.emplace_back(k, v);
        if (j.eat('}')) return true;
        if (!j.eat(',')) return false;
    }
}

void st_release(IroHipSafetensors *st) {
    if (!st) return;
    if (st->map) munmap(st->map, st->map_size);
    if (st->fd >= 0) close(st->fd);
    delete st;
}

}  // namespace

extern "C" {

const char *iro_hip_st_last_error(void) { return st_err; }

int iro_hip_st_open(const char *path, IroHipSafetensors **out) {
    st_err[0] = 0;
    if (!path || !out) return st_fail("st_open: invalid arguments%s", "");
    *out = nullptr;
    IroHipSafetensors *st = new (std::nothrow) IroHipSafetensors();
    if (!st) return st_fail("st_open: out of host memory%s", "");
    st->fd = open(path, O_RDONLY);
    struct stat sb;
    if (st->fd < 0 || fstat(st->fd, &sb) != 0) {
        st_release(st);
        return st_fail("st_open: cannot open %s", path);
    }
    if (sb.st_size < 10) {
        st_release(st);
        return st_fail("st_open: %s is too small for a safetensors file", path);
    }
    st->map_size = (size_t)sb.st_size;
    void *m = mmap(nullptr, st->map_size, PROT_READ, MAP_PRIVATE, st->fd, 0);
    if (m == MAP_FAILED) {
        st_release(st);
        return st_fail("st_open: mmap of %s failed", path);
    }
    st->map = static_cast<uint8_t *>(m);
    uint64_t hlen = 0;
    for (int i = 0; i < 8; ++i) hlen |= (uint64_t)st->map[i] << (8 * i);
    if (hlen == 0 || hlen > st->map_size - 8) {
        st_release(st);
        return st_fail("st_open: header length %s%llu does not fit the file", "",
                       (unsigned long long)hlen);
    }
    st->data_start = 8 + hlen;
    const uint64_t data_bytes = st->map_size - st->data_start;
    Json j{reinterpret_cast<const char *>(st->map + 8), (size_t)hlen};
    bool ok = j.eat('{');
    if (ok && !j.eat('}')) {
        for (;;) {
            std::string name;
            if (!j.str(name) || !j.eat(':')) {
                ok = false;
                break;
            }
            if (name == "__metadata__") {
                ok = parse_meta(j, *st);
            } else {
                IroHipSafetensors::Tensor t;
                t.name = name;
                ok = parse_tensor(j, t, data_bytes);
                if (ok) st->tensors.push_back(t);
            }
            if (!ok) break;
            if (j.eat('}')) break;
            if (!j.eat(',')) {
                ok = false;
                break;
            }
        }
    }
    if (ok) {
        j.ws();
        ok = j.i == j.n;
    }
    if (!ok) {
        const unsigned long long at = j.i;
        st_release(st);
        return st_fail("st_open: malformed header in %s near byte %llu", path, at);
    }
    *out = st;
    return 0;
}

void iro_hip_st_close(IroHipSafetensors *st) { st_release(st); }

int iro_hip_st_count(const IroHipSafetensors *st) { return st ? (int)st->tensors.size() : 0; }

const char *iro_hip_st_name(const IroHipSafetensors *st, int i) {
    return st && i >= 0 && i < (int)st->tensors.size() ? st->tensors[i].name.c_str() : nullptr;
}

int iro_hip_st_tensor(const IroHipSafetensors *st, const char *name, int *dtype, int *ndims,
                      uint64_t *shape, const void **data, uint64_t *nbytes) {
    if (!st || !name) return -1;
    for (const auto &t : st->tensors) {
        if (t.name != name) continue;
        if (dtype) *dtype = t.dtype;
        if (ndims) *ndims = t.ndims;
        if (shape)
            for (int d = 0; d < 8; ++d) shape[d] = d < t.ndims ? t.shape[d] : 0;
        if (data) *data = st->map + st->data_start + t.begin;
        if (nbytes) *nbytes = t.nbytes;
        return 0;
    }
    return st_fail("st_tensor: no tensor named %s", name);
}

const char *iro_hip_st_meta(const IroHipSafetensors *st, const char *key) {
    if (!st || !key) return nullptr;
    for (const auto &kv : st->meta)
        if (kv.first == key) return kv.second.c_str();
    return nullptr;
}

}  // extern "C"

// ---- weights from a checkpoint ---------------------------------------------

namespace {

// Exact widening of the 16-bit float formats to fp32.
float bf16_to_f32(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 31, m = h & 1023, u;
    if (e == 31) {
        u = sign | 0x7F800000u | (m << 13);  // inf / NaN
    } else if (e) {
        u = sign | ((e + 112) << 23) | (m << 13);
    } else if (!m) {
        u = sign;
    } else {  // subnormal: normalize
        int sh = 0;
        while (!(m & 1024)) {
            m <<= 1;
            ++sh;
        }
        u = sign | ((uint32_t)(113 - sh) << 23) | ((m & 1023) << 13);
    }
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

}  // namespace

using namespace iro;

extern "C" {

int iro_hip_weight_from_st(IroHipContext *ctx, const IroHipSafetensors *st, const char *name,
                           int transposed, IroHipWeight **out) {
    if (!ctx || !st || !name || !out) return set_error(ctx, "weight_from_st: invalid arguments");
    int dtype = 0, nd = 0;
    uint64_t shape[8];
    const void *data = nullptr;
    uint64_t nbytes = 0;
    if (iro_hip_st_tensor(st, name, &dtype, &nd, shape, &data, &nbytes))
        return set_error(ctx, "weight_from_st: %s", st_err);
    if (nd != 2 || shape[0] == 0 || shape[1] == 0 || shape[0] > (1u << 30) || shape[1] > (1u << 30))
        return set_error(ctx, "weight_from_st: %s is not a non-empty 2-D tensor", name);
    if (dtype != 0 && dtype != 1 && dtype != 2)
        return set_error(ctx, "weight_from_st: %s has dtype %s, not F32/F16/BF16", name,
                         kDtypeName[dtype]);
    const size_t numel = (size_t)shape[0] * shape[1];
    std::vector<float> widened;
    const float *src = static_cast<const float *>(data);
    if (dtype != 0) {
        widened.resize(numel);
        const uint16_t *h = static_cast<const uint16_t *>(data);
        for (size_t i = 0; i < numel; ++i)
            widened[i] = dtype == 2 ? bf16_to_f32(h[i]) : f16_to_f32(h[i]);
        src = widened.data();
    }
    void *dev = nullptr;
    if (iro_hip_alloc(ctx, numel * sizeof(float), &dev)) return -1;
    int rc = iro_hip_upload(ctx, dev, src, numel * sizeof(float));
    // [N, K] rows are output rows; a transposed source is [K, N].
    const int N = (int)(transposed ? shape[1] : shape[0]);
    const int K = (int)(transposed ? shape[0] : shape[1]);
    if (!rc)
        rc = transposed ? iro_hip_weight_create_transposed(ctx, static_cast<float *>(dev), N, K, out)
                        : iro_hip_weight_create(ctx, static_cast<float *>(dev), N, K, out);
    iro_hip_free(ctx, dev);
    return rc;
}

}  // extern "C"

// ---- the packed weight as a file ---------------------------------------------

namespace {

constexpr char kMagic[8] = {'I', 'R', 'O', 'W', '8', 'P', 'K', '1'};

struct FileHeader {
    char magic[8];
    int32_t N, K, Np, Kp, layout, nparts, part_N[8];
    int32_t convention;      // rounding convention of the codes, -1 if given
    int32_t separate_rowsum; // rowsum stored after colsum
    uint64_t payload_bytes;
    uint64_t checksum;       // payload_hash of the payload
};

// 64-bit hash of the payload, eight bytes per step (a multiply-xorshift
// mix per word, the tail bytes packed into a last word).
uint64_t payload_hash(const void *p, size_t n) {
    const uint8_t *b = static_cast<const uint8_t *>(p);
    uint64_t h = 0xcbf29ce484222325ull ^ n;
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        uint64_t w;
        std::memcpy(&w, b + i, 8);
        h = (h ^ w) * 0x9E3779B97F4A7C15ull;
        h ^= h >> 29;
    }
    uint64_t t = 0;
    for (size_t k = 0; i + k < n; ++k) t |= (uint64_t)b[i + k] << (8 * k);
    h = (h ^ t) * 0x9E3779B97F4A7C15ull;
    return h ^ (h >> 32);
}

}  // namespace

extern "C" {

int iro_hip_weight_save(IroHipContext *ctx, const IroHipWeight *w, const char *path) {
    if (!ctx || !w || !path) return set_error(ctx, "weight_save: invalid arguments");
    const bool sep = w->rowsum != w->colsum;
    const size_t pk = (size_t)w->Np * w->Kp, vec = sizeof(int32_t) * (size_t)w->Np;
    std::vector<uint8_t> payload(pk + vec * (sep ? 3 : 2));
    if (iro_hip_download(ctx, payload.data(), w->packed, pk) ||
        iro_hip_download(ctx, payload.data() + pk, w->scale, vec) ||
        iro_hip_download(ctx, payload.data() + pk + vec, w->colsum, vec) ||
        (sep && iro_hip_download(ctx, payload.data() + pk + 2 * vec, w->rowsum, vec)))
        return -1;
    FileHeader h;
    std::memset(&h, 0, sizeof(h));
    std::memcpy(h.magic, kMagic, 8);
    h.N = w->N;
    h.K = w->K;
    h.Np = w->Np;
    h.Kp = w->Kp;
    h.layout = w->layout;
    h.nparts = w->nparts;
    for (int i = 0; i < 8; ++i) h.part_N[i] = w->part_N[i];
    h.convention = w->convention;
    h.separate_rowsum = sep;
    h.payload_bytes = payload.size();
    h.checksum = payload_hash(payload.data(), payload.size());
    FILE *f = std::fopen(path, "wb");
    if (!f) return set_error(ctx, "weight_save: cannot create %s", path);
    const bool ok = std::fwrite(&h, sizeof(h), 1, f) == 1 &&
                    std::fwrite(payload.data(), 1, payload.size(), f) == payload.size();
    const bool closed = std::fclose(f) == 0;
    if (!ok || !closed) return set_error(ctx, "weight_save: write to %s failed", path);
    return 0;
}

int iro_hip_weight_load(IroHipContext *ctx, const char *path, IroHipWeight **out) {
    if (!ctx || !path || !out) return set_error(ctx, "weight_load: invalid arguments");
    FILE *f = std::fopen(path, "rb");
    if (!f) return set_error(ctx, "weight_load: cannot open %s", path);
    FileHeader h;
    std::vector<uint8_t> payload;
    bool ok = std::fread(&h, sizeof(h), 1, f) == 1 && std::memcmp(h.magic, kMagic, 8) == 0;
    const long long N = ok ? h.N : 0, K = ok ? h.K : 0;
    ok = ok && N > 0 && K > 0 && h.Np == packed_rows((int)N, (int)h.layout, (int)h.nparts) &&
         h.Kp == (int)round_up((size_t)K, kKPad) && (h.layout == 0 || h.layout == 1) &&
         h.nparts >= 1 && h.nparts <= 8 && (h.separate_rowsum == 0 || h.separate_rowsum == 1);
    long long parts = 0;
    for (int i = 0; ok && i < h.nparts; ++i) {
        ok = h.part_N[i] > 0;
        parts += h.part_N[i];
    }
    ok = ok && parts == N && (long long)h.Np * h.Kp < (1ll << 31);
    const size_t pk = ok ? (size_t)h.Np * h.Kp : 0, vec = ok ? sizeof(int32_t) * (size_t)h.Np : 0;
    ok = ok && h.payload_bytes == pk + vec * (h.separate_rowsum ? 3 : 2);
    if (ok) {
        payload.resize(h.payload_bytes);
        ok = std::fread(payload.data(), 1, payload.size(), f) == payload.size() &&
             std::fgetc(f) == EOF;
    }
    std::fclose(f);
    if (!ok) return set_error(ctx, "weight_load: %s is not a packed int8 weight file", path);
    if (payload_hash(payload.data(), payload.size()) != h.checksum)
        return set_error(ctx, "weight_load: checksum mismatch in %s", path);
    if (h.convention >= 0 && h.convention != ctx->convention)
        return set_error(ctx, "weight_load: %s was quantized under convention %d, the context "
                              "uses %d", path, h.convention, ctx->convention);
    IroHipWeight *w = nullptr;
    if (weight_alloc(ctx, (int)N, (int)K, h.layout, h.nparts, h.part_N, h.separate_rowsum != 0,
                     &w))
        return -1;
    w->convention = h.convention;
    int rc = iro_hip_upload(ctx, w->packed, payload.data(), pk);
    if (!rc) rc = iro_hip_upload(ctx, w->scale, payload.data() + pk, vec);
    if (!rc) rc = iro_hip_upload(ctx, w->colsum, payload.data() + pk + vec, vec);
    if (!rc && h.separate_rowsum) rc = iro_hip_upload(ctx, w->rowsum, payload.data() + pk + 2 * vec, vec);
    if (rc) {
        iro_hip_weight_destroy(w);
        return -1;
    }
    *out = w;
    return 0;
}

}  // extern "C"
