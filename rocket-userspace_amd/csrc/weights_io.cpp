// weights_io.cpp — the serialised form of resident int8 / int4 weights
// (rocket_weights_io.h): a 64-byte little-endian header with XXH64 checksums, the codes in
// the device layout, and optionally the fp32 group scales. Loading maps the file and copies
// the codes to HBM as they are: no re-pack.
#include "resident.h"
#include "rocket_weights_io.h"

#include <fcntl.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <new>
#include <thread>
#include <vector>

using namespace rk;

namespace {

constexpr uint32_t kVersion = 1;
constexpr size_t kHeader = 64;

// XXH64 with seed 0 (Yann Collet's published xxHash specification, 64-bit variant): four
// lanes over 32-byte stripes, then the 8-, 4- and 1-byte tail and the final avalanche.
constexpr uint64_t P1 = 0x9E3779B185EBCA87ull, P2 = 0xC2B2AE3D27D4EB4Full, P3 = 0x165667B19E3779F9ull,
                   P4 = 0x85EBCA77C2B2AE63ull, P5 = 0x27D4EB2F165667C5ull;
inline uint64_t rotl(uint64_t x, int r) { return (x << r) | (x >> (64 - r)); }
inline uint64_t rd64(const uint8_t *p) { uint64_t v; memcpy(&v, p, 8); return v; }   // little-endian host
inline uint32_t rd32(const uint8_t *p) { uint32_t v; memcpy(&v, p, 4); return v; }
inline uint64_t xround(uint64_t acc, uint64_t in) { return rotl(acc + in * P2, 31) * P1; }
inline uint64_t xmerge(uint64_t h, uint64_t v) { return (h ^ xround(0, v)) * P1 + P4; }

uint64_t xxh64(const uint8_t *p, size_t n)
{
    // offsets, not pointer comparisons: no pointer is formed past the buffer (or from null)
    size_t i = 0;
    uint64_t h;
    if (n >= 32) {
        uint64_t v1 = P1 + P2, v2 = P2, v3 = 0, v4 = 0 - P1;
        for (; n - i >= 32; i += 32) {
            v1 = xround(v1, rd64(p + i));
            v2 = xround(v2, rd64(p + i + 8));
            v3 = xround(v3, rd64(p + i + 16));
            v4 = xround(v4, rd64(p + i + 24));
        }
        h = rotl(v1, 1) + rotl(v2, 7) + rotl(v3, 12) + rotl(v4, 18);
        h = xmerge(h, v1);
        h = xmerge(h, v2);
        h = xmerge(h, v3);
        h = xmerge(h, v4);
    } else {
        h = P5;
    }
    h += (uint64_t)n;
    for (; n - i >= 8; i += 8) h = rotl(h ^ xround(0, rd64(p + i)), 27) * P1 + P4;
    if (n - i >= 4) {
        h = rotl(h ^ ((uint64_t)rd32(p + i) * P1), 23) * P2 + P3;
        i += 4;
    }
    for (; i < n; i++) h = rotl(h ^ ((uint64_t)p[i] * P5), 11) * P1;
    h ^= h >> 33;
    h *= P2;
    h ^= h >> 29;
    h *= P3;
    h ^= h >> 32;
    return h;
}

void put32(uint8_t *p, uint32_t v) { for (int i = 0; i < 4; i++) p[i] = (uint8_t)(v >> (8 * i)); }
void put64(uint8_t *p, uint64_t v) { for (int i = 0; i < 8; i++) p[i] = (uint8_t)(v >> (8 * i)); }
uint32_t get32(const uint8_t *p) { uint32_t v = 0; for (int i = 3; i >= 0; i--) v = (v << 8) | p[i]; return v; }
uint64_t get64(const uint8_t *p) { uint64_t v = 0; for (int i = 7; i >= 0; i--) v = (v << 8) | p[i]; return v; }

// What a serialised weight describes, from either side.
struct Desc {
    uint32_t kind;
    int M, K, N, group;
    const void *dev;
    size_t code_bytes;
};

size_t scale_bytes_of(int N, int K, int group)
{
    return group > 0 ? (size_t)N * (size_t)(K / group) * sizeof(float) : 0;
}

size_t total_bytes(const Desc &d, bool with_scales)
{
    return kHeader + d.code_bytes + (with_scales ? scale_bytes_of(d.N, d.K, d.group) : 0);
}

long serialize(int fd, const Desc &d, const float *bs, void *buf, size_t cap, const char *who)
{
    if (!buf) return ROCKET_E_SHAPE;
    if (bs && d.group <= 0) {
        ROCKET_LOGE("%s: scales given for a per-channel weight\n", who);
        return ROCKET_E_SHAPE;
    }
    const size_t sb = bs ? scale_bytes_of(d.N, d.K, d.group) : 0;
    const size_t need = kHeader + d.code_bytes + sb;
    if (cap < need) {
        ROCKET_LOGE("%s: buffer of %zu bytes, need %zu\n", who, cap, need);
        return ROCKET_E_SHAPE;
    }
    uint8_t *out = static_cast<uint8_t *>(buf);
    {
        Locked L(fd);
        if (!L.ok()) return ROCKET_E_DEVICE;
        if (hipMemcpyAsync(out + kHeader, d.dev, d.code_bytes, hipMemcpyDefault, L.h->stream) != hipSuccess ||
            (sb && hipMemcpyAsync(out + kHeader + d.code_bytes, bs, sb, hipMemcpyDefault, L.h->stream) != hipSuccess)) {
            (void)hipGetLastError();
            ROCKET_LOGE("%s: copy from the device failed\n", who);
            return ROCKET_E_DEVICE;
        }
        if (int rc = handle_wait(L.h, who)) return rc;
    }
    memcpy(out, "RKTW", 4);
    put32(out + 4, kVersion);
    put32(out + 8, d.kind);
    put32(out + 12, sb ? 1u : 0u);
    put32(out + 16, (uint32_t)d.N);
    put32(out + 20, (uint32_t)d.K);
    put32(out + 24, (uint32_t)(d.group > 0 ? d.group : 0));
    put32(out + 28, (uint32_t)d.M);
    put64(out + 32, d.code_bytes);
    put64(out + 40, sb);
    put64(out + 48, xxh64(out + kHeader, d.code_bytes + sb));
    put64(out + 56, xxh64(out, 56));
    return (long)need;
}

// The header checks (its own checksum, the kind, shape and sizes); the payload's checksum is
// left to payload_ok.
bool parse_header(const void *buf, size_t len, rocket_weights_info *info)
{
    if (!buf || len < kHeader) return false;
    const uint8_t *p = static_cast<const uint8_t *>(buf);
    if (memcmp(p, "RKTW", 4) != 0 || get32(p + 4) != kVersion) return false;
    if (get64(p + 56) != xxh64(p, 56)) return false;
    rocket_weights_info in;
    in.kind = get32(p + 8);
    in.flags = get32(p + 12);
    in.N = get32(p + 16);
    in.K = get32(p + 20);
    in.group = get32(p + 24);
    in.M = get32(p + 28);
    in.code_bytes = get64(p + 32);
    in.scale_bytes = get64(p + 40);
    if (in.kind != ROCKET_WEIGHTS_KIND_INT8 && in.kind != ROCKET_WEIGHTS_KIND_INT4) return false;
    if (in.flags & ~1u) return false;
    if (in.N == 0 || in.K == 0 || in.N > (uint32_t)kDimMax || in.K > (uint32_t)kDimMax || in.M > (uint32_t)kDimMax)
        return false;
    if (in.group && (in.group < 32 || in.group % 32 || in.K % in.group)) return false;
    const uint64_t code = in.kind == ROCKET_WEIGHTS_KIND_INT8 ? (uint64_t)in.N * in.K : (uint64_t)in.N * in.K / 2;
    if (in.kind == ROCKET_WEIGHTS_KIND_INT4 && in.K % 2) return false;
    if (in.code_bytes != code) return false;
    const uint64_t sb = (in.flags & 1u) ? (in.group ? (uint64_t)in.N * (in.K / in.group) * 4 : ~0ull) : 0;
    if (in.scale_bytes != sb) return false;
    if (len - kHeader < in.code_bytes || len - kHeader - in.code_bytes < in.scale_bytes) return false;
    if (info) *info = in;
    return true;
}

bool payload_ok(const void *buf, const rocket_weights_info &in)
{
    const uint8_t *p = static_cast<const uint8_t *>(buf);
    return get64(p + 48) == xxh64(p + kHeader, (size_t)(in.code_bytes + in.scale_bytes));
}

bool parse(const void *buf, size_t len, rocket_weights_info *info)
{
    rocket_weights_info in;
    if (!parse_header(buf, len, &in) || !payload_ok(buf, in)) return false;
    if (info) *info = in;
    return true;
}

// Validated header + the per-kind shape rules of the pack entries; uploads the codes and
// hands out the scales. Returns the device buffer (nullptr on failure).
// The payload's checksum runs on a second thread while the codes upload (a single XXH64
// stream cannot be split; on a load of config 3's 31 MB weight it is the larger of the two);
// a mismatch frees the upload and fails the call as before.
void *restore(int fd, const void *buf, size_t len, uint32_t kind, float *b_scale_out, rocket_weights_info *info,
              const char *who)
{
    if (!parse_header(buf, len, info)) {
        ROCKET_LOGE("%s: not a valid serialised weight (header, size or checksum)\n", who);
        return nullptr;
    }
    if (info->kind != kind) {
        ROCKET_LOGE("%s: serialised weight is of kind %u, expected %u\n", who, info->kind, kind);
        return nullptr;
    }
    const bool shape_ok = kind == ROCKET_WEIGHTS_KIND_INT8
                              ? (info->N % 32 == 0 && info->K % 32 == 0)
                              : (info->N % 64 == 0 && info->K % 32 == 0 && (!info->group || 49 * info->group < 32767));
    if (!shape_ok || info->M == 0 || info->M % 4) {
        ROCKET_LOGE("%s: serialised shape M=%u K=%u N=%u group=%u is not packable\n", who, info->M, info->K, info->N,
                    info->group);
        return nullptr;
    }
    const uint8_t *p = static_cast<const uint8_t *>(buf);
    bool sum_ok = false;
    std::thread hasher;
    try {
        hasher = std::thread([&sum_ok, buf, &info] { sum_ok = payload_ok(buf, *info); });
    } catch (...) {   // no thread: check first, then upload
        if (!payload_ok(buf, *info)) {
            ROCKET_LOGE("%s: not a valid serialised weight (header, size or checksum)\n", who);
            return nullptr;
        }
        sum_ok = true;
    }
    void *d = nullptr;
    try {   // the checksum thread is joined on every path
        d = upload(fd, p + kHeader, (size_t)info->code_bytes, who);
    } catch (...) {
        d = nullptr;
    }
    if (hasher.joinable()) hasher.join();
    if (!d) return nullptr;
    if (!sum_ok) {
        ROCKET_LOGE("%s: not a valid serialised weight (header, size or checksum)\n", who);
        release(fd, d);
        return nullptr;
    }
    if (b_scale_out && info->scale_bytes) {
        Locked L(fd);
        if (!L.ok() || hipMemcpy(b_scale_out, p + kHeader + info->code_bytes, (size_t)info->scale_bytes,
                                 hipMemcpyDefault) != hipSuccess) {
            (void)hipGetLastError();
            ROCKET_LOGE("%s: copying the scales out failed\n", who);
            dev_free(d);
            return nullptr;
        }
    }
    return d;
}

int save_file(const std::vector<uint8_t> &bytes, const char *path, const char *who)
{
    FILE *f = fopen(path, "wb");
    if (!f) {
        ROCKET_LOGE("%s: cannot open %s for writing\n", who, path);
        return ROCKET_E_SHAPE;
    }
    const bool ok = fwrite(bytes.data(), 1, bytes.size(), f) == bytes.size();
    if (fclose(f) != 0 || !ok) {
        ROCKET_LOGE("%s: writing %s failed\n", who, path);
        return ROCKET_E_SHAPE;
    }
    return ROCKET_OK;
}

// A read-only mapping of a whole file (the page cache serves it; nothing is copied).
struct Mapped {
    const uint8_t *p = nullptr;
    size_t n = 0;
    ~Mapped()
    {
        if (p) munmap(const_cast<uint8_t *>(p), n);
    }
    bool open(const char *path, const char *who)
    {
        const int f = path ? ::open(path, O_RDONLY | O_CLOEXEC) : -1;
        if (f < 0) {
            ROCKET_LOGE("%s: cannot open %s\n", who, path ? path : "(null)");
            return false;
        }
        struct stat st;
        bool ok = fstat(f, &st) == 0 && st.st_size > 0;
        if (ok) {
            void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE | MAP_POPULATE, f, 0);
            ok = m != MAP_FAILED;
            if (ok) {
                p = static_cast<const uint8_t *>(m);
                n = (size_t)st.st_size;
            }
        }
        ::close(f);
        if (!ok) ROCKET_LOGE("%s: mapping %s failed\n", who, path);
        return ok;
    }
};

Desc desc_of(const rocket_i8_weights *w)
{
    return Desc{ROCKET_WEIGHTS_KIND_INT8, w->M, w->K, w->N, w->group, w->dev, w->bytes};
}

Desc desc_of(const rocket_i4_weights *w)
{
    return Desc{ROCKET_WEIGHTS_KIND_INT4, w->M, w->K, w->N, w->group, w->dev, w->bytes};
}

template <class Ctx, class W>
int save(Ctx *ctx, const W *w, const float *b_scale, const char *path, const char *who)
{
    if (!ctx || !w || !path) return ROCKET_E_SHAPE;
    const Desc d = desc_of(w);
    std::vector<uint8_t> bytes;
    try {
        bytes.resize(total_bytes(d, b_scale != nullptr));
    } catch (...) {
        return ROCKET_E_NOMEM;
    }
    const long n = serialize(ctx->fd, d, b_scale, bytes.data(), bytes.size(), who);
    if (n < 0) return (int)n;
    return save_file(bytes, path, who);
}

template <class W, class Ctx>
W *deserialize(Ctx *ctx, const void *buf, size_t len, float *b_scale_out, uint32_t kind, const char *who)
{
    if (!ctx) return nullptr;
    rocket_weights_info info;
    void *d = restore(ctx->fd, buf, len, kind, b_scale_out, &info, who);
    if (!d) return nullptr;
    W *w = new (std::nothrow) W{(int)info.M, (int)info.K, (int)info.N, (int)info.group, d, (size_t)info.code_bytes};
    if (!w) release(ctx->fd, d);
    return w;
}

}  // namespace

extern "C" {

uint64_t rocket_weights_xxh64(const void *buf, size_t len)
{
    return xxh64(static_cast<const uint8_t *>(buf), buf ? len : 0);
}

int rocket_weights_info_read(const void *buf, size_t len, rocket_weights_info *info)
{
    return parse(buf, len, info) ? ROCKET_OK : ROCKET_E_SHAPE;
}

size_t rocket_i8_weights_serialized_bytes(const rocket_i8_weights *w, int with_scales)
{
    return w ? total_bytes(desc_of(w), with_scales != 0) : 0;
}

size_t rocket_i4_weights_serialized_bytes(const rocket_i4_weights *w, int with_scales)
{
    return w ? total_bytes(desc_of(w), with_scales != 0) : 0;
}

long rocket_i8_weights_serialize(rocket_i8_ctx *ctx, const rocket_i8_weights *w, const float *b_scale, void *buf,
                                 size_t cap)
{
    if (!ctx || !w) return ROCKET_E_SHAPE;
    return serialize(ctx->fd, desc_of(w), b_scale, buf, cap, "rocket_i8_weights_serialize");
}

long rocket_i4_weights_serialize(rocket_i4_ctx *ctx, const rocket_i4_weights *w, const float *b_scale, void *buf,
                                 size_t cap)
{
    if (!ctx || !w) return ROCKET_E_SHAPE;
    return serialize(ctx->fd, desc_of(w), b_scale, buf, cap, "rocket_i4_weights_serialize");
}

rocket_i8_weights *rocket_i8_weights_deserialize(rocket_i8_ctx *ctx, const void *buf, size_t len, float *b_scale_out)
{
    return deserialize<rocket_i8_weights>(ctx, buf, len, b_scale_out, ROCKET_WEIGHTS_KIND_INT8,
                                          "rocket_i8_weights_deserialize");
}

rocket_i4_weights *rocket_i4_weights_deserialize(rocket_i4_ctx *ctx, const void *buf, size_t len, float *b_scale_out)
{
    return deserialize<rocket_i4_weights>(ctx, buf, len, b_scale_out, ROCKET_WEIGHTS_KIND_INT4,
                                          "rocket_i4_weights_deserialize");
}

int rocket_i8_weights_save(rocket_i8_ctx *ctx, const rocket_i8_weights *w, const float *b_scale, const char *path)
{
    return save(ctx, w, b_scale, path, "rocket_i8_weights_save");
}

int rocket_i4_weights_save(rocket_i4_ctx *ctx, const rocket_i4_weights *w, const float *b_scale, const char *path)
{
    return save(ctx, w, b_scale, path, "rocket_i4_weights_save");
}

rocket_i8_weights *rocket_i8_weights_load(rocket_i8_ctx *ctx, const char *path, float *b_scale_out)
{
    Mapped m;
    if (!ctx || !m.open(path, "rocket_i8_weights_load")) return nullptr;
    return rocket_i8_weights_deserialize(ctx, m.p, m.n, b_scale_out);
}

rocket_i4_weights *rocket_i4_weights_load(rocket_i4_ctx *ctx, const char *path, float *b_scale_out)
{
    Mapped m;
    if (!ctx || !m.open(path, "rocket_i4_weights_load")) return nullptr;
    return rocket_i4_weights_deserialize(ctx, m.p, m.n, b_scale_out);
}

}  // extern "C"
