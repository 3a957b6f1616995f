// resident.cpp — resident-weight contexts, streaming/batched/multi-worker wrappers and
// the MI355X-only entries of rocket_hip.h.
//
// The reference keeps packed weights in per-worker NPU buffer objects, one DRM fd per
// worker thread (reference src/rocket_prepacked.c, rocket_prepacked_int8.c,
// rocket_prepacked_int4.c, rocket_bf16_stream.c, rocket_matmul_mt.c). Here a context is
// one HIP handle and a weight is one HBM buffer laid out for the kernels: int8 and fp16
// rows as given, int4 nibble-packed (half the bytes). The layout does not depend on M,
// so a weight packed at one M serves every M.
#include "resident.h"
#include "rocket_activation.h"
#include "rocket_hip.h"
#include "rocket_quant.h"

#include <stdlib.h>
#include <string.h>

#include <new>

using namespace rk;

struct rocket_ctx         { int fd; int nthreads; };
struct rocket_weights     { int M, K, N; void *dev; };
struct rocket_stream      { int fd; };
struct rocket_bf16_stream { int fd; };
struct rocket_mm_batch    { int fd; };

namespace rk {

void *upload(int fd, const void *src, size_t bytes, const char *who)
{
    Locked L(fd);
    if (!L.ok()) return nullptr;
    void *d = dev_alloc(bytes, who);
    if (!d) return nullptr;
    if (hipMemcpyAsync(d, src, bytes, hipMemcpyDefault, L.h->stream) != hipSuccess) {
        (void)hipGetLastError();
        dev_free(d);
        return nullptr;
    }
    if (handle_wait(L.h, who)) { dev_free(d); return nullptr; }
    return d;
}

void release(int fd, void *dev)
{
    if (!dev) return;
    Locked L(fd);
    if (L.ok()) (void)hipStreamSynchronize(L.h->stream);
    dev_free(dev);
}

}  // namespace rk

namespace {

int clamp_threads(int n) { return n < 1 ? 1 : (n > 8 ? 8 : n); }

int open_handle(const char *who)
{
    const int fd = rocket_open();
    if (fd < 0) ROCKET_LOGE("%s: rocket_open failed (%d)\n", who, fd);
    return fd;
}

// int4 values one per byte -> resident nibble-packed buffer (blocking).
void *upload_int4(int fd, const int8_t *B, int N, int K, const char *who)
{
    void *tmp = upload(fd, B, (size_t)N * K, who);
    if (!tmp) return nullptr;
    Locked L(fd);
    void *d = L.ok() ? dev_alloc((size_t)N * K / 2, who) : nullptr;
    if (d) {
        if (pack_int4(static_cast<const int8_t *>(tmp), static_cast<uint8_t *>(d), N, K, L.h->stream) != hipSuccess ||
            handle_wait(L.h, who)) {
            (void)hipGetLastError();
            dev_free(d);
            d = nullptr;
        } else {
            count_launch((uint64_t)(((size_t)N * K / 8 + 255) / 256));
        }
    }
    if (L.ok()) (void)hipStreamSynchronize(L.h->stream);
    dev_free(tmp);
    return d;
}

bool call_m_ok(const char *who, int M)
{   // reference rocket_prepacked_int8.c:678-682 / rocket_prepacked_int4.c:257-264
    if (M % 4 != 0 || M <= 0) {
        ROCKET_LOGE("%s: M=%d must be a positive multiple of 4 — pad rows caller-side\n", who, M);
        return false;
    }
    return true;
}

// quant_a: A holds fp32 activations quantised per row on the device (as unused).
int gw_resident(int fd, const char *who, bool int4, int M, int K, int N, const void *A,
                const float *as, const float *bs, float *Cf, const void *wdev, int group,
                int32_t *dump, int row0, int nrows, bool rowscale = false, int quant_a = 0)
{
    if (!A || (!as && !quant_a) || !bs || !Cf) return ROCKET_E_SHAPE;
    Req r;
    const void *a = A, *b = wdev;
    void *c = Cf;
    r.who = who; r.fa = Fmt::I8; r.fb = int4 ? Fmt::I4P : Fmt::I8; r.b_packed = int4;
    r.epi = Epi::GW; r.K = K; r.N = N; r.M = &M; r.A = &a; r.B = &b; r.C = &c;
    r.a_scale = &as; r.b_scale = &bs; r.group = group;
    r.dump = &dump; r.dump_row0 = &row0; r.dump_rows = &nrows;
    r.rowscale = rowscale;
    r.quant_a = quant_a;
    return run(fd, r);
}

bool dump_args_ok(int M, int row0, int nrows, const int32_t *P)
{
    if (nrows < 0 || row0 < 0 || (nrows > 0 && (!P || row0 + nrows > M))) return false;
    return true;
}

}  // namespace

extern "C" {

// =====================================================================================
// fp16 resident weights (reference rocket_prepacked.c:106-250, 411-447)
// =====================================================================================
rocket_ctx *rocket_ctx_create(int nthreads)
{
    const int fd = open_handle("rocket_ctx_create");
    if (fd < 0) return nullptr;
    rocket_ctx *c = new (std::nothrow) rocket_ctx{fd, clamp_threads(nthreads)};
    if (!c) rocket_close(fd);
    return c;
}

void rocket_ctx_free(rocket_ctx *ctx)
{
    if (!ctx) return;
    rocket_close(ctx->fd);
    delete ctx;
}

rocket_weights *rocket_weights_pack(rocket_ctx *ctx, int M, int K, int N, const _Float16 *B)
{
    if (!ctx || !B) return nullptr;
    if (rocket_matmul_plan(M, K, N, nullptr, nullptr, nullptr) < 0) {
        ROCKET_LOGE("rocket_weights_pack: unsupported shape M=%d K=%d N=%d (need K%%32, N%%16, M%%4)\n", M, K, N);
        return nullptr;
    }
    void *d = upload(ctx->fd, B, (size_t)N * K * 2, "rocket_weights_pack");
    if (!d) return nullptr;
    rocket_weights *w = new (std::nothrow) rocket_weights{M, K, N, d};
    if (!w) release(ctx->fd, d);
    return w;
}

void rocket_weights_free(rocket_ctx *ctx, rocket_weights *w)
{
    if (!w) return;
    if (ctx) release(ctx->fd, w->dev);
    else dev_free(w->dev);
    delete w;
}

int rocket_matmul_fp16_prepacked(rocket_ctx *ctx, int M, int K, int N, const _Float16 *A, _Float16 *C,
                                 rocket_weights *w)
{
    if (!ctx || !w || !A || !C) return ROCKET_E_SHAPE;
    if (K != w->K || N != w->N) return ROCKET_E_SHAPE;
    if (rocket_matmul_plan(M, K, N, nullptr, nullptr, nullptr) < 0) return ROCKET_E_SHAPE;
    Req r;
    const void *a = A, *b = w->dev;
    void *c = C;
    r.who = "rocket_matmul_fp16_prepacked"; r.fa = r.fb = Fmt::F16; r.epi = Epi::F16;
    r.K = K; r.N = N; r.M = &M; r.A = &a; r.B = &b; r.C = &c;
    return run(ctx->fd, r);
}

// =====================================================================================
// fp16 streaming / fused streaming (reference rocket_prepacked.c:455-505)
// =====================================================================================
rocket_stream *rocket_stream_create(int nthreads)
{
    (void)nthreads;
    const int fd = open_handle("rocket_stream_create");
    if (fd < 0) return nullptr;
    rocket_stream *s = new (std::nothrow) rocket_stream{fd};
    if (!s) rocket_close(fd);
    return s;
}

void rocket_stream_free(rocket_stream *s)
{
    if (!s) return;
    rocket_close(s->fd);
    delete s;
}

int rocket_matmul_fp16_stream(rocket_stream *s, int M, int K, int N, const _Float16 *A, const _Float16 *B,
                              _Float16 *C)
{
    if (!s || !A || !B || !C) return ROCKET_E_SHAPE;
    if (rocket_matmul_plan(M, K, N, nullptr, nullptr, nullptr) < 0) return ROCKET_E_SHAPE;
    Req r;
    const void *a = A, *b = B;
    void *c = C;
    r.who = "rocket_matmul_fp16_stream"; r.fa = r.fb = Fmt::F16; r.epi = Epi::F16;
    r.K = K; r.N = N; r.M = &M; r.A = &a; r.B = &b; r.C = &c;
    return run(s->fd, r);
}

int rocket_matmul_fp16_stream_fused(rocket_stream *s, int M, int K, const _Float16 *const *Bs, const int *Ns,
                                    int nseg, const _Float16 *A, _Float16 *C)
{
    if (!s || nseg < 1 || nseg > ROCKET_MAX_FUSE || !Bs || !Ns || !A || !C) return ROCKET_E_SHAPE;
    long Ntot = 0;
    for (int i = 0; i < nseg; i++) {
        if (!Bs[i] || Ns[i] <= 0) return ROCKET_E_SHAPE;
        Ntot += Ns[i];
    }
    if (Ntot > kDimMax || rocket_matmul_plan(M, K, (int)Ntot, nullptr, nullptr, nullptr) < 0)
        return ROCKET_E_SHAPE;
    // the segments become contiguous rows of one [Ntot, K] weight in HBM (device copies
    // for device segments), then one launch over the combined N
    const size_t row = (size_t)K * 2;
    void *cat = nullptr;
    {
        Locked L(s->fd);
        if (!L.ok()) return ROCKET_E_DEVICE;
        cat = dev_alloc((size_t)Ntot * row, "rocket_matmul_fp16_stream_fused");
        if (!cat) return ROCKET_E_NOMEM;
        size_t off = 0;
        for (int i = 0; i < nseg; i++) {
            if (hipMemcpyAsync(static_cast<char *>(cat) + off, Bs[i], (size_t)Ns[i] * row, hipMemcpyDefault,
                               L.h->stream) != hipSuccess) {
                (void)hipGetLastError();
                (void)hipStreamSynchronize(L.h->stream);
                dev_free(cat);
                return ROCKET_E_DEVICE;
            }
            off += (size_t)Ns[i] * row;
        }
    }
    Req r;
    const int Nt = (int)Ntot;
    const void *a = A, *b = cat;
    void *c = C;
    r.who = "rocket_matmul_fp16_stream_fused"; r.fa = r.fb = Fmt::F16; r.epi = Epi::F16;
    r.K = K; r.N = Nt; r.M = &M; r.A = &a; r.B = &b; r.C = &c;
    const int rc = run(s->fd, r);
    release(s->fd, cat);
    return rc;
}

// =====================================================================================
// batched fp16 context (reference rocket_matmul.c:2042-2310)
// =====================================================================================
rocket_mm_batch *rocket_mm_batch_create(int fd)
{
    if (!handle_get(fd)) return nullptr;
    return new (std::nothrow) rocket_mm_batch{fd};
}

void rocket_mm_batch_free(rocket_mm_batch *b) { delete b; }

int rocket_mm_batch_run(rocket_mm_batch *b, int M, int K, int N, int nbatch, const _Float16 *const *A,
                        const _Float16 *const *B, _Float16 *const *C)
{
    if (!b) return ROCKET_E_SHAPE;
    return rocket_matmul_fp16_batch(b->fd, M, K, N, nbatch, A, B, C);
}

// =====================================================================================
// multi-worker and streaming wrappers (reference rocket_matmul_mt.c:58-99,
// rocket_bf16_stream.c:344-549): one GPU grid covers every N slice
// =====================================================================================
int rocket_matmul_fp16_mt(int M, int K, int N, const _Float16 *A, const _Float16 *B, _Float16 *C, int nthreads)
{
    (void)clamp_threads(nthreads);
    const int fd = open_handle("rocket_matmul_fp16_mt");
    if (fd < 0) return ROCKET_E_DEVICE;
    const int rc = rocket_matmul_fp16(fd, M, K, N, A, B, C);
    rocket_close(fd);
    return rc;
}

int rocket_matmul_bf16_mt(int M, int K, int N, const float *A, const float *B, float *C, int nthreads)
{
    (void)clamp_threads(nthreads);
    const int fd = open_handle("rocket_matmul_bf16_mt");
    if (fd < 0) return ROCKET_E_DEVICE;
    const int rc = rocket_matmul_bf16(fd, M, K, N, A, B, C);
    rocket_close(fd);
    return rc;
}

rocket_bf16_stream *rocket_bf16_stream_create(int nthreads)
{
    (void)nthreads;
    const int fd = open_handle("rocket_bf16_stream_create");
    if (fd < 0) return nullptr;
    rocket_bf16_stream *s = new (std::nothrow) rocket_bf16_stream{fd};
    if (!s) rocket_close(fd);
    return s;
}

void rocket_bf16_stream_free(rocket_bf16_stream *s)
{
    if (!s) return;
    rocket_close(s->fd);
    delete s;
}

int rocket_matmul_bf16_stream(rocket_bf16_stream *s, int M, int K, int N, const float *A, const float *B, float *C)
{
    if (!s) return ROCKET_E_SHAPE;
    if (rocket_matmul_plan_bf16(M, K, N, nullptr, nullptr, nullptr) < 0) return ROCKET_E_SHAPE;
    return rocket_matmul_bf16(s->fd, M, K, N, A, B, C);
}

// =====================================================================================
// int8 resident weights (reference rocket_prepacked_int8.c:167-767)
// =====================================================================================
rocket_i8_ctx *rocket_i8_ctx_create(int nthreads)
{
    const int fd = open_handle("rocket_i8_ctx_create");
    if (fd < 0) return nullptr;
    rocket_i8_ctx *c = new (std::nothrow) rocket_i8_ctx{fd, clamp_threads(nthreads)};
    if (!c) rocket_close(fd);
    return c;
}

void rocket_i8_ctx_free(rocket_i8_ctx *ctx)
{
    if (!ctx) return;
    rocket_close(ctx->fd);
    delete ctx;
}

static bool i8_shape_ok(const char *who, int M, int K, int N)
{   // reference rocket_prepacked_int8.c:404-415
    if (N % 32 != 0 || K % 32 != 0 || M % 4 != 0 || N <= 0 || K <= 0 || M <= 0 ||
        N > kDimMax || K > kDimMax || M > kDimMax) {
        ROCKET_LOGE("%s: unsupported shape M=%d K=%d N=%d (need N%%32, K%%32, M%%4)\n", who, M, K, N);
        return false;
    }
    return true;
}

static rocket_i8_weights *i8_pack(rocket_i8_ctx *ctx, int M, int K, int N, const int8_t *B, int group,
                                  const char *who)
{
    if (!ctx || !B || !i8_shape_ok(who, M, K, N)) return nullptr;
    if (group && (group < 32 || group % 32 || K % group)) {
        ROCKET_LOGE("%s: bad group=%d (need >=32, %%32, |K) K=%d\n", who, group, K);
        return nullptr;
    }
    void *d = upload(ctx->fd, B, (size_t)N * K, who);
    if (!d) return nullptr;
    rocket_i8_weights *w = new (std::nothrow) rocket_i8_weights{M, K, N, group, d, (size_t)N * K};
    if (!w) release(ctx->fd, d);
    return w;
}

rocket_i8_weights *rocket_i8_weights_pack(rocket_i8_ctx *ctx, int M, int K, int N, const int8_t *B)
{
    return i8_pack(ctx, M, K, N, B, 0, "rocket_i8_weights_pack");
}

rocket_i8_weights *rocket_i8_weights_pack_gw(rocket_i8_ctx *ctx, int M, int K, int N, const int8_t *B, int group)
{
    return i8_pack(ctx, M, K, N, B, group, "rocket_i8_weights_pack_gw");
}

void rocket_i8_weights_free(rocket_i8_ctx *ctx, rocket_i8_weights *w)
{
    if (!w) return;
    if (ctx) release(ctx->fd, w->dev);
    else dev_free(w->dev);
    delete w;
}

size_t rocket_i8_weights_bytes(const rocket_i8_weights *w) { return w ? w->bytes : 0; }

static int i8_resolve(rocket_i8_ctx *ctx, const char *who, int M, int K, int N, const rocket_i8_weights *w)
{   // reference rocket_prepacked_int8.c:666-694
    if (!call_m_ok(who, M)) return ROCKET_E_SHAPE;
    if (K != w->K || N != w->N) {
        ROCKET_LOGE("%s: shape K=%d N=%d != packed %d/%d\n", who, K, N, w->K, w->N);
        return ROCKET_E_SHAPE;
    }
    (void)ctx;
    return ROCKET_OK;
}

int rocket_matmul_int8_prepacked(rocket_i8_ctx *ctx, int M, int K, int N, const int8_t *A, int32_t *C,
                                 rocket_i8_weights *w)
{
    if (!ctx || !w || !A || !C) return ROCKET_E_SHAPE;
    if (w->group != 0) {
        ROCKET_LOGE("rocket_matmul_int8_prepacked: weight is group-wise (group=%d) — "
                    "use rocket_matmul_int8_prepacked_gw\n", w->group);
        return ROCKET_E_SHAPE;
    }
    if (int rc = i8_resolve(ctx, "rocket_matmul_int8_prepacked", M, K, N, w)) return rc;
    Req r;
    const void *a = A, *b = w->dev;
    void *c = C;
    r.who = "rocket_matmul_int8_prepacked"; r.fa = r.fb = Fmt::I8; r.epi = Epi::I32;
    r.K = K; r.N = N; r.M = &M; r.A = &a; r.B = &b; r.C = &c;
    return run(ctx->fd, r);
}

int rocket_matmul_int8_prepacked_gw(rocket_i8_ctx *ctx, int M, int K, int N, const int8_t *A,
                                    const float *a_scale, const float *b_scale, float *Cf, rocket_i8_weights *w)
{
    if (!ctx || !w || !A || !a_scale || !b_scale || !Cf) return ROCKET_E_SHAPE;
    if (w->group <= 0) {
        ROCKET_LOGE("rocket_matmul_int8_prepacked_gw: weight is per-channel — use rocket_matmul_int8_prepacked\n");
        return ROCKET_E_SHAPE;
    }
    if (int rc = i8_resolve(ctx, "rocket_matmul_int8_prepacked_gw", M, K, N, w)) return rc;
    return gw_resident(ctx->fd, "rocket_matmul_int8_prepacked_gw", false, M, K, N, A, a_scale, b_scale, Cf,
                       w->dev, w->group, nullptr, 0, 0);
}

// =====================================================================================
// int4 resident weights (reference rocket_prepacked_int4.c:122-686)
// =====================================================================================
rocket_i4_ctx *rocket_i4_ctx_create(int nthreads)
{
    const int fd = open_handle("rocket_i4_ctx_create");
    if (fd < 0) return nullptr;
    rocket_i4_ctx *c = new (std::nothrow) rocket_i4_ctx{fd, clamp_threads(nthreads)};
    if (!c) rocket_close(fd);
    return c;
}

void rocket_i4_ctx_free(rocket_i4_ctx *ctx)
{
    if (!ctx) return;
    rocket_close(ctx->fd);
    delete ctx;
}

static rocket_i4_weights *i4_pack(rocket_i4_ctx *ctx, int M, int K, int N, const int8_t *B, int group,
                                  const char *who)
{
    if (!ctx || !B) return nullptr;
    if (N % 64 != 0 || K % 32 != 0 || M % 4 != 0 || N <= 0 || K <= 0 || M <= 0 ||
        N > kDimMax || K > kDimMax || M > kDimMax) {
        ROCKET_LOGE("%s: unsupported shape M=%d K=%d N=%d (need N%%64, K%%32, M%%4)\n", who, M, K, N);
        return nullptr;
    }
    if (group && (group < 32 || group % 32 || K % group || 49 * group >= 32767)) {
        ROCKET_LOGE("%s: bad group=%d (need %%32, |K, 49*group<32767) K=%d\n", who, group, K);
        return nullptr;
    }
    void *d = upload_int4(ctx->fd, B, N, K, who);
    if (!d) return nullptr;
    rocket_i4_weights *w = new (std::nothrow) rocket_i4_weights{M, K, N, group, d, (size_t)N * K / 2};
    if (!w) release(ctx->fd, d);
    return w;
}

rocket_i4_weights *rocket_i4_weights_pack(rocket_i4_ctx *ctx, int M, int K, int N, const int8_t *B)
{
    return i4_pack(ctx, M, K, N, B, 0, "rocket_i4_weights_pack");
}

rocket_i4_weights *rocket_i4_weights_pack_gw(rocket_i4_ctx *ctx, int M, int K, int N, const int8_t *B, int group)
{
    return i4_pack(ctx, M, K, N, B, group, "rocket_i4_weights_pack_gw");
}

void rocket_i4_weights_free(rocket_i4_ctx *ctx, rocket_i4_weights *w)
{
    if (!w) return;
    if (ctx) release(ctx->fd, w->dev);
    else dev_free(w->dev);
    delete w;
}

size_t rocket_i4_weights_bytes(const rocket_i4_weights *w) { return w ? w->bytes : 0; }

int rocket_matmul_int4_prepacked(rocket_i4_ctx *ctx, int M, int K, int N, const int8_t *A, int32_t *C,
                                 rocket_i4_weights *w)
{
    if (!ctx || !w || !A || !C) return ROCKET_E_SHAPE;
    if (!call_m_ok("rocket_matmul_int4_prepacked", M)) return ROCKET_E_SHAPE;
    if (K != w->K || N != w->N) {
        ROCKET_LOGE("rocket_matmul_int4_prepacked: shape K=%d N=%d != packed %d/%d\n", K, N, w->K, w->N);
        return ROCKET_E_SHAPE;
    }
    Req r;
    const void *a = A, *b = w->dev;
    void *c = C;
    r.who = "rocket_matmul_int4_prepacked"; r.fa = Fmt::I8; r.fb = Fmt::I4P; r.b_packed = true;
    r.epi = Epi::I32; r.K = K; r.N = N; r.M = &M; r.A = &a; r.B = &b; r.C = &c;
    r.kchunk = 65536;
    return run(ctx->fd, r);
}

int rocket_matmul_int4_prepacked_gw(rocket_i4_ctx *ctx, int M, int K, int N, const int8_t *A,
                                    const float *a_scale, const float *b_scale, float *Cf, rocket_i4_weights *w)
{
    if (!ctx || !w || w->group <= 0) return ROCKET_E_SHAPE;
    if (!call_m_ok("rocket_matmul_int4_prepacked_gw", M)) return ROCKET_E_SHAPE;
    if (K != w->K || N != w->N) {
        ROCKET_LOGE("rocket_matmul_int4_prepacked_gw: shape K=%d N=%d != packed %d/%d\n", K, N, w->K, w->N);
        return ROCKET_E_SHAPE;
    }
    return gw_resident(ctx->fd, "rocket_matmul_int4_prepacked_gw", true, M, K, N, A, a_scale, b_scale, Cf,
                       w->dev, w->group, nullptr, 0, 0);
}

// =====================================================================================
// rocket_hip.h
// =====================================================================================
void *rocket_hip_stream(int fd)
{
    Locked L(fd);
    return L.ok() ? (void *)L.h->stream : nullptr;
}

int rocket_hip_set_stream(int fd, void *stream)
{
    Locked L(fd);
    if (!L.ok()) return ROCKET_E_DEVICE;
    // work already queued on the old stream completes before the new one is used
    if (hipStreamSynchronize(L.h->stream) != hipSuccess) { (void)hipGetLastError(); return ROCKET_E_DEVICE; }
    L.h->stream = stream ? static_cast<hipStream_t>(stream) : L.h->own;
    return ROCKET_OK;
}

int rocket_hip_set_mode(int fd, unsigned mode)
{
    Locked L(fd);
    if (!L.ok()) return ROCKET_E_DEVICE;
    if (mode & ~(ROCKET_HIP_ASYNC | ROCKET_HIP_DEVICE_OPERANDS)) return ROCKET_E_SHAPE;
    L.h->async = (mode & ROCKET_HIP_ASYNC) != 0;
    L.h->trust_device = (mode & ROCKET_HIP_DEVICE_OPERANDS) != 0;
    return ROCKET_OK;
}

int rocket_hip_sync(int fd)
{
    Locked L(fd);
    if (!L.ok()) return ROCKET_E_DEVICE;
    return handle_wait(L.h, "rocket_hip_sync");
}

int rocket_ctx_fd(const rocket_ctx *ctx) { return ctx ? ctx->fd : ROCKET_E_SHAPE; }
int rocket_i8_ctx_fd(const rocket_i8_ctx *ctx) { return ctx ? ctx->fd : ROCKET_E_SHAPE; }
int rocket_i4_ctx_fd(const rocket_i4_ctx *ctx) { return ctx ? ctx->fd : ROCKET_E_SHAPE; }
int rocket_stream_fd(const rocket_stream *s) { return s ? s->fd : ROCKET_E_SHAPE; }
int rocket_bf16_stream_fd(const rocket_bf16_stream *s) { return s ? s->fd : ROCKET_E_SHAPE; }

const void *rocket_i8_weights_device(const rocket_i8_weights *w) { return w ? w->dev : nullptr; }
const void *rocket_i4_weights_device(const rocket_i4_weights *w) { return w ? w->dev : nullptr; }

int rocket_matmul_int8_groupwise_dump(int fd, int M, int K, int N, const int8_t *A, const int8_t *B,
                                      const float *a_scale, const float *b_scale, float *Cf, int group,
                                      int row0, int nrows, int32_t *P)
{
    if (rocket_matmul_plan_int8_gw(M, K, N, group, nullptr, nullptr, nullptr) < 0) return ROCKET_E_SHAPE;
    if (!dump_args_ok(M, row0, nrows, P) || gw_period(group) != group) return ROCKET_E_SHAPE;
    if (!A || !B || !a_scale || !b_scale || !Cf) return ROCKET_E_SHAPE;
    Req r;
    const void *a = A, *b = B;
    void *c = Cf;
    r.who = "rocket_matmul_int8_groupwise_dump"; r.fa = r.fb = Fmt::I8; r.epi = Epi::GW;
    r.K = K; r.N = N; r.M = &M; r.A = &a; r.B = &b; r.C = &c;
    r.a_scale = &a_scale; r.b_scale = &b_scale; r.group = group;
    r.dump = &P; r.dump_row0 = &row0; r.dump_rows = &nrows;
    return run(fd, r);
}

int rocket_matmul_int4_groupwise_dump(int fd, int M, int K, int N, const int8_t *A, const int8_t *B,
                                      const float *a_scale, const float *b_scale, float *Cf, int group,
                                      int row0, int nrows, int32_t *P)
{
    if (group < 32 || group % 32 || K % group || M % 4 || 49 * group >= 32767) return ROCKET_E_SHAPE;
    if (rocket_matmul_plan_int4(M, K, N, nullptr, nullptr, nullptr) < 0) return ROCKET_E_SHAPE;
    if (!dump_args_ok(M, row0, nrows, P)) return ROCKET_E_SHAPE;
    if (!A || !B || !a_scale || !b_scale || !Cf) return ROCKET_E_SHAPE;
    Req r;
    const void *a = A, *b = B;
    void *c = Cf;
    r.who = "rocket_matmul_int4_groupwise_dump"; r.fa = Fmt::I8; r.fb = Fmt::I4P; r.pack_b_int4 = true;
    r.epi = Epi::GW; r.K = K; r.N = N; r.M = &M; r.A = &a; r.B = &b; r.C = &c;
    r.a_scale = &a_scale; r.b_scale = &b_scale; r.group = group;
    r.dump = &P; r.dump_row0 = &row0; r.dump_rows = &nrows;
    return run(fd, r);
}

int rocket_matmul_int8_prepacked_gw_dump(rocket_i8_ctx *ctx, int M, int K, int N, const int8_t *A,
                                         const float *a_scale, const float *b_scale, float *Cf,
                                         rocket_i8_weights *w, int row0, int nrows, int32_t *P)
{
    if (!ctx || !w || w->group <= 0) return ROCKET_E_SHAPE;
    if (int rc = i8_resolve(ctx, "rocket_matmul_int8_prepacked_gw_dump", M, K, N, w)) return rc;
    if (!dump_args_ok(M, row0, nrows, P) || gw_period(w->group) != w->group) return ROCKET_E_SHAPE;
    return gw_resident(ctx->fd, "rocket_matmul_int8_prepacked_gw_dump", false, M, K, N, A, a_scale, b_scale,
                       Cf, w->dev, w->group, nrows ? P : nullptr, row0, nrows);
}

int rocket_matmul_int4_prepacked_gw_dump(rocket_i4_ctx *ctx, int M, int K, int N, const int8_t *A,
                                         const float *a_scale, const float *b_scale, float *Cf,
                                         rocket_i4_weights *w, int row0, int nrows, int32_t *P)
{
    if (!ctx || !w || w->group <= 0) return ROCKET_E_SHAPE;
    if (!call_m_ok("rocket_matmul_int4_prepacked_gw_dump", M)) return ROCKET_E_SHAPE;
    if (K != w->K || N != w->N) return ROCKET_E_SHAPE;
    if (!dump_args_ok(M, row0, nrows, P)) return ROCKET_E_SHAPE;
    return gw_resident(ctx->fd, "rocket_matmul_int4_prepacked_gw_dump", true, M, K, N, A, a_scale, b_scale,
                       Cf, w->dev, w->group, nrows ? P : nullptr, row0, nrows);
}

static int gw_grouped(const char *who, bool rowscale, rocket_i8_ctx *ctx, int n, const int *M, int K, int N,
                      const void *const *A, const float *const *a_scale, const float *const *b_scale,
                      float *const *Cf, rocket_i8_weights *const *w, int quant_a = 0,
                      const int *row0 = nullptr, const int *nrows = nullptr, int32_t *const *P = nullptr,
                      bool glu = false, const void *const *A2 = nullptr, int act = 0, bool f16out = false)
{
    if (glu && (!A2 || (act != ROCKET_ACTIVATION_SILU && act != ROCKET_ACTIVATION_GELU))) {
        ROCKET_LOGE("%s: activation kind %d (SILU or GELU) or a null up-operand array\n", who, act);
        return ROCKET_E_SHAPE;
    }
    if (!ctx || n < 1 || !M || !A || (!a_scale && !quant_a) || !b_scale || !Cf || !w) return ROCKET_E_SHAPE;
    std::vector<const void *> As(n), Bs(n);
    std::vector<void *> Cs(n);
    const int group = w[0] ? w[0]->group : 0;
    if (group <= 0) return ROCKET_E_SHAPE;
    for (int e = 0; e < n; e++) {
        if (!w[e] || w[e]->group != group || w[e]->K != K || w[e]->N != N) {
            ROCKET_LOGE("%s: weight %d does not match (K=%d N=%d group=%d)\n", who, e, K, N, group);
            return ROCKET_E_SHAPE;
        }
        if (M[e] < 0 || M[e] % 4 || M[e] > kDimMax) {
            ROCKET_LOGE("%s: M[%d]=%d must be a multiple of 4\n", who, e, M[e]);
            return ROCKET_E_SHAPE;
        }
        if (M[e] && (!A[e] || (!quant_a && !a_scale[e]) || !b_scale[e] || !Cf[e])) return ROCKET_E_SHAPE;
        if (M[e] && glu && !A2[e]) return ROCKET_E_SHAPE;
        if (P && (!row0 || !nrows || !dump_args_ok(M[e], row0[e], nrows[e], P[e]))) return ROCKET_E_SHAPE;
        As[e] = A[e]; Bs[e] = w[e]->dev; Cs[e] = Cf[e];
    }
    if (P && gw_period(group) != group) return ROCKET_E_SHAPE;
    Req r;
    r.who = who; r.fa = r.fb = Fmt::I8; r.epi = Epi::GW; r.K = K; r.N = N; r.nprob = n;
    r.M = M; r.A = As.data(); r.B = Bs.data(); r.C = Cs.data();
    r.a_scale = a_scale; r.b_scale = b_scale; r.group = group; r.rowscale = rowscale;
    r.quant_a = quant_a;
    r.A2 = glu ? A2 : nullptr;
    r.act = glu ? act : 0;
    r.f16out = f16out;
    if (P) { r.dump = P; r.dump_row0 = row0; r.dump_rows = nrows; }
    return run(ctx->fd, r);
}

int rocket_matmul_int8_prepacked_gw_grouped(rocket_i8_ctx *ctx, int n, const int *M, int K, int N,
                                            const int8_t *const *A, const float *const *a_scale,
                                            const float *const *b_scale, float *const *Cf,
                                            rocket_i8_weights *const *w)
{
    return gw_grouped("rocket_matmul_int8_prepacked_gw_grouped", false, ctx, n, M, K, N,
                      reinterpret_cast<const void *const *>(A), a_scale, b_scale, Cf, w);
}

int rocket_matmul_int8_prepacked_gw_grouped_rowscale(rocket_i8_ctx *ctx, int n, const int *M, int K, int N,
                                                     const int8_t *const *A, const float *const *a_row_scale,
                                                     const float *const *b_scale, float *const *Cf,
                                                     rocket_i8_weights *const *w)
{
    return gw_grouped("rocket_matmul_int8_prepacked_gw_grouped_rowscale", true, ctx, n, M, K, N,
                      reinterpret_cast<const void *const *>(A), a_row_scale, b_scale, Cf, w);
}

int rocket_matmul_int8_prepacked_gw_rowscale(rocket_i8_ctx *ctx, int M, int K, int N, const int8_t *A,
                                             const float *a_row_scale, const float *b_scale, float *Cf,
                                             rocket_i8_weights *w)
{   // the checks of rocket_matmul_int8_prepacked_gw
    static const char *who = "rocket_matmul_int8_prepacked_gw_rowscale";
    if (!ctx || !w || !A || !a_row_scale || !b_scale || !Cf) return ROCKET_E_SHAPE;
    if (w->group <= 0) {
        ROCKET_LOGE("%s: weight is per-channel — use rocket_matmul_int8_prepacked\n", who);
        return ROCKET_E_SHAPE;
    }
    if (int rc = i8_resolve(ctx, who, M, K, N, w)) return rc;
    return gw_resident(ctx->fd, who, false, M, K, N, A, a_row_scale, b_scale, Cf, w->dev, w->group, nullptr, 0, 0,
                       true);
}

int rocket_matmul_int4_prepacked_gw_rowscale(rocket_i4_ctx *ctx, int M, int K, int N, const int8_t *A,
                                             const float *a_row_scale, const float *b_scale, float *Cf,
                                             rocket_i4_weights *w)
{   // the checks of rocket_matmul_int4_prepacked_gw
    static const char *who = "rocket_matmul_int4_prepacked_gw_rowscale";
    if (!ctx || !w || w->group <= 0) return ROCKET_E_SHAPE;
    if (!call_m_ok(who, M)) return ROCKET_E_SHAPE;
    if (K != w->K || N != w->N) {
        ROCKET_LOGE("%s: shape K=%d N=%d != packed %d/%d\n", who, K, N, w->K, w->N);
        return ROCKET_E_SHAPE;
    }
    return gw_resident(ctx->fd, who, true, M, K, N, A, a_row_scale, b_scale, Cf, w->dev, w->group, nullptr, 0, 0,
                       true);
}

int rocket_matmul_int8_prepacked_gw_rowscale_dump(rocket_i8_ctx *ctx, int M, int K, int N, const int8_t *A,
                                                  const float *a_row_scale, const float *b_scale, float *Cf,
                                                  rocket_i8_weights *w, int row0, int nrows, int32_t *P)
{   // the checks of rocket_matmul_int8_prepacked_gw_rowscale, then those of the dump
    static const char *who = "rocket_matmul_int8_prepacked_gw_rowscale_dump";
    if (!ctx || !w || w->group <= 0 || !A || !a_row_scale || !b_scale || !Cf) return ROCKET_E_SHAPE;
    if (int rc = i8_resolve(ctx, who, M, K, N, w)) return rc;
    if (!dump_args_ok(M, row0, nrows, P) || gw_period(w->group) != w->group) return ROCKET_E_SHAPE;
    return gw_resident(ctx->fd, who, false, M, K, N, A, a_row_scale, b_scale, Cf, w->dev, w->group, nrows ? P : nullptr,
                       row0, nrows, true);
}

int rocket_matmul_int4_prepacked_gw_rowscale_dump(rocket_i4_ctx *ctx, int M, int K, int N, const int8_t *A,
                                                  const float *a_row_scale, const float *b_scale, float *Cf,
                                                  rocket_i4_weights *w, int row0, int nrows, int32_t *P)
{   // the checks of rocket_matmul_int4_prepacked_gw_rowscale, then those of the dump
    static const char *who = "rocket_matmul_int4_prepacked_gw_rowscale_dump";
    if (!ctx || !w || w->group <= 0 || !A || !a_row_scale || !b_scale || !Cf) return ROCKET_E_SHAPE;
    if (!call_m_ok(who, M)) return ROCKET_E_SHAPE;
    if (K != w->K || N != w->N) return ROCKET_E_SHAPE;
    if (!dump_args_ok(M, row0, nrows, P)) return ROCKET_E_SHAPE;
    return gw_resident(ctx->fd, who, true, M, K, N, A, a_row_scale, b_scale, Cf, w->dev, w->group, nrows ? P : nullptr,
                       row0, nrows, true);
}

int rocket_matmul_int8_prepacked_gw_grouped_dump(rocket_i8_ctx *ctx, int n, const int *M, int K, int N,
                                                 const int8_t *const *A, const float *const *a_scale,
                                                 const float *const *b_scale, float *const *Cf,
                                                 rocket_i8_weights *const *w, const int *row0, const int *nrows,
                                                 int32_t *const *P)
{
    if (!P) return ROCKET_E_SHAPE;
    return gw_grouped("rocket_matmul_int8_prepacked_gw_grouped_dump", false, ctx, n, M, K, N,
                      reinterpret_cast<const void *const *>(A), a_scale, b_scale, Cf, w, 0, row0, nrows, P);
}

int rocket_matmul_int8_prepacked_gw_grouped_rowscale_dump(rocket_i8_ctx *ctx, int n, const int *M, int K, int N,
                                                          const int8_t *const *A, const float *const *a_row_scale,
                                                          const float *const *b_scale, float *const *Cf,
                                                          rocket_i8_weights *const *w, const int *row0,
                                                          const int *nrows, int32_t *const *P)
{
    if (!P) return ROCKET_E_SHAPE;
    return gw_grouped("rocket_matmul_int8_prepacked_gw_grouped_rowscale_dump", true, ctx, n, M, K, N,
                      reinterpret_cast<const void *const *>(A), a_row_scale, b_scale, Cf, w, 0, row0, nrows, P);
}

// =====================================================================================
// rocket_quant.h: resident group-wise products on fp32 activations, quantised per row on
// the device first (the *_rowscale entries' formula with that quantisation)
// =====================================================================================
int rocket_matmul_int8_prepacked_gw_f32in(rocket_i8_ctx *ctx, int M, int K, int N, const float *A,
                                          const float *b_scale, float *Cf, rocket_i8_weights *w)
{   // the checks of rocket_matmul_int8_prepacked_gw_rowscale
    static const char *who = "rocket_matmul_int8_prepacked_gw_f32in";
    if (!ctx || !w || !A || !b_scale || !Cf) return ROCKET_E_SHAPE;
    if (w->group <= 0) {
        ROCKET_LOGE("%s: weight is per-channel — use rocket_matmul_int8_prepacked\n", who);
        return ROCKET_E_SHAPE;
    }
    if (int rc = i8_resolve(ctx, who, M, K, N, w)) return rc;
    return gw_resident(ctx->fd, who, false, M, K, N, A, nullptr, b_scale, Cf, w->dev, w->group, nullptr, 0, 0,
                       true, 1);
}

int rocket_matmul_int4_prepacked_gw_f32in(rocket_i4_ctx *ctx, int M, int K, int N, const float *A,
                                          const float *b_scale, float *Cf, rocket_i4_weights *w)
{   // the checks of rocket_matmul_int4_prepacked_gw_rowscale
    static const char *who = "rocket_matmul_int4_prepacked_gw_f32in";
    if (!ctx || !w || w->group <= 0 || !A || !b_scale || !Cf) return ROCKET_E_SHAPE;
    if (!call_m_ok(who, M)) return ROCKET_E_SHAPE;
    if (K != w->K || N != w->N) {
        ROCKET_LOGE("%s: shape K=%d N=%d != packed %d/%d\n", who, K, N, w->K, w->N);
        return ROCKET_E_SHAPE;
    }
    return gw_resident(ctx->fd, who, true, M, K, N, A, nullptr, b_scale, Cf, w->dev, w->group, nullptr, 0, 0,
                       true, 1);
}

int rocket_matmul_int8_prepacked_gw_grouped_f32in(rocket_i8_ctx *ctx, int n, const int *M, int K, int N,
                                                  const float *const *A, const float *const *b_scale,
                                                  float *const *Cf, rocket_i8_weights *const *w)
{
    return gw_grouped("rocket_matmul_int8_prepacked_gw_grouped_f32in", true, ctx, n, M, K, N,
                      reinterpret_cast<const void *const *>(A), nullptr, b_scale, Cf, w, 1);
}

int rocket_matmul_int8_prepacked_gw_grouped_rowscale_f16out(rocket_i8_ctx *ctx, int n, const int *M, int K, int N,
                                                            const int8_t *const *A, const float *const *a_row_scale,
                                                            const float *const *b_scale, _Float16 *const *C,
                                                            rocket_i8_weights *const *w)
{
    return gw_grouped("rocket_matmul_int8_prepacked_gw_grouped_rowscale_f16out", true, ctx, n, M, K, N,
                      reinterpret_cast<const void *const *>(A), a_row_scale, b_scale,
                      reinterpret_cast<float *const *>(C), w, 0, nullptr, nullptr, nullptr, false, nullptr, 0, true);
}

int rocket_matmul_int8_prepacked_gw_grouped_glu_f16in(rocket_i8_ctx *ctx, int n, const int *M, int K, int N,
                                                      const _Float16 *const *gate, const _Float16 *const *up,
                                                      int act, const float *const *b_scale, float *const *Cf,
                                                      rocket_i8_weights *const *w)
{
    return gw_grouped("rocket_matmul_int8_prepacked_gw_grouped_glu_f16in", true, ctx, n, M, K, N,
                      reinterpret_cast<const void *const *>(gate), nullptr, b_scale, Cf, w, 2, nullptr, nullptr,
                      nullptr, true, reinterpret_cast<const void *const *>(up), act);
}

int rocket_matmul_int8_prepacked_gw_grouped_glu_f32in(rocket_i8_ctx *ctx, int n, const int *M, int K, int N,
                                                      const float *const *gate, const float *const *up, int act,
                                                      const float *const *b_scale, float *const *Cf,
                                                      rocket_i8_weights *const *w)
{
    return gw_grouped("rocket_matmul_int8_prepacked_gw_grouped_glu_f32in", true, ctx, n, M, K, N,
                      reinterpret_cast<const void *const *>(gate), nullptr, b_scale, Cf, w, 1, nullptr, nullptr,
                      nullptr, true, reinterpret_cast<const void *const *>(up), act);
}

}  // extern "C"
