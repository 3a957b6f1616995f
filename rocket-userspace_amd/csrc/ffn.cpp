// ffn.cpp — the gated-FFN and MLP blocks of rocket_ffn.h on the GPU (reference
// src/rocket_ffn.c). Each block is two kernel launches on the handle's stream: the first
// product with its activation epilogue (gate/up paired, or bias + activation), the second a
// plain fp16 product reading the intermediate from the handle's arena. fd < 0 runs the
// exact fp64 host paths of host_ref.cpp.
#include "host_ref.h"
#include "internal.h"
#include "rocket_ffn.h"

#include <limits.h>
#include <math.h>
#include <vector>

using namespace rk;

namespace {

bool kind_ok(int kind) { return kind == ROCKET_ACTIVATION_SILU || kind == ROCKET_ACTIVATION_GELU; }
bool rows_ok(int M) { return M == 1 || (M > 0 && M % 4 == 0); }

size_t h16(size_t n) { return n * sizeof(_Float16); }

// A plain fp16 product out = A W^T (A[M, K], W[N, K]) as one launch; its split-K workspace
// (if the plan takes one) is requested with want_ws before the call's begin().
struct F16Product {
    Launch L;
    size_t ws = 0;
    F16Product(int M, int K, int N)
    {
        L.fmt_a = L.fmt_b = Fmt::F16;
        L.epi = Epi::F16;
        L.N = N;
        L.K = K;
        L.kbeg = 0;
        L.kend = K;
        L.nprob = 1;
        L.prob[0].M = M;
        ws = gemm_ws_bytes(L);
    }
    void want_ws(Call &c) const { c.want_scratch(ws); }
    int run(Call &c, const void *A, const void *W, void *out)
    {
        L.prob[0] = Problem{L.prob[0].M, A, W, out, nullptr, nullptr, nullptr};
        L.ws = ws ? static_cast<int32_t *>(c.scratch(ws)) : nullptr;
        L.ws_bytes = L.ws ? ws : 0;
        return c.launch(L);
    }
};

// gate/up with the gated epilogue into arena scratch, then the down product.
int ffn_gpu(int fd, const char *who, int M, int H, int I, const _Float16 *x, const _Float16 *Wg,
            const _Float16 *Wu, const _Float16 *Wd, int kind, _Float16 *out)
{
    Locked L(fd);
    if (!L.ok()) {
        ROCKET_LOGE("%s: fd %d is not an open rocket handle\n", who, fd);
        return ROCKET_E_DEVICE;
    }
    Call c(L.h, who);
    c.want(x, h16((size_t)M * H));
    c.want(Wg, h16((size_t)I * H));
    c.want(Wu, h16((size_t)I * H));
    c.want(Wd, h16((size_t)H * I));
    c.want(out, h16((size_t)M * H));
    c.want_scratch(h16((size_t)M * I));
    F16Product down(M, I, H);
    down.want_ws(c);
    if (int rc = c.begin()) return rc;
    const void *dx = c.in(x, h16((size_t)M * H));
    const void *dg = c.in(Wg, h16((size_t)I * H));
    const void *du = c.in(Wu, h16((size_t)I * H));
    const void *dd = c.in(Wd, h16((size_t)H * I));
    void *dout = c.out(out, h16((size_t)M * H));
    void *prod = c.scratch(h16((size_t)M * I));
    if (!dx || !dg || !du || !dd || !dout || !prod) return c.finish();

    Launch a;
    a.fmt_a = a.fmt_b = Fmt::F16;
    a.epi = Epi::GLU;
    a.N = 2 * I;
    a.K = H;
    a.kbeg = 0;
    a.kend = H;
    a.act = kind;
    a.nprob = 1;
    a.prob[0] = Problem{M, dx, dg, prod, nullptr, nullptr, du};
    if (c.launch(a)) return c.finish();
    if (down.run(c, prod, dd, dout)) return c.finish();
    return c.finish();
}

int ffn_entry(int fd, const char *who, int M, int H, int I, const _Float16 *x, const _Float16 *Wg,
              const _Float16 *Wu, const _Float16 *Wd, int kind, _Float16 *out)
{
    // reference rocket_ffn.c:87-92
    if (M < 1 || H < 1 || I < 1) return ROCKET_E_SHAPE;
    if ((size_t)M * I > INT_MAX) return ROCKET_E_SHAPE;
    if (fd < 0) return ffn_ref_fp16(M, H, I, x, Wg, Wu, Wd, kind, out) ? ROCKET_OK : ROCKET_E_NOMEM;
    if (!x || !Wg || !Wu || !Wd || !out) return ROCKET_E_SHAPE;
    if (!kind_ok(kind)) {
        ROCKET_LOGE("%s: activation kind %d (SiLU or GELU only)\n", who, kind);
        return ROCKET_E_SHAPE;
    }
    if (!rows_ok(M) || H % 32 || I % 32 || H > (1 << 24) || I > (1 << 24)) {
        ROCKET_LOGE("%s: unsupported shape M=%d H=%d I=%d (need H%%32, I%%32, M%%4||1)\n", who, M, H, I);
        return ROCKET_E_SHAPE;
    }
    return ffn_gpu(fd, who, M, H, I, x, Wg, Wu, Wd, kind, out);
}

}  // namespace

extern "C" {

int rocket_geglu_fp16(int fd, const _Float16 *gate, const _Float16 *up, int kind, _Float16 *prod, int n)
{   // reference rocket_ffn.c:40-54
    if (n <= 0) return ROCKET_E_SHAPE;
    if (fd < 0) {
        rocket_geglu_ref_fp16(gate, up, kind, prod, n);
        return ROCKET_OK;
    }
    if (!gate || !up || !prod || !kind_ok(kind)) return ROCKET_E_SHAPE;
    Locked L(fd);
    if (!L.ok()) return ROCKET_E_DEVICE;
    Call c(L.h, "rocket_geglu_fp16");
    c.want(gate, h16((size_t)n));
    c.want(up, h16((size_t)n));
    c.want(prod, h16((size_t)n));
    if (int rc = c.begin()) return rc;
    const void *dg = c.in(gate, h16((size_t)n));
    const void *du = c.in(up, h16((size_t)n));
    void *dp = c.out(prod, h16((size_t)n));
    if (!dg || !du || !dp) return c.finish();
    if (geglu_f16(static_cast<const _Float16 *>(dg), static_cast<const _Float16 *>(du), static_cast<_Float16 *>(dp),
                  n, kind, c.stream()) != hipSuccess) {
        (void)hipGetLastError();
        ROCKET_LOGE("rocket_geglu_fp16: kernel launch rejected\n");
        (void)c.finish();
        return ROCKET_E_DEVICE;
    }
    count_launch((uint64_t)((n + 2047) / 2048));
    return c.finish();
}

int rocket_ffn_fp16(int fd, int M, int H, int I, const _Float16 *x, const _Float16 *Wg, const _Float16 *Wu,
                    const _Float16 *Wd, int kind, _Float16 *out)
{   // reference rocket_ffn.c:84-121
    return ffn_entry(fd, "rocket_ffn_fp16", M, H, I, x, Wg, Wu, Wd, kind, out);
}

int rocket_ffn_fp16_fused(int fd, int M, int H, int I, const _Float16 *x, const _Float16 *Wg, const _Float16 *Wu,
                          const _Float16 *Wd, int kind, _Float16 *out)
{   // reference rocket_ffn.c:125-211 (its intermediates stay on the device: so do these)
    return ffn_entry(fd, "rocket_ffn_fp16_fused", M, H, I, x, Wg, Wu, Wd, kind, out);
}

int rocket_mlp_fp16_fused(int fd, int M, int Din, int Dff, int Dout, const _Float16 *x, const _Float16 *W1,
                          const _Float16 *b1, const _Float16 *W2, int kind, _Float16 *out)
{   // reference rocket_ffn.c:268-330
    if (M < 1 || Din < 1 || Dff < 1 || Dout < 1) return ROCKET_E_SHAPE;
    if ((size_t)M * Dff > INT_MAX) return ROCKET_E_SHAPE;
    if (fd < 0)   // the exact host path (host_ref.cpp)
        return mlp_ref_fp16(M, Din, Dff, Dout, x, W1, b1, W2, kind, out) ? ROCKET_OK : ROCKET_E_NOMEM;
    if (!x || !W1 || !W2 || !out) return ROCKET_E_SHAPE;
    if (!kind_ok(kind)) {
        ROCKET_LOGE("rocket_mlp_fp16_fused: activation kind %d (SiLU or GELU only)\n", kind);
        return ROCKET_E_SHAPE;
    }
    if (!rows_ok(M) || Din % 32 || Dff % 32 || Dout % 16 || Din > (1 << 24) || Dff > (1 << 24) || Dout > (1 << 24)) {
        ROCKET_LOGE("rocket_mlp_fp16_fused: unsupported shape M=%d Din=%d Dff=%d Dout=%d\n", M, Din, Dff, Dout);
        return ROCKET_E_SHAPE;
    }
    Locked L(fd);
    if (!L.ok()) return ROCKET_E_DEVICE;
    Call c(L.h, "rocket_mlp_fp16_fused");
    c.want(x, h16((size_t)M * Din));
    c.want(W1, h16((size_t)Dff * Din));
    if (b1) c.want(b1, h16((size_t)Dff));
    c.want(W2, h16((size_t)Dout * Dff));
    c.want(out, h16((size_t)M * Dout));
    c.want_scratch(h16((size_t)M * Dff));
    F16Product fc2(M, Dff, Dout);
    fc2.want_ws(c);
    if (int rc = c.begin()) return rc;
    const void *dx = c.in(x, h16((size_t)M * Din));
    const void *d1 = c.in(W1, h16((size_t)Dff * Din));
    const void *db = b1 ? c.in(b1, h16((size_t)Dff)) : nullptr;
    const void *d2 = c.in(W2, h16((size_t)Dout * Dff));
    void *dout = c.out(out, h16((size_t)M * Dout));
    void *act = c.scratch(h16((size_t)M * Dff));
    if (!dx || !d1 || (b1 && !db) || !d2 || !dout || !act) return c.finish();

    Launch a;
    a.fmt_a = a.fmt_b = Fmt::F16;
    a.epi = Epi::ACT;
    a.N = Dff;
    a.K = Din;
    a.kbeg = 0;
    a.kend = Din;
    a.act = kind;
    a.nprob = 1;
    a.prob[0] = Problem{M, dx, d1, act, nullptr, nullptr, db};
    if (c.launch(a)) return c.finish();
    if (fc2.run(c, act, d2, dout)) return c.finish();
    return c.finish();
}

}  // extern "C"
