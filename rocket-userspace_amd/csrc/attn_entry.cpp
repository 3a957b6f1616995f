// attn_entry.cpp — rocket_attn.h on the GPU (reference src/rocket_attn.c): argument checks,
// the fused attention kernel (attn.hip) and the projection GEMMs. fd < 0 runs the fp64 host
// references of host_ref.cpp.
#include "attn.h"
#include "host_ref.h"
#include "ops.h"
#include "rocket_attn.h"

#include <math.h>

#include <new>
#include <vector>

using namespace rk;

struct rocket_fa_ctx { int fd; int nthreads; };

namespace {

size_t h16(size_t n) { return n * sizeof(_Float16); }
int round_up(int x, int m) { return (x + m - 1) / m * m; }

// reference rocket_attn.c:733-734 (the same checks in every flash entry)
bool fa_args_ok(int n_tokens, int n_kv, int head_dim, int dv, int n_head, int n_kv_heads)
{
    if (n_tokens < 1 || n_kv < 1 || head_dim < 1 || dv < 1 || n_head < 1 || n_kv_heads < 1) return false;
    return n_head % n_kv_heads == 0 && head_dim % 32 == 0 && dv % 16 == 0;
}

int fa_gpu(int fd, const char *who, int T, int n_kv, int dk, int dv, int n_head, int n_kv_heads, float scale,
           float softcap, const _Float16 *Q, const _Float16 *K, const _Float16 *V, const _Float16 *mask, _Float16 *out)
{
    if (!Q || !K || !V || !out) return ROCKET_E_SHAPE;
    if (dk > kAttnMaxHeadDim || dv > kAttnMaxHeadDim) {
        ROCKET_LOGE("%s: head_dim %d / dv %d above %d\n", who, dk, dv, kAttnMaxHeadDim);
        return ROCKET_E_SHAPE;
    }
    Locked L(fd);
    if (!L.ok()) {
        ROCKET_LOGE("%s: fd %d is not an open rocket handle\n", who, fd);
        return ROCKET_E_DEVICE;
    }
    const size_t nq = (size_t)n_head * T * dk, nk = (size_t)n_kv_heads * n_kv * dk;
    const size_t nv = (size_t)n_kv_heads * dv * n_kv, no = (size_t)n_head * T * dv, nm = (size_t)T * n_kv;
    // V^T rows padded to a multiple of 64 keys (zeros) unless they already are
    const int n_kvp = round_up(n_kv, 64);
    const bool pad = n_kvp != n_kv;
    FaLaunch f;
    f.T = T; f.n_kv = n_kv; f.dk = dk; f.dv = dv; f.n_head = n_head; f.gqa = n_head / n_kv_heads;
    f.scale = scale; f.softcap = softcap;
    const size_t ws = flash_attn_ws_bytes(f);
    Call c(L.h, who);
    if (ws) c.want_scratch(ws);
    c.want(Q, h16(nq));
    c.want(K, h16(nk));
    c.want(V, h16(nv));
    if (mask) c.want(mask, h16(nm));
    c.want(out, h16(no));
    if (pad) c.want_scratch(h16((size_t)n_kv_heads * dv * n_kvp));
    if (int rc = c.begin()) return rc;
    f.ws = ws ? static_cast<float *>(c.scratch(ws)) : nullptr;
    f.ws_bytes = f.ws ? ws : 0;
    f.Q = static_cast<const _Float16 *>(c.in(Q, h16(nq)));
    f.K = static_cast<const _Float16 *>(c.in(K, h16(nk)));
    const _Float16 *dV = static_cast<const _Float16 *>(c.in(V, h16(nv)));
    f.mask = mask ? static_cast<const _Float16 *>(c.in(mask, h16(nm))) : nullptr;
    f.O = static_cast<_Float16 *>(c.out(out, h16(no)));
    if (!f.Q || !f.K || !dV || (mask && !f.mask) || !f.O) return c.finish();
    if (pad) {
        _Float16 *vp = static_cast<_Float16 *>(c.scratch(h16((size_t)n_kv_heads * dv * n_kvp)));
        if (!vp) return c.finish();
        if (pad_cols_f16(dV, n_kv, vp, (long)n_kv_heads * dv, n_kv, n_kvp, c.stream()) != hipSuccess) {
            (void)hipGetLastError();
            ROCKET_LOGE("%s: V pad launch rejected\n", who);
            (void)c.finish();
            return ROCKET_E_DEVICE;
        }
        count_launch((uint64_t)(((size_t)n_kv_heads * dv * n_kvp + 255) / 256));
        dV = vp;
    }
    f.Vt = dV;
    f.q_hs = (long)T * dk; f.q_rs = dk;
    f.k_hs = (long)n_kv * dk; f.k_rs = dk;
    f.v_hs = (long)dv * n_kvp; f.v_rs = n_kvp;
    f.o_hs = (long)T * dv; f.o_rs = dv;
    f.m_rs = n_kv;
    uint64_t blocks = 0;
    if (flash_attn(f, c.stream(), &blocks) != hipSuccess) {
        (void)hipGetLastError();
        ROCKET_LOGE("%s: attention launch rejected (T=%d n_kv=%d dk=%d dv=%d)\n", who, T, n_kv, dk, dv);
        (void)c.finish();
        return ROCKET_E_SHAPE;
    }
    count_launch(blocks);
    return c.finish();
}

}  // namespace

extern "C" {

int rocket_flash_attn_fp16(int fd, int n_tokens, int n_kv, int head_dim, int dv, int n_head, int n_kv_heads,
                           float scale, float softcap, const _Float16 *Q, const _Float16 *K, const _Float16 *V,
                           const _Float16 *mask, _Float16 *out)
{   // reference rocket_attn.c:728-745
    if (!fa_args_ok(n_tokens, n_kv, head_dim, dv, n_head, n_kv_heads)) return ROCKET_E_SHAPE;
    if (fd < 0)
        return flash_attn_ref_fp16(n_tokens, n_kv, head_dim, dv, n_head, n_kv_heads, scale, softcap, Q, K, V, mask,
                                   out)
                   ? ROCKET_OK
                   : ROCKET_E_NOMEM;
    return fa_gpu(fd, "rocket_flash_attn_fp16", n_tokens, n_kv, head_dim, dv, n_head, n_kv_heads, scale, softcap, Q,
                  K, V, mask, out);
}

int rocket_flash_attn_fp16_mt(int fd, int n_tokens, int n_kv, int head_dim, int dv, int n_head, int n_kv_heads,
                              float scale, float softcap, const _Float16 *Q, const _Float16 *K, const _Float16 *V,
                              const _Float16 *mask, _Float16 *out, int nthreads)
{   // reference rocket_attn.c:842-871: the heads are independent; here one launch runs them all
    (void)nthreads;
    return rocket_flash_attn_fp16(fd, n_tokens, n_kv, head_dim, dv, n_head, n_kv_heads, scale, softcap, Q, K, V,
                                  mask, out);
}

rocket_fa_ctx *rocket_fa_ctx_create(int nthreads)
{   // reference rocket_attn.c:886-913: NULL when the device cannot be opened
    const int fd = rocket_open();
    if (fd < 0) return nullptr;
    rocket_fa_ctx *c = new (std::nothrow) rocket_fa_ctx{fd, nthreads < 1 ? 1 : (nthreads > 8 ? 8 : nthreads)};
    if (!c) rocket_close(fd);
    return c;
}

void rocket_fa_ctx_free(rocket_fa_ctx *c)
{
    if (!c) return;
    rocket_close(c->fd);
    delete c;
}

int rocket_flash_attn_fp16_ctx(rocket_fa_ctx *c, int n_tokens, int n_kv, int head_dim, int dv, int n_head,
                               int n_kv_heads, float scale, float softcap, const _Float16 *Q, const _Float16 *K,
                               const _Float16 *V, const _Float16 *mask, _Float16 *out)
{   // reference rocket_attn.c:925-949
    if (!c) return ROCKET_E_SHAPE;
    if (!fa_args_ok(n_tokens, n_kv, head_dim, dv, n_head, n_kv_heads)) return ROCKET_E_SHAPE;
    return fa_gpu(c->fd, "rocket_flash_attn_fp16_ctx", n_tokens, n_kv, head_dim, dv, n_head, n_kv_heads, scale,
                  softcap, Q, K, V, mask, out);
}

int rocket_mha_self_fp16(int fd, int T, int d, int n_head, const _Float16 *x, const _Float16 *Wq, const _Float16 *bq,
                         const _Float16 *Wk, const _Float16 *bk, const _Float16 *Wv, const _Float16 *bv,
                         const _Float16 *Wo, const _Float16 *bo, _Float16 *out)
{   // reference rocket_attn.c:92-172
    static const char *who = "rocket_mha_self_fp16";
    if (T < 1 || d < 1 || n_head < 1 || d % n_head) return ROCKET_E_SHAPE;
    if (fd < 0) return mha_self_ref_fp16(T, d, n_head, x, Wq, bq, Wk, bk, Wv, bv, Wo, bo, out) ? ROCKET_OK : ROCKET_E_NOMEM;
    const int dh = d / n_head;
    if (!x || !Wq || !Wk || !Wv || !Wo || !out) return ROCKET_E_SHAPE;
    if (d % 32 || dh % 16 || dh > kAttnMaxHeadDim || d > kDimMax || T > kDimMax) {
        ROCKET_LOGE("%s: unsupported shape T=%d d=%d n_head=%d (need d%%32, d_head%%16, d_head<=%d)\n", who, T, d,
                    n_head, kAttnMaxHeadDim);
        return ROCKET_E_SHAPE;
    }
    Locked L(fd);
    if (!L.ok()) {
        ROCKET_LOGE("%s: fd %d is not an open rocket handle\n", who, fd);
        return ROCKET_E_DEVICE;
    }
    const size_t Td = (size_t)T * d, dd = (size_t)d * d;
    const int Tp = round_up(T, 64);
    Call c(L.h, who);
    c.want(x, h16(Td));
    for (const _Float16 *w : {Wq, Wk, Wv, Wo}) c.want(w, h16(dd));
    for (const _Float16 *b : {bq, bk, bv, bo})
        if (b) c.want(b, h16((size_t)d));
    c.want(out, h16(Td));
    c.want_scratch(h16(3 * Td));              // q, k, v (token-major)
    c.want_scratch(h16((size_t)d * Tp));      // v per head, transposed and padded
    c.want_scratch(h16(Td));                  // the heads' context (token-major)
    FaLaunch f;
    f.T = T; f.n_kv = T; f.dk = dh; f.dv = dh; f.n_head = n_head; f.gqa = 1;
    f.scale = (float)(1.0 / sqrt((double)dh));
    f.softcap = 0.f;
    const size_t ws = flash_attn_ws_bytes(f);
    if (ws) c.want_scratch(ws);
    if (int rc = c.begin()) return rc;
    const void *dx = c.in(x, h16(Td));
    const void *dW[4], *dB[4];
    const _Float16 *Ws[4] = {Wq, Wk, Wv, Wo}, *Bs[4] = {bq, bk, bv, bo};
    for (int i = 0; i < 4; i++) {
        dW[i] = c.in(Ws[i], h16(dd));
        dB[i] = Bs[i] ? c.in(Bs[i], h16((size_t)d)) : nullptr;
        if (!dW[i] || (Bs[i] && !dB[i])) return c.finish();
    }
    void *dout = c.out(out, h16(Td));
    _Float16 *qkv = static_cast<_Float16 *>(c.scratch(h16(3 * Td)));
    _Float16 *vt = static_cast<_Float16 *>(c.scratch(h16((size_t)d * Tp)));
    _Float16 *ctx = static_cast<_Float16 *>(c.scratch(h16(Td)));
    if (!dx || !dout || !qkv || !vt || !ctx) return c.finish();

    // q, k, v = x W^T + b: one launch of three problems, the bias in the epilogue
    Launch p;
    p.fmt_a = p.fmt_b = Fmt::F16;
    p.epi = Epi::ACT;
    p.act = kActIdentity;
    p.N = d;
    p.K = d;
    p.kbeg = 0;
    p.kend = d;
    p.nprob = 3;
    for (int i = 0; i < 3; i++) p.prob[i] = Problem{T, dx, dW[i], qkv + i * Td, nullptr, nullptr, dB[i]};
    if (c.launch(p)) return c.finish();
    // v per head as [h][dh][Tp]
    if (heads_transpose_f16(qkv + 2 * Td, vt, T, n_head, dh, Tp, c.stream()) != hipSuccess) {
        (void)hipGetLastError();
        (void)c.finish();
        return ROCKET_E_DEVICE;
    }
    count_launch(((size_t)d * Tp + 255) / 256);
    // attention over the heads, context written token-major
    f.Q = qkv; f.q_hs = dh; f.q_rs = d;
    f.K = qkv + Td; f.k_hs = dh; f.k_rs = d;
    f.Vt = vt; f.v_hs = (long)dh * Tp; f.v_rs = Tp;
    f.O = ctx; f.o_hs = dh; f.o_rs = d;
    f.ws = ws ? static_cast<float *>(c.scratch(ws)) : nullptr;
    f.ws_bytes = f.ws ? ws : 0;
    uint64_t blocks = 0;
    if (flash_attn(f, c.stream(), &blocks) != hipSuccess) {
        (void)hipGetLastError();
        (void)c.finish();
        return ROCKET_E_DEVICE;
    }
    count_launch(blocks);
    // out = ctx Wo^T + bo
    Launch o = p;
    o.nprob = 1;
    o.prob[0] = Problem{T, ctx, dW[3], dout, nullptr, nullptr, dB[3]};
    if (c.launch(o)) return c.finish();
    return c.finish();
}

}  // extern "C"
