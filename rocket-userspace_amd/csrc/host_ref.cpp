// host_ref.cpp — the exact fp64 host paths of rocket_ffn.h and rocket_attn.h (fd < 0).
//
// The contracts these follow (reference src/rocket_ffn.c:23-82, :236-254 and
// src/rocket_attn.c:41-84, :181-228, as the public headers state them):
//   * every product is an fp64 sum over the contraction index in ascending order;
//   * the gated FFN applies act(gate) * up in fp64 and rounds only its output to fp16;
//   * the MLP starts each first-layer sum at its bias and rounds the activation to fp16;
//   * flash attention forms each score in fp32 (scale, soft-cap, mask, clamp at -30000),
//     then an fp64 softmax and P·V scaled by 1/sum; self-attention keeps the whole chain
//     in fp64 (scores scaled by d_head^-1/2, P·V divided by the sum) and adds each
//     projection's bias after its products.
// The code is organised around widened operand matrices: each fp16 operand is converted
// once, linear layers run over blocks of four rows sharing each weight row, and attention
// runs over blocks of queries that share one pass over the keys.
#include "host_ref.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <new>
#include <vector>

#include "rocket_activation.h"
#include "rocket_attn.h"
#include "rocket_ffn.h"

namespace rk {
namespace hostref {

Mat::Mat(int r, int c) : rows(r), cols(c), data(new double[(size_t)r * c]()) {}
Mat::Mat(Mat &&o) noexcept : rows(o.rows), cols(o.cols), data(o.data) { o.data = nullptr; o.rows = o.cols = 0; }
Mat &Mat::operator=(Mat &&o) noexcept
{
    if (this != &o) {
        delete[] data;
        rows = o.rows; cols = o.cols; data = o.data;
        o.data = nullptr; o.rows = o.cols = 0;
    }
    return *this;
}
Mat::~Mat() { delete[] data; }

Mat widen(const _Float16 *p, int rows, int cols, bool transposed)
{
    Mat m(transposed ? cols : rows, transposed ? rows : cols);
    for (int r = 0; r < rows; r++) {
        const _Float16 *src = p + (size_t)r * cols;
        if (transposed)
            for (int c = 0; c < cols; c++) m.row(c)[r] = (double)src[c];
        else
            for (int c = 0; c < cols; c++) m.row(r)[c] = (double)src[c];
    }
    return m;
}

Mat linear(const Mat &x, const Mat &w, const _Float16 *b, Bias at)
{
    const int R = x.rows, O = w.rows, D = x.cols;
    Mat y(R, O);
    constexpr int RB = 4;   // rows sharing one pass over each weight row
    for (int r0 = 0; r0 < R; r0 += RB) {
        const int nr = std::min(RB, R - r0);
        for (int o = 0; o < O; o++) {
            const double *wr = w.row(o);
            const double start = (b && at == Bias::First) ? (double)b[o] : 0.0;
            double acc[RB] = {start, start, start, start};
            for (int i = 0; i < D; i++) {
                const double wi = wr[i];
                for (int k = 0; k < nr; k++) acc[k] += x.row(r0 + k)[i] * wi;
            }
            for (int k = 0; k < nr; k++)
                y.row(r0 + k)[o] = (b && at == Bias::Last) ? acc[k] + (double)b[o] : acc[k];
        }
    }
    return y;
}

double activation(int kind, double g)
{
    if (kind == ROCKET_ACTIVATION_GELU) return 0.5 * g * (1.0 + erf(g * 0.70710678118654752440));
    return g / (1.0 + exp(-g));
}

namespace {

// One head of softmax attention over a block of queries. q: [nq, dk] rows of this block,
// keys: [n_kv, dk], vt: values key-major [n_kv, dv]. score(t, j, qk) maps the fp64 dot of
// query t (block-relative) and key j to the score; NORM_MUL scales the weighted sum by
// 1/sum (0 when the sum is 0), otherwise divides it by the sum. out(t, c, value).
template <bool NORM_MUL, class Score, class Out>
void attend_block(const double *q, int nq, int dk, const Mat &keys, const Mat &vt, Score score, Out out)
{
    const int n_kv = keys.rows, dv = vt.cols;
    std::vector<double> s((size_t)nq * n_kv), o((size_t)dv);
    std::vector<double> mx((size_t)nq, -INFINITY);
    // scores: one pass over the keys serves every query of the block
    for (int j = 0; j < n_kv; j++) {
        const double *kr = keys.row(j);
        for (int t = 0; t < nq; t++) {
            const double *qr = q + (size_t)t * dk;
            double qk = 0;
            for (int c = 0; c < dk; c++) qk += qr[c] * kr[c];
            const double v = score(t, j, qk);
            s[(size_t)t * n_kv + j] = v;
            mx[(size_t)t] = std::max(mx[(size_t)t], v);
        }
    }
    for (int t = 0; t < nq; t++) {
        double *st = s.data() + (size_t)t * n_kv;
        double sum = 0;
        for (int j = 0; j < n_kv; j++) {
            st[j] = exp(st[j] - mx[(size_t)t]);
            sum += st[j];
        }
        // weighted values, accumulated key by key (each output column in ascending key order)
        std::fill(o.begin(), o.end(), 0.0);
        for (int j = 0; j < n_kv; j++) {
            const double *vr = vt.row(j);
            const double p = st[j];
            for (int c = 0; c < dv; c++) o[(size_t)c] += p * vr[c];
        }
        if (NORM_MUL) {
            const double inv = sum > 0 ? 1.0 / sum : 0.0;
            for (int c = 0; c < dv; c++) out(t, c, o[(size_t)c] * inv);
        } else {
            for (int c = 0; c < dv; c++) out(t, c, o[(size_t)c] / sum);
        }
    }
}

constexpr int kQueryBlock = 16;

// The fp32 score steps of the flash entries: scale, optional soft-cap, additive mask, clamp.
struct FlashScore {
    float scale, softcap;
    float operator()(double qk, float mask) const
    {
        float v = (float)qk * scale;
        if (softcap != 0.0f) v = softcap * tanhf(v / softcap);
        v += mask;
        return std::max(v, -30000.0f);
    }
};

}  // namespace
}  // namespace hostref

namespace {

// Runs f; false when it ran out of host memory (the fp64 operand copies are the large
// allocations). Nothing may throw across the C ABI, so the entries turn this into a return.
template <class F> bool no_throw(F &&f) noexcept
{
    try {
        f();
        return true;
    } catch (const std::bad_alloc &) {
        return false;
    }
}

void mlp_ref_impl(int M, int Din, int Dff, int Dout, const _Float16 *x, const _Float16 *W1, const _Float16 *b1,
                  const _Float16 *W2, int kind, _Float16 *out)
{
    using namespace hostref;
    const Mat xs = widen(x, M, Din), w1 = widen(W1, Dff, Din), w2 = widen(W2, Dout, Dff);
    Mat h = linear(xs, w1, b1, Bias::First);
    // the activation is stored as fp16 before the second layer reads it
    for (int m = 0; m < M; m++)
        for (int o = 0; o < Dff; o++) h.row(m)[o] = (double)(_Float16)activation(kind, h.row(m)[o]);
    const Mat y = linear(h, w2, nullptr, Bias::Last);
    for (int m = 0; m < M; m++)
        for (int o = 0; o < Dout; o++) out[(size_t)m * Dout + o] = (_Float16)y.row(m)[o];
}

using namespace hostref;

void ffn_ref_impl(int M, int H, int I, const _Float16 *x, const _Float16 *Wg, const _Float16 *Wu, const _Float16 *Wd,
                  int kind, _Float16 *out)
{
    const Mat xs = widen(x, M, H);
    const Mat g = linear(xs, widen(Wg, I, H), nullptr, Bias::Last);
    Mat u = linear(xs, widen(Wu, I, H), nullptr, Bias::Last);
    for (int m = 0; m < M; m++)   // u becomes the gated product act(g) * u, kept in fp64
        for (int i = 0; i < I; i++) u.row(m)[i] = activation(kind, g.row(m)[i]) * u.row(m)[i];
    const Mat y = linear(u, widen(Wd, H, I), nullptr, Bias::Last);
    for (int m = 0; m < M; m++)
        for (int h = 0; h < H; h++) out[(size_t)m * H + h] = (_Float16)y.row(m)[h];
}

void flash_attn_ref_impl(int n_tokens, int n_kv, int head_dim, int dv, int n_head, int n_kv_heads, float scale,
                         float softcap, const _Float16 *Q, const _Float16 *K, const _Float16 *V, const _Float16 *mask,
                         _Float16 *out)
{
    const int per_kv = n_head / n_kv_heads;
    const FlashScore rule{scale, softcap};
    for (int hk = 0; hk < n_kv_heads; hk++) {
        // this KV head's keys [n_kv, dk] and values made key-major [n_kv, dv], once
        const Mat keys = widen(K + (size_t)hk * n_kv * head_dim, n_kv, head_dim);
        const Mat vt = widen(V + (size_t)hk * dv * n_kv, dv, n_kv, true);
        for (int h = hk * per_kv; h < (hk + 1) * per_kv; h++) {
            const Mat qh = widen(Q + (size_t)h * n_tokens * head_dim, n_tokens, head_dim);
            _Float16 *oh = out + (size_t)h * n_tokens * dv;
            for (int t0 = 0; t0 < n_tokens; t0 += kQueryBlock) {
                const int nq = std::min(kQueryBlock, n_tokens - t0);
                auto score = [&](int t, int j, double qk) -> double {
                    return rule(qk, mask ? (float)mask[(size_t)(t0 + t) * n_kv + j] : 0.0f);
                };
                auto put = [&](int t, int c, double v) { oh[(size_t)(t0 + t) * dv + c] = (_Float16)v; };
                attend_block<true>(qh.row(t0), nq, head_dim, keys, vt, score, put);
            }
        }
    }
}

void mha_self_ref_impl(int T, int d, int n_head, const _Float16 *x, const _Float16 *Wq, const _Float16 *bq,
                       const _Float16 *Wk, const _Float16 *bk, const _Float16 *Wv, const _Float16 *bv,
                       const _Float16 *Wo, const _Float16 *bo, _Float16 *out)
{
    const int dh = d / n_head;
    const double scale = 1.0 / sqrt((double)dh);
    const Mat xs = widen(x, T, d);
    const Mat q = linear(xs, widen(Wq, d, d), bq, Bias::Last);
    const Mat k = linear(xs, widen(Wk, d, d), bk, Bias::Last);
    const Mat v = linear(xs, widen(Wv, d, d), bv, Bias::Last);
    Mat ctx(T, d);
    for (int h = 0; h < n_head; h++) {
        // the head's columns as their own matrices
        Mat qh(T, dh), kh(T, dh), vh(T, dh);
        for (int t = 0; t < T; t++) {
            memcpy(qh.row(t), q.row(t) + (size_t)h * dh, sizeof(double) * dh);
            memcpy(kh.row(t), k.row(t) + (size_t)h * dh, sizeof(double) * dh);
            memcpy(vh.row(t), v.row(t) + (size_t)h * dh, sizeof(double) * dh);
        }
        for (int t0 = 0; t0 < T; t0 += kQueryBlock) {
            const int nq = std::min(kQueryBlock, T - t0);
            auto score = [&](int, int, double qk) -> double { return qk * scale; };
            auto put = [&](int t, int c, double val) { ctx.row(t0 + t)[(size_t)h * dh + c] = val; };
            attend_block<false>(qh.row(t0), nq, dh, kh, vh, score, put);
        }
    }
    const Mat y = linear(ctx, widen(Wo, d, d), bo, Bias::Last);
    for (int t = 0; t < T; t++)
        for (int o = 0; o < d; o++) out[(size_t)t * d + o] = (_Float16)y.row(t)[o];
}

}  // namespace

bool mlp_ref_fp16(int M, int Din, int Dff, int Dout, const _Float16 *x, const _Float16 *W1, const _Float16 *b1,
                  const _Float16 *W2, int kind, _Float16 *out)
{
    return no_throw([&] { mlp_ref_impl(M, Din, Dff, Dout, x, W1, b1, W2, kind, out); });
}

bool ffn_ref_fp16(int M, int H, int I, const _Float16 *x, const _Float16 *Wg, const _Float16 *Wu, const _Float16 *Wd,
                  int kind, _Float16 *out)
{
    return no_throw([&] { ffn_ref_impl(M, H, I, x, Wg, Wu, Wd, kind, out); });
}

bool flash_attn_ref_fp16(int n_tokens, int n_kv, int head_dim, int dv, int n_head, int n_kv_heads, float scale,
                         float softcap, const _Float16 *Q, const _Float16 *K, const _Float16 *V, const _Float16 *mask,
                         _Float16 *out)
{
    return no_throw([&] {
        flash_attn_ref_impl(n_tokens, n_kv, head_dim, dv, n_head, n_kv_heads, scale, softcap, Q, K, V, mask, out);
    });
}

bool mha_self_ref_fp16(int T, int d, int n_head, const _Float16 *x, const _Float16 *Wq, const _Float16 *bq,
                       const _Float16 *Wk, const _Float16 *bk, const _Float16 *Wv, const _Float16 *bv,
                       const _Float16 *Wo, const _Float16 *bo, _Float16 *out)
{
    return no_throw([&] { mha_self_ref_impl(T, d, n_head, x, Wq, bq, Wk, bk, Wv, bv, Wo, bo, out); });
}

}  // namespace rk

// The public host references return early when host memory runs out, leaving out untouched
// (the reference's host paths do the same on a failed malloc).
extern "C" {

void rocket_geglu_ref_fp16(const _Float16 *gate, const _Float16 *up, int kind, _Float16 *prod, int n)
{
    for (int i = 0; i < n; i++)
        prod[i] = (_Float16)(rk::hostref::activation(kind, (double)gate[i]) * (double)up[i]);
}

void rocket_ffn_ref_fp16(int M, int H, int I, const _Float16 *x, const _Float16 *Wg, const _Float16 *Wu,
                         const _Float16 *Wd, int kind, _Float16 *out)
{
    (void)rk::ffn_ref_fp16(M, H, I, x, Wg, Wu, Wd, kind, out);
}

void rocket_flash_attn_ref_fp16(int n_tokens, int n_kv, int head_dim, int dv, int n_head, int n_kv_heads, float scale,
                                float softcap, const _Float16 *Q, const _Float16 *K, const _Float16 *V,
                                const _Float16 *mask, _Float16 *out)
{
    (void)rk::flash_attn_ref_fp16(n_tokens, n_kv, head_dim, dv, n_head, n_kv_heads, scale, softcap, Q, K, V, mask,
                                  out);
}

void rocket_mha_self_ref_fp16(int T, int d, int n_head, const _Float16 *x, const _Float16 *Wq, const _Float16 *bq,
                              const _Float16 *Wk, const _Float16 *bk, const _Float16 *Wv, const _Float16 *bv,
                              const _Float16 *Wo, const _Float16 *bo, _Float16 *out)
{
    (void)rk::mha_self_ref_fp16(T, d, n_head, x, Wq, bq, Wk, bk, Wv, bv, Wo, bo, out);
}

}  // extern "C"
