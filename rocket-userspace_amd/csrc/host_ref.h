// host_ref.h — the exact fp64 host paths of the FFN and attention blocks (fd < 0), built on a
// small dense-double toolkit: operands are widened from fp16 once, products run over blocks
// of rows, and every output element is one ascending sum, rounded to fp16 once at the end.
#pragma once

#include <stddef.h>

namespace rk {
namespace hostref {

// Row-major matrix of doubles.
struct Mat {
    int rows = 0, cols = 0;
    double *data = nullptr;   // owned
    Mat() = default;
    Mat(int r, int c);
    Mat(Mat &&o) noexcept;
    Mat &operator=(Mat &&o) noexcept;
    Mat(const Mat &) = delete;
    Mat &operator=(const Mat &) = delete;
    ~Mat();
    double *row(int r) { return data + (size_t)r * cols; }
    const double *row(int r) const { return data + (size_t)r * cols; }
};

// fp16 [rows, cols] row-major -> doubles; transposed: the result is [cols, rows].
Mat widen(const _Float16 *p, int rows, int cols, bool transposed = false);

// Where a linear layer's bias enters its sum: as the starting value, or after the products.
enum class Bias { First, Last };

// y[r, o] = sum_i x[r, i] * w[o, i] over i ascending, with bias b[o] (b may be null: no
// bias term at all) at the start or the end of the sum.
Mat linear(const Mat &x, const Mat &w, const _Float16 *b, Bias at);

// The activation of the gated FFN / MLP blocks in fp64: GELU with erf for
// ROCKET_ACTIVATION_GELU, SiLU for every other kind.
double activation(int kind, double g);

}  // namespace hostref

// The host references behind rocket_ffn_ref_fp16, rocket_flash_attn_ref_fp16,
// rocket_mha_self_ref_fp16 (rocket_ffn.h / rocket_attn.h) and the fd < 0 paths of the FFN,
// MLP and attention entries. Each returns false, having written nothing, when host memory
// runs out (no exception leaves them).
bool mlp_ref_fp16(int M, int Din, int Dff, int Dout, const _Float16 *x, const _Float16 *W1, const _Float16 *b1,
                  const _Float16 *W2, int kind, _Float16 *out);
bool ffn_ref_fp16(int M, int H, int I, const _Float16 *x, const _Float16 *Wg, const _Float16 *Wu, const _Float16 *Wd,
                  int kind, _Float16 *out);
bool flash_attn_ref_fp16(int n_tokens, int n_kv, int head_dim, int dv, int n_head, int n_kv_heads, float scale,
                         float softcap, const _Float16 *Q, const _Float16 *K, const _Float16 *V, const _Float16 *mask,
                         _Float16 *out);
bool mha_self_ref_fp16(int T, int d, int n_head, const _Float16 *x, const _Float16 *Wq, const _Float16 *bq,
                       const _Float16 *Wk, const _Float16 *bk, const _Float16 *Wv, const _Float16 *bv,
                       const _Float16 *Wo, const _Float16 *bo, _Float16 *out);

}  // namespace rk
