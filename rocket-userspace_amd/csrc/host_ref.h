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

// The five host references (declared in rocket_ffn.h / rocket_attn.h):
//   rocket_geglu_ref_fp16, rocket_ffn_ref_fp16, rocket_flash_attn_ref_fp16,
//   rocket_mha_self_ref_fp16, and the MLP's fd < 0 path below.
void mlp_ref_fp16(int M, int Din, int Dff, int Dout, const _Float16 *x, const _Float16 *W1, const _Float16 *b1,
                  const _Float16 *W2, int kind, _Float16 *out);

}  // namespace rk
