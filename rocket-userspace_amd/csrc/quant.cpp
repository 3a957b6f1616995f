// quant.cpp — per-row int8 quantisation of activations on the GPU (rocket_quant.h). The
// formula is the host quantisation of the reference's W8A8 tool
// (tools/rk3576-w8a8-hostterm.c:51-68); the kernel is k_quant_rows.
#include "ops.h"
#include "rocket_quant.h"

using namespace rk;

namespace {

int quantize(int fd, const char *who, int M, int K, const void *A, bool f16, int8_t *Aq, float *row_scale)
{
    if (M < 1 || K < 8 || K % 8 || M > kDimMax || K > kDimMax || !A || !Aq || !row_scale) {
        ROCKET_LOGE("%s: M=%d K=%d (need M >= 1, K %% 8 == 0) or a null operand\n", who, M, K);
        return ROCKET_E_SHAPE;
    }
    Locked L(fd);
    if (!L.ok()) {
        ROCKET_LOGE("%s: fd %d is not an open rocket handle\n", who, fd);
        return ROCKET_E_DEVICE;
    }
    const size_t in_bytes = (size_t)M * K * (f16 ? 2 : 4);
    Call c(L.h, who);
    c.want(A, in_bytes);
    c.want(Aq, (size_t)M * K);
    c.want(row_scale, (size_t)M * sizeof(float));
    if (int rc = c.begin()) return rc;
    QuantRows q;
    q.n = 1;
    q.K = K;
    q.f16 = f16;
    q.M[0] = M;
    q.A[0] = c.in(A, in_bytes);
    q.Aq[0] = static_cast<int8_t *>(c.out(Aq, (size_t)M * K));
    q.row_scale[0] = static_cast<float *>(c.out(row_scale, (size_t)M * sizeof(float)));
    if (!q.A[0] || !q.Aq[0] || !q.row_scale[0]) return c.finish();
    uint64_t blocks = 0;
    if (quant_rows(q, c.stream(), &blocks) != hipSuccess) {
        (void)hipGetLastError();
        ROCKET_LOGE("%s: kernel launch rejected\n", who);
        (void)c.finish();
        return ROCKET_E_DEVICE;
    }
    count_launch(blocks);
    return c.finish();
}

}  // namespace

extern "C" {

int rocket_quantize_rows_int8(int fd, int M, int K, const float *A, int8_t *Aq, float *row_scale)
{
    return quantize(fd, "rocket_quantize_rows_int8", M, K, A, false, Aq, row_scale);
}

int rocket_quantize_rows_int8_fp16(int fd, int M, int K, const _Float16 *A, int8_t *Aq, float *row_scale)
{
    return quantize(fd, "rocket_quantize_rows_int8_fp16", M, K, A, true, Aq, row_scale);
}

}  // extern "C"
