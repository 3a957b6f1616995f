/*
 * rocket_ffn.h — the transformer feed-forward blocks of librocketnpu on MI355X (reference
 * include/rocket_ffn.h, src/rocket_ffn.c), the callers the matmul path feeds.
 *
 *     gate = x Wg^T,  up = x Wu^T        [M, I]
 *     prod = act(gate) * up              [M, I]   (the gated core)
 *     out  = prod Wd^T                   [M, H]
 *
 * All operands are row-major fp16 in the [N, K] weight convention. `kind` is
 * ROCKET_ACTIVATION_SILU or ROCKET_ACTIVATION_GELU (rocket_activation.h); any other kind
 * returns -1. fd < 0 selects the exact host reference (as the reference library does);
 * fd >= 0 runs on the handle's GPU. Operands may be host or device pointers (as every
 * matmul entry). Returns 0, or a negative rocket_status.
 *
 * On the GPU the gate and up products run as one kernel whose epilogue applies the gated
 * activation to the fp32 accumulators and writes prod in fp16 (the two weights' rows are
 * paired inside each tile), and the down product reads prod straight from HBM: the
 * intermediates never leave the device, so rocket_ffn_fp16 and rocket_ffn_fp16_fused are the
 * same computation here.
 */
#ifndef ROCKET_FFN_H
#define ROCKET_FFN_H

#include <stdint.h>

#include "rocket_activation.h"

#ifdef __cplusplus
extern "C" {
#endif

/* prod[i] = act(gate[i]) * up[i] for i < n (reference rocket_ffn.c:33-54). fp32
 * arithmetic on the GPU (the activation to a few fp32 ulp: SiLU with the hardware exp and
 * reciprocal, GELU's erfc from a Chebyshev fit, fractional error below ~1e-5), one rounding
 * to fp16, within one fp16 step of the host reference, which rounds a double. */
int  rocket_geglu_fp16(int fd, const _Float16 *gate, const _Float16 *up,
                       int kind, _Float16 *prod, int n);
void rocket_geglu_ref_fp16(const _Float16 *gate, const _Float16 *up,
                           int kind, _Float16 *prod, int n);

/* Gated FFN block (reference rocket_ffn.c:58-121). x[M,H], Wg[I,H], Wu[I,H], Wd[H,I],
 * out[M,H]. Needs H%32, I%32 and M%4 (M == 1 allowed); M*I must fit an int. */
int  rocket_ffn_fp16(int fd, int M, int H, int I,
                     const _Float16 *x, const _Float16 *Wg, const _Float16 *Wu,
                     const _Float16 *Wd, int kind, _Float16 *out);
void rocket_ffn_ref_fp16(int M, int H, int I,
                         const _Float16 *x, const _Float16 *Wg, const _Float16 *Wu,
                         const _Float16 *Wd, int kind, _Float16 *out);
/* The reference's cube-resident variant (rocket_ffn.c:125-211): same signature and result. */
int  rocket_ffn_fp16_fused(int fd, int M, int H, int I,
                           const _Float16 *x, const _Float16 *Wg, const _Float16 *Wu,
                           const _Float16 *Wd, int kind, _Float16 *out);

/* Non-gated MLP (reference rocket_ffn.c:217-330): out = act(x W1^T + b1) W2^T. x[M,Din],
 * W1[Dff,Din], b1[Dff] (NULL: no bias), W2[Dout,Dff], out[M,Dout]. Needs Din%32, Dff%32,
 * Dout%16, M%4 (M == 1 allowed). The bias and activation run in the first product's
 * epilogue on the fp32 accumulators. */
int  rocket_mlp_fp16_fused(int fd, int M, int Din, int Dff, int Dout,
                           const _Float16 *x, const _Float16 *W1, const _Float16 *b1,
                           const _Float16 *W2, int kind, _Float16 *out);

#ifdef __cplusplus
}
#endif
#endif /* ROCKET_FFN_H */
