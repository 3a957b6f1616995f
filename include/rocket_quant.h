/*
 * rocket_quant.h — per-row int8 quantisation of activations on the GPU, ahead of the
 * integer GEMMs (MI355X additions; the reference library has no counterpart: its callers
 * quantise on the host, rocket_matmul.h:130-135 and 719-726, with the formula of
 * tools/rk3576-w8a8-hostterm.c:51-68, which these entries reproduce bit for bit).
 *
 * For each row m of A[M, K]:
 *     amax         = max_k |A[m, k]|
 *     row_scale[m] = amax / 127            (0 for an all-zero row)
 *     Aq[m, k]     = clamp(rint(A[m, k] * (127 / amax)), -128, 127)     (0 for a zero row)
 * in fp32 arithmetic: both divisions IEEE-rounded, the product one fp32 multiply, rint
 * rounding to nearest even. A[m, k] ~= row_scale[m] * Aq[m, k]. Inputs must be finite.
 *
 * Callers: GPU-resident inference backends that hold fp32 (or fp16) activations and run the
 * W8A8 / W4A8 resident products (ggml-style runners, the MoE dispatch). Operands may be host
 * or device pointers, as every entry. K % 8 == 0. Return 0, or -1 (shape / argument),
 * ROCKET_E_DEVICE.
 */
#ifndef ROCKET_QUANT_H
#define ROCKET_QUANT_H

#include <stddef.h>
#include <stdint.h>

#include "rocket_matmul.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Aq[M, K] int8 and row_scale[M] from fp32 (or fp16) activations, one kernel launch. */
int rocket_quantize_rows_int8(int fd, int M, int K, const float *A, int8_t *Aq, float *row_scale);
int rocket_quantize_rows_int8_fp16(int fd, int M, int K, const _Float16 *A, int8_t *Aq, float *row_scale);

/* The resident group-wise products on fp32 activations: A is quantised per row into the
 * handle's arena by the pre-pass above, then the *_rowscale kernel runs with those codes and
 * scales — the same bits as rocket_quantize_rows_int8 followed by
 * rocket_matmul_int{8,4}_prepacked_gw_rowscale, in one call (two launches, the int8 codes
 * never leave the GPU). Same checks and return codes as the *_rowscale entry each mirrors. */
int rocket_matmul_int8_prepacked_gw_f32in(rocket_i8_ctx *ctx, int M, int K, int N, const float *A,
                                          const float *b_scale, float *Cf, rocket_i8_weights *w);
int rocket_matmul_int4_prepacked_gw_f32in(rocket_i4_ctx *ctx, int M, int K, int N, const float *A,
                                          const float *b_scale, float *Cf, rocket_i4_weights *w);
/* MoE experts: every A_e quantised in one pre-pass launch, then the grouped launch of
 * rocket_matmul_int8_prepacked_gw_grouped_rowscale. */
int rocket_matmul_int8_prepacked_gw_grouped_f32in(rocket_i8_ctx *ctx, int n, const int *M, int K, int N,
                                                  const float *const *A, const float *const *b_scale,
                                                  float *const *Cf, rocket_i8_weights *const *w);
/* MoE down products on gated activations: expert e's input rows are act(gate_e) * up_e of
 * fp32 [M_e, K] rows (act: ROCKET_ACTIVATION_SILU or _GELU, in fp32 as the FFN block entries
 * compute them), formed and quantised per row in the same one pre-pass launch, then the
 * grouped launch of rocket_matmul_int8_prepacked_gw_grouped_rowscale. No counterpart in the
 * reference library (which has no grouped MoE entries): it replaces a separate gating pass
 * whose fp32 output the pre-pass would read again. Other checks and codes as
 * rocket_matmul_int8_prepacked_gw_grouped_f32in; another act is ROCKET_E_SHAPE. */
int rocket_matmul_int8_prepacked_gw_grouped_glu_f32in(rocket_i8_ctx *ctx, int n, const int *M, int K, int N,
                                                      const float *const *gate, const float *const *up, int act,
                                                      const float *const *b_scale, float *const *Cf,
                                                      rocket_i8_weights *const *w);
/* The same on fp16 gate and up rows (as rocket_matmul_int8_prepacked_gw_grouped_rowscale_f16out
 * writes them): each value widened to fp32 exactly, then act(gate) * up in fp32 as above. */
int rocket_matmul_int8_prepacked_gw_grouped_glu_f16in(rocket_i8_ctx *ctx, int n, const int *M, int K, int N,
                                                      const _Float16 *const *gate, const _Float16 *const *up,
                                                      int act, const float *const *b_scale, float *const *Cf,
                                                      rocket_i8_weights *const *w);

/* rocket_matmul_int4_prepacked_gw_f32in without any device allocation. It has no counterpart
 * in the reference library; it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The pre-pass's
 * int8 codes and row scales go to a fixed 16 MiB device array that each GPU holds for the life
 * of the process, so M * K rounded up to 256 plus M * 4 must stay within 16 MiB (-1 otherwise:
 * split the rows). A, b_scale and Cf must be device memory on the context's GPU, and A and Cf
 * 16-byte aligned (nothing is staged; a host or misaligned pointer is -1). Same results and
 * other checks as the entry it mirrors. All calls on one GPU share the array: calls queued on
 * one stream are ordered and safe, calls that overlap on one GPU (several handles or streams
 * at once) race. While the handle's stream is being captured into a HIP graph the call only
 * records its two kernel launches (no wait, no memset, no copy) and returns 0; it returns -4
 * if an earlier wait on the handle gave up, since draining it would end the capture. */
int rocket_matmul_int4_prepacked_gw_f32in_noalloc(rocket_i4_ctx *ctx, int M, int K, int N, const float *A,
                                                   const float *b_scale, float *Cf, rocket_i4_weights *w);

#ifdef __cplusplus
}
#endif
#endif /* ROCKET_QUANT_H */
