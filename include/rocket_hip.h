/*
 * rocket_hip.h — MI355X additions to librocketnpu. None of these has a counterpart in the
 * reference library; they are additive and change no existing entry's behaviour.
 *
 * Device operands. Every matmul entry in rocket_matmul.h also accepts HIP device
 * pointers (hipMalloc'd, 16-byte aligned, on the handle's device) for any operand: such
 * operands are used in place, with no host copy. Host pointers are staged as before.
 * Callers: GPU-resident consumers (a llama.cpp/ggml HIP backend, PyTorch, the bench).
 */
#ifndef ROCKET_HIP_H
#define ROCKET_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "rocket_matmul.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- streams and completion ----
 * rocket_hip_stream: the hipStream_t the handle's kernels run on.
 * rocket_hip_set_stream: run the handle's work on a caller's stream (NULL restores the
 *   handle's own); the caller keeps ownership of the stream and must not destroy it while
 *   bound. Default-priority streams only.
 * rocket_hip_set_mode: a mask of
 *   ROCKET_HIP_ASYNC           an entry whose operands are ALL device pointers returns as
 *                              soon as its kernels are queued (the caller orders and waits
 *                              on the stream itself). Entries with a host operand still wait.
 *   ROCKET_HIP_DEVICE_OPERANDS the caller guarantees every operand pointer is device memory
 *                              on the handle's device; the per-call pointer classification
 *                              (hipPointerGetAttributes) is skipped.
 *   0 (default) = classify every pointer and wait for every result, as the reference does.
 * rocket_hip_sync: wait for the handle's queued work (bounded by ROCKET_WAIT_MS).
 * All return 0 / ROCKET_E_DEVICE for a bad fd. */
#define ROCKET_HIP_ASYNC           1u
#define ROCKET_HIP_DEVICE_OPERANDS 2u
void *rocket_hip_stream(int fd);
int   rocket_hip_set_stream(int fd, void *stream);
int   rocket_hip_set_mode(int fd, unsigned mode);
int   rocket_hip_sync(int fd);

/* The handle a context or stream object runs on (for the calls above). */
int rocket_ctx_fd(const rocket_ctx *ctx);
int rocket_i8_ctx_fd(const rocket_i8_ctx *ctx);
int rocket_i4_ctx_fd(const rocket_i4_ctx *ctx);
int rocket_stream_fd(const rocket_stream *s);
int rocket_bf16_stream_fd(const rocket_bf16_stream *s);

/* ---- group-wise partial dump (debug) ----
 * The group-wise entries plus a copy of the exact per-group int32 partials
 * P[r][g][n] = sum over K-group g of A[row0+r, k] * B[n, k], for rows
 * [row0, row0 + nrows) (nrows may be 0), taken from the same kernel and the same
 * accumulator registers that feed Cf. P holds nrows * (K/group) * N int32.
 * Same validation and return codes as the entry each one extends. */
int rocket_matmul_int8_groupwise_dump(int fd, int M, int K, int N, const int8_t *A, const int8_t *B,
                                      const float *a_scale, const float *b_scale, float *Cf, int group,
                                      int row0, int nrows, int32_t *P);
int rocket_matmul_int4_groupwise_dump(int fd, int M, int K, int N, const int8_t *A, const int8_t *B,
                                      const float *a_scale, const float *b_scale, float *Cf, int group,
                                      int row0, int nrows, int32_t *P);
int rocket_matmul_int8_prepacked_gw_dump(rocket_i8_ctx *ctx, int M, int K, int N, const int8_t *A,
                                         const float *a_scale, const float *b_scale, float *Cf,
                                         rocket_i8_weights *w, int row0, int nrows, int32_t *P);
int rocket_matmul_int4_prepacked_gw_dump(rocket_i4_ctx *ctx, int M, int K, int N, const int8_t *A,
                                         const float *a_scale, const float *b_scale, float *Cf,
                                         rocket_i4_weights *w, int row0, int nrows, int32_t *P);
/* The same dump for the per-row-scale entries below (validation of the entry each extends,
 * then the dump arguments) and for the grouped launches: one window per product, rows
 * [row0[e], row0[e] + nrows[e]) of product e into P[e] (nrows[e] == 0: none for that
 * product). The partials come from the kernel the plain entry runs: the dump is a run-time
 * switch of the same instantiation, so the tile, group cadence and fold are the ones a call
 * without the dump uses. Group sizes above 65536 are refused (their partials are split). */
int rocket_matmul_int8_prepacked_gw_rowscale_dump(rocket_i8_ctx *ctx, int M, int K, int N, const int8_t *A,
                                                  const float *a_row_scale, const float *b_scale, float *Cf,
                                                  rocket_i8_weights *w, int row0, int nrows, int32_t *P);
int rocket_matmul_int4_prepacked_gw_rowscale_dump(rocket_i4_ctx *ctx, int M, int K, int N, const int8_t *A,
                                                  const float *a_row_scale, const float *b_scale, float *Cf,
                                                  rocket_i4_weights *w, int row0, int nrows, int32_t *P);
int rocket_matmul_int8_prepacked_gw_grouped_dump(rocket_i8_ctx *ctx, int n, const int *M, int K, int N,
                                                 const int8_t *const *A, const float *const *a_scale,
                                                 const float *const *b_scale, float *const *Cf,
                                                 rocket_i8_weights *const *w, const int *row0, const int *nrows,
                                                 int32_t *const *P);
int rocket_matmul_int8_prepacked_gw_grouped_rowscale_dump(rocket_i8_ctx *ctx, int n, const int *M, int K, int N,
                                                          const int8_t *const *A, const float *const *a_row_scale,
                                                          const float *const *b_scale, float *const *Cf,
                                                          rocket_i8_weights *const *w, const int *row0,
                                                          const int *nrows, int32_t *const *P);

/* ---- grouped resident group-wise launch (MoE experts) ----
 * n independent rocket_matmul_int8_prepacked_gw products that share (K, N, group),
 * C_e[M_e, N] for e < n, run as ONE kernel launch per 16 products. Each M_e must be a
 * multiple of 4 (0 allowed: that product is skipped). Every weight must be group-wise,
 * packed on this ctx with the same K, N and group. Results are bit-identical to n
 * separate rocket_matmul_int8_prepacked_gw calls. Returns 0, -1 on a contract violation. */
int rocket_matmul_int8_prepacked_gw_grouped(rocket_i8_ctx *ctx, int n, const int *M, int K, int N,
                                            const int8_t *const *A, const float *const *a_scale,
                                            const float *const *b_scale, float *const *Cf,
                                            rocket_i8_weights *const *w);

/* ---- per-row activation scales ----
 * Group-wise products whose activation scale is one fp32 per row (per-token quantised
 * activations, the usual W8A8 / W4A8 inference layout): a_row_scale holds M floats where
 * the entries they mirror take M * (K/group). With P_g[m, n] the exact int32 partial of
 * K-group g, acc = fmaf(b_scale[n*(K/group) + g], (float)P_g[m, n], acc) for g ascending
 * from acc = 0, then Cf[m, n] = a_row_scale[m] * acc: the reference's group sum with the
 * row scale factored out (one fp32 multiply per row instead of one per group). Results
 * differ from the mirrored entry called with the row scale repeated over the groups only
 * in fp32 rounding. Validation and return codes are those of the mirrored entry:
 *   rocket_matmul_int8_groupwise_rowscale            rocket_matmul_int8_groupwise
 *   rocket_matmul_int4_groupwise_rowscale            rocket_matmul_int4_groupwise
 *   rocket_matmul_int8_prepacked_gw_rowscale         rocket_matmul_int8_prepacked_gw
 *   rocket_matmul_int4_prepacked_gw_rowscale         rocket_matmul_int4_prepacked_gw
 *   rocket_matmul_int8_prepacked_gw_grouped_rowscale rocket_matmul_int8_prepacked_gw_grouped */
int rocket_matmul_int8_groupwise_rowscale(int fd, int M, int K, int N, const int8_t *A, const int8_t *B,
                                          const float *a_row_scale, const float *b_scale, float *Cf, int group);
int rocket_matmul_int4_groupwise_rowscale(int fd, int M, int K, int N, const int8_t *A, const int8_t *B,
                                          const float *a_row_scale, const float *b_scale, float *Cf, int group);
int rocket_matmul_int8_prepacked_gw_rowscale(rocket_i8_ctx *ctx, int M, int K, int N, const int8_t *A,
                                             const float *a_row_scale, const float *b_scale, float *Cf,
                                             rocket_i8_weights *w);
int rocket_matmul_int4_prepacked_gw_rowscale(rocket_i4_ctx *ctx, int M, int K, int N, const int8_t *A,
                                             const float *a_row_scale, const float *b_scale, float *Cf,
                                             rocket_i4_weights *w);
int rocket_matmul_int8_prepacked_gw_grouped_rowscale(rocket_i8_ctx *ctx, int n, const int *M, int K, int N,
                                                     const int8_t *const *A, const float *const *a_row_scale,
                                                     const float *const *b_scale, float *const *Cf,
                                                     rocket_i8_weights *const *w);
/* The same grouped products with fp16 results: C_e[m, n] is the fp32 result of
 * rocket_matmul_int8_prepacked_gw_grouped_rowscale rounded once to fp16 (half the bytes
 * written, for results that a later pass reads again, such as a MoE layer's gate and up
 * products). No counterpart in the reference library. Same checks and codes. */
int rocket_matmul_int8_prepacked_gw_grouped_rowscale_f16out(rocket_i8_ctx *ctx, int n, const int *M, int K, int N,
                                                            const int8_t *const *A, const float *const *a_row_scale,
                                                            const float *const *b_scale, _Float16 *const *C,
                                                            rocket_i8_weights *const *w);

/* Device address of a resident weight (row-major int8 [N,K], or the nibble-packed int4
 * layout, K/2 bytes per row: byte j of packed word d holds k = 8d+j in its high nibble
 * and k = 8d+4+j in its low nibble). For inspection and tests. */
const void *rocket_i8_weights_device(const rocket_i8_weights *w);
const void *rocket_i4_weights_device(const rocket_i4_weights *w);

#ifdef __cplusplus
}
#endif
#endif /* ROCKET_HIP_H */
