/*
 * rocket_matmul.h — the matmul family of librocketnpu, re-implemented for MI355X.
 *
 * Every prototype below is the reference's (reference include/rocket_matmul.h:50-778);
 * argument meaning, alignment rules, M==1 handling and return codes are kept. What runs
 * underneath is new: each entry stages its host operands into HBM (or uses them in place
 * when they already are device pointers, see rocket_hip.h), launches one hand-written
 * gfx950 MFMA kernel on the handle's HIP stream and waits for it.
 *
 * Convention (reference rocket_matmul.h:16-36): C[M,N] = A[M,K] * B[N,K]^T, all operands
 * row-major, caller-owned, never retained past return.
 *
 * Numerics on MI355X (what the parity tests hold the kernels to):
 *   fp16        fp16 x fp16 products, fp32 accumulation over the whole K, one RNE
 *               rounding to fp16 at the end (the reference's default DPU fp16
 *               K-accumulation drifts ~0.4%; this path does not).
 *   fp16_f32out same products, fp32 result.
 *   int8        int8 x int8, int32 accumulation over the whole K; the int32 result equals
 *               the reference's int64 host sum cast to int32.
 *   int4        int4 weights, int8 (or int4) activations, exact int32; no per-K-tile
 *               int16 saturation (the reference saturates; results agree wherever it
 *               does not).
 *   group-wise  per-group partials P_g exact in int32, Cf[m,n] = sum over g ascending of
 *               fmaf(a_scale[m,g]*b_scale[n,g], (float)P_g, Cf) in fp32.
 *   int16_exact inputs clamped to [-32768, 32639], balanced byte split, four int8 planes
 *               multiplied in one kernel, int64 result; bit-exact.
 *   bf16        fp32 inputs truncated to bf16, exact products, fp32 accumulation.
 *   tf32        fp32 inputs truncated to 10 mantissa bits; gfx950 has no tf32 MFMA, so
 *               each value is split exactly into two bf16 halves and three bf16 MFMAs
 *               (hi*hi + hi*lo + lo*hi) are accumulated in fp32 (relative error of the
 *               dropped lo*lo term <= 2^-16 per product).
 *
 * The planners keep the reference's validation and return contract (a POSITIVE count on
 * success, a negative rocket_status otherwise: test with `< 0`) and report the MI355X
 * workgroup tiling: Mt x Nt is the output tile of one workgroup, Kt the K extent one
 * workgroup accumulates in registers before its epilogue (the whole K, or the quant
 * group for the group-wise paths), and the count is the number of workgroups.
 *
 * The ROCKET_MM_MT/NT/KT, ROCKET_KACC, ROCKET_REUSE, ROCKET_MM_PIPE and ROCKET_MM_ASYM
 * knobs tuned NPU tiling; they are accepted and ignored.
 */
#ifndef ROCKET_MATMUL_H
#define ROCKET_MATMUL_H

#include <stdint.h>
#include <stddef.h>

/* A consumer whose compiler lacks _Float16 predefines ROCKET_FLOAT16_T to a 16-bit
 * storage type (reference rocket_matmul.h:12-14). */
#ifdef ROCKET_FLOAT16_T
typedef ROCKET_FLOAT16_T _Float16;
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 (reference rocket_matmul.h:50-62; rocket_matmul.c:498-568, 1945-1998) ----
 * Requires K%32, N%16, M%4; the one-shot entry pads M==1 to 4 and returns row 0. */
int rocket_matmul_plan(int M, int K, int N, int *Mt, int *Kt, int *Nt);
int rocket_matmul_fp16(int fd, int M, int K, int N,
                       const _Float16 *A, const _Float16 *B, _Float16 *C);

/* ---- batched same-shape fp16 (reference rocket_matmul.h:80-115; rocket_matmul.c:2042-2310)
 * nbatch independent products sharing (M,K,N), run as ONE grouped launch. Bit-identical to
 * calling rocket_matmul_fp16 per item. nbatch==1 falls through to rocket_matmul_fp16. */
int rocket_matmul_fp16_batch(int fd, int M, int K, int N, int nbatch,
                             const _Float16 *const *A, const _Float16 *const *B,
                             _Float16 *const *C);

typedef struct rocket_mm_batch rocket_mm_batch;
rocket_mm_batch *rocket_mm_batch_create(int fd);
void             rocket_mm_batch_free(rocket_mm_batch *b);
int rocket_mm_batch_run(rocket_mm_batch *b, int M, int K, int N, int nbatch,
                        const _Float16 *const *A, const _Float16 *const *B,
                        _Float16 *const *C);

/* ---- fp16 in, fp32 out (reference rocket_matmul.h:127-128; rocket_matmul.c:3620-3758) */
int rocket_matmul_fp16_f32out(int fd, int M, int K, int N,
                              const _Float16 *A, const _Float16 *B, float *C);

/* ---- RK3576-only entries (reference rocket_matmul.h:206-412) ----
 * A different chip with a requantising int8-output contract. Exported so a consumer that
 * links them still resolves; every one returns ROCKET_E_UNSUPPORTED (the planner
 * returns ROCKET_E_UNSUPPORTED as well) and writes nothing. */
int rocket_matmul_plan_int8_rk3576(int M, int K, int N, int *Mt, int *Kt, int *Nt);
int rocket_matmul_int8_rk3576(int fd, int M, int K, int N,
                              const int8_t *A, const int8_t *B,
                              const int32_t *bias, float scale, int8_t *C);
int rocket_matmul_int8_rk3576_perc(int fd, int M, int K, int N,
                                   const int8_t *A, const int8_t *B,
                                   const int32_t *bias, const float *scale_n,
                                   int8_t *C, double *worst_rel_err);
int rocket_matmul_int8_rk3576_perc_sa(int fd, int M, int K, int N,
                                      const int8_t *A, const int8_t *B,
                                      const int32_t *bias, const float *scale_n,
                                      const int64_t *sum_abs_w,
                                      int8_t *C, double *worst_rel_err);
struct rocket_rk3576_wbo;
int  rocket_rk3576_wbo_create(int fd, int K, int N, const int8_t *B,
                              struct rocket_rk3576_wbo **out);
void rocket_rk3576_wbo_free(int fd, struct rocket_rk3576_wbo *w);
int  rocket_matmul_int8_rk3576_perc_wbo(int fd, int M, int K, int N,
                                        const int8_t *A,
                                        const struct rocket_rk3576_wbo *wbo,
                                        const int32_t *bias, const float *scale_n,
                                        const int64_t *sum_abs_w,
                                        int8_t *C, double *worst_rel_err);
void rocket_rk3576_bo_pool_drain(int fd);
int  rocket_matmul_int8_rk3576_i32(int fd, int M, int K, int N,
                                   const int8_t *A, const int8_t *B,
                                   const int32_t *bias, int32_t *C);
typedef struct rocket_rk3576_i32_stats {
    unsigned submits;
    unsigned tasks;
    unsigned redo_empty;
    unsigned redo_zeroed;
    unsigned atoms_empty;
    unsigned atoms_zeroed;
    unsigned accepted_zero;
    unsigned refused;
} rocket_rk3576_i32_stats;
void rocket_rk3576_i32_last_stats(rocket_rk3576_i32_stats *out);   /* zero-fills *out */

/* ---- int8 -> raw int32 (reference rocket_matmul.h:414-416; rocket_matmul.c:2383-2627)
 * Requires K%32, N%32, M%4; one-shot pads M==1. */
int rocket_matmul_plan_int8(int M, int K, int N, int *Mt, int *Kt, int *Nt);
int rocket_matmul_int8(int fd, int M, int K, int N,
                       const int8_t *A, const int8_t *B, int32_t *C);

/* ---- group-wise int8 (reference rocket_matmul.h:435-440; rocket_matmul.c:2671-2871) ----
 * Cf[m,n] = sum_g a_scale[m*nG+g] * b_scale[n*nG+g] * P_g[m,n], nG = K/group.
 * group >= 32, group%32, K%group; K%32, N%32, M%4 (no M==1 pad). Cf is overwritten. */
int rocket_matmul_plan_int8_gw(int M, int K, int N, int group,
                               int *Mt, int *Kt, int *Nt);
int rocket_matmul_int8_groupwise(int fd, int M, int K, int N,
                                 const int8_t *A, const int8_t *B,
                                 const float *a_scale, const float *b_scale,
                                 float *Cf, int group);

/* ---- int4 (reference rocket_matmul.h:455-475; rocket_matmul.c:2917-3282) ----
 * One value per int8_t. B must lie in [-8,7] (it is nibble-packed in HBM); A may use the
 * whole int8 range (W4A8). Requires K%32, N%64, M%4; one-shot pads M==1.
 * kt_cap only tuned the reference's int16 readback; the result here is exact for any
 * kt_cap. The group-wise entry keeps the reference's bounds (group%32, group|K,
 * 49*group < 32767, M%4). */
int rocket_matmul_plan_int4(int M, int K, int N, int *Mt, int *Kt, int *Nt);
int rocket_matmul_int4(int fd, int M, int K, int N,
                       const int8_t *A, const int8_t *B, int32_t *C);
int rocket_matmul_int4_ex(int fd, int M, int K, int N,
                          const int8_t *A, const int8_t *B, int32_t *C, int kt_cap);
int rocket_matmul_int4_groupwise(int fd, int M, int K, int N,
                                 const int8_t *A, const int8_t *B,
                                 const float *a_scale, const float *b_scale,
                                 float *Cf, int group);

/* ---- int16 plan + bit-exact int16 -> int64 (reference rocket_matmul.h:487-501;
 * rocket_matmul.c:3320-3421). int16_exact requires K%32, N%32, M%4 (pads M==1). */
int rocket_matmul_plan_int16(int M, int K, int N, int *Mt, int *Kt, int *Nt);
int rocket_matmul_int16_exact(int fd, int M, int K, int N,
                              const int16_t *A, const int16_t *B, int64_t *C);

/* ---- bf16 (reference rocket_matmul.h:515-517; rocket_matmul.c:3444-3596) ----
 * fp32 A/B truncated to bf16, fp32 C. K%32, N%16, M%4 (pads M==1). */
int rocket_matmul_plan_bf16(int M, int K, int N, int *Mt, int *Kt, int *Nt);
int rocket_matmul_bf16(int fd, int M, int K, int N,
                       const float *A, const float *B, float *C);

/* ---- bf16 multi-worker and streaming (reference rocket_matmul.h:529-549;
 * rocket_bf16_stream.c:344-549). One GPU grid replaces the per-fd N-split, so these are
 * the single-handle computation; results equal rocket_matmul_bf16 bit for bit.
 * nthreads is clamped to [1,8] and otherwise ignored. */
int rocket_matmul_bf16_mt(int M, int K, int N,
                          const float *A, const float *B, float *C, int nthreads);
typedef struct rocket_bf16_stream rocket_bf16_stream;
rocket_bf16_stream *rocket_bf16_stream_create(int nthreads);
void                rocket_bf16_stream_free(rocket_bf16_stream *s);
int rocket_matmul_bf16_stream(rocket_bf16_stream *s, int M, int K, int N,
                              const float *A, const float *B, float *C);

/* ---- tf32 (reference rocket_matmul.h:568-570; rocket_matmul.c:3782-3982) ----
 * K%16, N%16, M%4 (pads M==1). */
int rocket_matmul_plan_tf32(int M, int K, int N, int *Mt, int *Kt, int *Nt);
int rocket_matmul_tf32(int fd, int M, int K, int N,
                       const float *A, const float *B, float *C);

/* ---- fp16 multi-worker (reference rocket_matmul.h:579-581; rocket_matmul_mt.c:58-99) */
int rocket_matmul_fp16_mt(int M, int K, int N,
                          const _Float16 *A, const _Float16 *B, _Float16 *C,
                          int nthreads);

/* ---- resident fp16 weights (reference rocket_matmul.h:609-619; rocket_prepacked.c) ----
 * rocket_weights_pack copies B[N,K] into HBM once; every _prepacked call reuses it at any
 * M (the HBM layout does not depend on M, so -2 is never returned for a compatible M).
 * K or N different from the packed ones: -1. Free weights before their ctx. A ctx is not
 * thread-safe: one per host thread. */
typedef struct rocket_ctx     rocket_ctx;
typedef struct rocket_weights rocket_weights;

rocket_ctx     *rocket_ctx_create(int nthreads);
void            rocket_ctx_free(rocket_ctx *ctx);
rocket_weights *rocket_weights_pack(rocket_ctx *ctx, int M, int K, int N, const _Float16 *B);
void            rocket_weights_free(rocket_ctx *ctx, rocket_weights *w);
int rocket_matmul_fp16_prepacked(rocket_ctx *ctx, int M, int K, int N,
                                 const _Float16 *A, _Float16 *C, rocket_weights *w);

/* ---- fp16 streaming and fused streaming (reference rocket_matmul.h:644-670;
 * rocket_prepacked.c:455-505). The fused entry runs the nseg weights as one launch over
 * the concatenated N and writes C[M, sum(Ns)]. */
typedef struct rocket_stream rocket_stream;
rocket_stream *rocket_stream_create(int nthreads);
void           rocket_stream_free(rocket_stream *s);
int rocket_matmul_fp16_stream(rocket_stream *s, int M, int K, int N,
                              const _Float16 *A, const _Float16 *B, _Float16 *C);
#define ROCKET_MAX_FUSE 8
int rocket_matmul_fp16_stream_fused(rocket_stream *s, int M, int K,
                                    const _Float16 *const *Bs, const int *Ns, int nseg,
                                    const _Float16 *A, _Float16 *C);

/* ---- resident int8 (reference rocket_matmul.h:703-741; rocket_prepacked_int8.c) ----
 * Shape rules K%32, N%32, M%4 at pack and at every call (call M%4 != 0 or M <= 0: -1).
 * K/N mismatch: -1. Per-channel entry on a group-wise weight, or the reverse: -1.
 * The weight lives in HBM in a tile-major pre-swizzled layout independent of M.
 * Results are bit-identical to the one-shot entries. */
typedef struct rocket_i8_ctx     rocket_i8_ctx;
typedef struct rocket_i8_weights rocket_i8_weights;

rocket_i8_ctx     *rocket_i8_ctx_create(int nthreads);
void               rocket_i8_ctx_free(rocket_i8_ctx *ctx);
rocket_i8_weights *rocket_i8_weights_pack(rocket_i8_ctx *ctx, int M, int K, int N,
                                          const int8_t *B);
void               rocket_i8_weights_free(rocket_i8_ctx *ctx, rocket_i8_weights *w);
size_t             rocket_i8_weights_bytes(const rocket_i8_weights *w);
int rocket_matmul_int8_prepacked(rocket_i8_ctx *ctx, int M, int K, int N,
                                 const int8_t *A, int32_t *C, rocket_i8_weights *w);
rocket_i8_weights *rocket_i8_weights_pack_gw(rocket_i8_ctx *ctx, int M, int K, int N,
                                             const int8_t *B, int group);
int rocket_matmul_int8_prepacked_gw(rocket_i8_ctx *ctx, int M, int K, int N,
                                    const int8_t *A, const float *a_scale,
                                    const float *b_scale, float *Cf, rocket_i8_weights *w);

/* ---- resident int4 (reference rocket_matmul.h:748-778; rocket_prepacked_int4.c) ----
 * The weight is nibble-packed in HBM (K/2 bytes per row, half the int8 footprint).
 * N%64, K%32, M%4 at pack; call M%4 (-1 otherwise); the gw pack keeps
 * group%32, group|K, 49*group < 32767. */
typedef struct rocket_i4_ctx     rocket_i4_ctx;
typedef struct rocket_i4_weights rocket_i4_weights;

rocket_i4_ctx     *rocket_i4_ctx_create(int nthreads);
void               rocket_i4_ctx_free(rocket_i4_ctx *ctx);
rocket_i4_weights *rocket_i4_weights_pack(rocket_i4_ctx *ctx, int M, int K, int N, const int8_t *B);
void               rocket_i4_weights_free(rocket_i4_ctx *ctx, rocket_i4_weights *w);
int rocket_matmul_int4_prepacked(rocket_i4_ctx *ctx, int M, int K, int N,
                                 const int8_t *A, int32_t *C, rocket_i4_weights *w);
rocket_i4_weights *rocket_i4_weights_pack_gw(rocket_i4_ctx *ctx, int M, int K, int N,
                                             const int8_t *B, int group);
int rocket_matmul_int4_prepacked_gw(rocket_i4_ctx *ctx, int M, int K, int N,
                                    const int8_t *A, const float *a_scale,
                                    const float *b_scale, float *Cf, rocket_i4_weights *w);
size_t rocket_i4_weights_bytes(const rocket_i4_weights *w);

#ifdef __cplusplus
}
#endif
#endif /* ROCKET_MATMUL_H */
