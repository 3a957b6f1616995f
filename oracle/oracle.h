/*
 * oracle.h — CPU restatement of librocketnpu's host references for the matmul path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the shipped library links, loads or calls this
 * code; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as
 * the checker or as the timed CPU baseline. Each function names the reference file:line
 * whose arithmetic it restates (paths relative to the reference repository root).
 *
 * Layout convention everywhere: C[M,N] = A[M,K] * B[N,K]^T, row-major.
 * fp16 values are passed as their uint16_t bit patterns.
 */
#ifndef RK_ORACLE_H
#define RK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- portable generators (splitmix64, as tests/matmul_correctness_matrix_rocket.c:50-61)
 * All generators are pure functions of (seed, index), so any slice can be regenerated
 * without the rest: element i of a stream is f(splitmix64 output number i). */
uint64_t rko_splitmix64_next(uint64_t *state);
uint64_t rko_splitmix64_at(uint64_t seed, uint64_t i);          /* output number i (0-based) */
void rko_gen_i8(int8_t *out, size_t n, uint64_t seed, int lo, int hi);        /* U{lo..hi} */
void rko_gen_i16(int16_t *out, size_t n, uint64_t seed, int lo, int hi);      /* U{lo..hi} */
void rko_gen_f32_uniform(float *out, size_t n, uint64_t seed, float lo, float hi);
void rko_gen_f32_normal(float *out, size_t n, uint64_t seed, float mean, float std);

/* ---- scalar conversions ---- */
uint16_t rko_f32_to_f16(float f);           /* IEEE binary16, round to nearest even */
float    rko_f16_to_f32(uint16_t h);
void     rko_f32_to_f16_n(const float *in, uint16_t *out, size_t n);
void     rko_f16_to_f32_n(const uint16_t *in, float *out, size_t n);
uint16_t rko_f32_to_bf16_trunc(float f);    /* rocket_matmul.c:3444-3446 */
float    rko_bf16_to_f32(uint16_t b);
float    rko_tf32_trunc(float f);           /* tests/matmul_tf32_tiled_rocket.c:52-56 */
/* Balanced signed byte split of a clamped int16 (rocket_matmul.c:3399-3406):
 * x -> clamp to [-32768, 32639]; lo = ((x+128)&0xFF)-128; hi = (x-lo)>>8. */
void     rko_int16_split(int16_t x, int8_t *hi, int8_t *lo);

/* ---- references ---- */

/* fp16 in, fp32 accumulation, one RNE rounding to fp16 (tests/matmul_fp16_rocket.c:43-50;
 * tests/matmul_tiled_rocket.c:76-82). */
void rko_matmul_fp16(int M, int K, int N, const uint16_t *A, const uint16_t *B, uint16_t *C);
void rko_matmul_fp16_naive(int M, int K, int N, const uint16_t *A, const uint16_t *B, uint16_t *C);
/* fp16 in, fp32 out with a double accumulation (rocket_matmul.c:3620-3758). */
void rko_matmul_fp16_f32out(int M, int K, int N, const uint16_t *A, const uint16_t *B, float *C);

/* int8 -> int32: exact int64 sum cast to int32 (tests/matmul_int8_tiled_rocket.c:77-83). */
void rko_matmul_int8(int M, int K, int N, const int8_t *A, const int8_t *B, int32_t *C);

/* int16 -> int64 with the reference clamp (rocket_matmul.c:3377-3421;
 * tests/matmul_int16_exact_rocket.c:88-94). */
void rko_matmul_int16_exact(int M, int K, int N, const int16_t *A, const int16_t *B, int64_t *C);

/* Exact per-group int32 partials P[m][g][n] (the K-tile partials the reference reads back,
 * rocket_matmul.c:2842-2856, with Kt == group). P has M*nG*N entries. */
void rko_gw_partials(int M, int K, int N, int group, const int8_t *A, const int8_t *B, int32_t *P);

/* Group-wise fp32 combine, g ascending, one fused multiply-add per group:
 *   acc = 0; for g: acc = fmaf(a_scale[m,g]*b_scale[n,g], (float)P_g[m,n], acc)
 * (rocket_matmul.c:2846-2854 and :3254-3267 with the products contracted). */
void rko_matmul_gw_f32(int M, int K, int N, int group, const int8_t *A, const int8_t *B,
                       const float *a_scale, const float *b_scale, float *Cf);
/* Group-wise with one activation scale per row (librocketnpu's *_rowscale additions; no
 * reference counterpart): acc = 0; for g ascending: acc = fmaf(b_scale[n,g], (float)P_g[m,n], acc);
 * Cf[m,n] = a_row[m] * acc. With a_row = 1 it equals rko_matmul_gw_f32 with a_scale = 1. */
void rko_matmul_gw_rowscale_f32(int M, int K, int N, int group, const int8_t *A, const int8_t *B,
                                const float *a_row, const float *b_scale, float *Cf);
/* Same quantity in fp64, the reference tests' oracle (tests/matmul_int8_groupwise_rocket.c:41-57;
 * tests/matmul_int4_groupwise_rocket.c:55-66). */
void rko_matmul_gw_f64(int M, int K, int N, int group, const int8_t *A, const int8_t *B,
                       const float *a_scale, const float *b_scale, double *Cd);

/* bf16: truncate both fp32 operands, exact products, double accumulation
 * (tests/matmul_bf16_tiled_rocket.c:45-49, 84-111). */
void rko_matmul_bf16(int M, int K, int N, const float *A, const float *B, float *C);
/* tf32: clear the 13 low mantissa bits, double accumulation
 * (tests/matmul_tf32_tiled_rocket.c:52-56, 96-130). */
void rko_matmul_tf32(int M, int K, int N, const float *A, const float *B, float *C);
/* Plain fp32 operands, double accumulation: the "fp32 reference" the tolerances are
 * stated against. */
void rko_matmul_f32(int M, int K, int N, const float *A, const float *B, float *C);

/* ---- feed-forward blocks (reference src/rocket_ffn.c) ----
 * binary64 -> binary16, round to nearest even, one rounding (the reference's
 * `(_Float16)double` casts). */
uint16_t rko_f64_to_f16(double d);
/* The reference host nonlinearity (rocket_ffn.c:23-27): GELU (kind 5) = 0.5 g (1 + erf(g/√2)),
 * every other kind SiLU = g / (1 + exp(-g)). */
double rko_act_exact(int kind, double g);
/* prod[i] = f16(act(gate[i]) * up[i]) in double (rocket_ffn.c:33-38). */
void rko_geglu_f16(const uint16_t *gate, const uint16_t *up, int kind, uint16_t *prod, size_t n);
/* Gated FFN, fp64 throughout, fp16 output (rocket_ffn.c:58-82): x[M,H], Wg/Wu[I,H], Wd[H,I]. */
void rko_ffn_f16(int M, int H, int I, const uint16_t *x, const uint16_t *Wg, const uint16_t *Wu,
                 const uint16_t *Wd, int kind, uint16_t *out);
/* MLP host path (rocket_ffn.c:236-254): act(x W1^T + b1) rounded to fp16, then W2 in fp64,
 * fp16 output. b1 may be NULL. */
void rko_mlp_f16(int M, int Din, int Dff, int Dout, const uint16_t *x, const uint16_t *W1, const uint16_t *b1,
                 const uint16_t *W2, int kind, uint16_t *out);

/* ---- per-row activation quantisation (reference tools/rk3576-w8a8-hostterm.c:51-68) ----
 * amax = max|a|; s = 127/amax (fp32); q = nearbyintf(a*s) clamped to int8; rs = amax/127
 * (s = rs = 0 for an all-zero row). */
void rko_quant_rows_f32(int M, int K, const float *A, int8_t *Aq, float *row_scale);

/* ---- attention (reference src/rocket_attn.c) ----
 * Masked grouped-query attention, fp64 (rocket_attn.c:181-228): per head h (kv head
 * h / (n_head / n_kv_heads)) and token t, s_j = clamp(softcap·tanh(f32(q·k_j)·scale / softcap)
 * + mask[t][j], -30000) in fp32 (no tanh when softcap == 0), softmax over j in fp64, fp16
 * output. Q [n_head][T][dk], K [n_kv_heads][n_kv][dk], V [n_kv_heads][dv][n_kv] (transposed),
 * mask [T][n_kv] or NULL, out [n_head][T][dv]. */
void rko_flash_attn_f16(int T, int n_kv, int dk, int dv, int n_head, int n_kv_heads, float scale, float softcap,
                        const uint16_t *Q, const uint16_t *K, const uint16_t *V, const uint16_t *mask, uint16_t *out);
/* Encoder self-attention sublayer, fp64 throughout (rocket_attn.c:41-84): q/k/v = x W^T + b,
 * per-head softmax(q k^T / sqrt(dh)) v, out = ctx Wo^T + bo. Biases may be NULL. */
void rko_mha_self_f16(int T, int d, int n_head, const uint16_t *x, const uint16_t *Wq, const uint16_t *bq,
                      const uint16_t *Wk, const uint16_t *bk, const uint16_t *Wv, const uint16_t *bv,
                      const uint16_t *Wo, const uint16_t *bo, uint16_t *out);

/* Threads the oracle's OpenMP loops use (0 = OpenMP default). Returns the count in use. */
int  rko_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif /* RK_ORACLE_H */
