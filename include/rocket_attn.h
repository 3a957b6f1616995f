/*
 * rocket_attn.h — attention on MI355X (reference include/rocket_attn.h, src/rocket_attn.c):
 * the encoder self-attention sublayer and masked grouped-query (flash) attention, same
 * prototypes and argument rules as the reference.
 *
 * rocket_flash_attn_fp16 runs ONE fused kernel: per 128 queries of a head, the key axis in
 * tiles of 64 with the online (FlashAttention-2) softmax in fp32, the scores never leave
 * the GPU's registers. The reference's score steps are kept: S = scale·(q·k) in fp32,
 * soft-cap softcap·tanh(S/softcap) when softcap != 0, + the additive mask, clamped at -30000.
 * Layouts (dense fp16, head-major):
 *   Q [n_head][n_tokens][head_dim], K [n_kv_heads][n_kv][head_dim],
 *   V [n_kv_heads][dv][n_kv] (V transposed), mask [n_tokens][n_kv] or NULL,
 *   out [n_head][n_tokens][dv].
 * Requires n_head % n_kv_heads == 0, head_dim % 32 == 0 and dv % 16 == 0 (as the
 * reference) and, on the GPU, head_dim <= 256 and dv <= 256. fd < 0 = the exact fp64 host
 * reference. Returns 0, < 0 on error. _mt and _ctx are the same computation (one GPU runs
 * every head at once; nthreads is accepted and clamped as in the reference, and a context
 * holds one handle). Operands may be host or device pointers.
 *
 * rocket_mha_self_fp16: q/k/v = x·W^T + b (one grouped GEMM launch, bias in the epilogue),
 * the fused attention kernel over the heads (scale d_head^-0.5, no mask), then
 * out = ctx·Wo^T + bo. Weights row-major [out,in]; biases optional (NULL). Needs d % n_head
 * == 0 (reference) and, on the GPU, d % 32 == 0, d_head % 16 == 0, d_head <= 256.
 */
#ifndef ROCKET_ATTN_H
#define ROCKET_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int  rocket_mha_self_fp16(int fd, int T, int d, int n_head, const _Float16 *x,
                          const _Float16 *Wq, const _Float16 *bq,
                          const _Float16 *Wk, const _Float16 *bk,
                          const _Float16 *Wv, const _Float16 *bv,
                          const _Float16 *Wo, const _Float16 *bo, _Float16 *out);
void rocket_mha_self_ref_fp16(int T, int d, int n_head, const _Float16 *x,
                              const _Float16 *Wq, const _Float16 *bq,
                              const _Float16 *Wk, const _Float16 *bk,
                              const _Float16 *Wv, const _Float16 *bv,
                              const _Float16 *Wo, const _Float16 *bo, _Float16 *out);

typedef struct rocket_fa_ctx rocket_fa_ctx;
rocket_fa_ctx *rocket_fa_ctx_create(int nthreads);
void           rocket_fa_ctx_free(rocket_fa_ctx *c);

int  rocket_flash_attn_fp16(int fd, int n_tokens, int n_kv, int head_dim, int dv,
                            int n_head, int n_kv_heads, float scale, float softcap,
                            const _Float16 *Q, const _Float16 *K, const _Float16 *V,
                            const _Float16 *mask, _Float16 *out);
int  rocket_flash_attn_fp16_mt(int fd, int n_tokens, int n_kv, int head_dim, int dv,
                               int n_head, int n_kv_heads, float scale, float softcap,
                               const _Float16 *Q, const _Float16 *K, const _Float16 *V,
                               const _Float16 *mask, _Float16 *out, int nthreads);
int  rocket_flash_attn_fp16_ctx(rocket_fa_ctx *c, int n_tokens, int n_kv, int head_dim, int dv,
                                int n_head, int n_kv_heads, float scale, float softcap,
                                const _Float16 *Q, const _Float16 *K, const _Float16 *V,
                                const _Float16 *mask, _Float16 *out);
void rocket_flash_attn_ref_fp16(int n_tokens, int n_kv, int head_dim, int dv,
                                int n_head, int n_kv_heads, float scale, float softcap,
                                const _Float16 *Q, const _Float16 *K, const _Float16 *V,
                                const _Float16 *mask, _Float16 *out);

#ifdef __cplusplus
}
#endif
#endif /* ROCKET_ATTN_H */
