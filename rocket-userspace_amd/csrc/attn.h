// attn.h — the fused attention kernel behind rocket_attn.h (device side in attn.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace rk {

// out_h = softmax(clamp(softcap * tanh(scale * Q_h K_hk^T / softcap) + mask, -30000)) V_hk
// for every query head h (kv head hk = h / gqa), all operands fp16, strides in elements.
// Q[h][t][c] at Q + h*q_hs + t*q_rs + c; K[hk][j][c] at K + hk*k_hs + j*k_rs + c;
// Vt[hk][c][j] (V transposed: keys contiguous) at Vt + hk*v_hs + c*v_rs + j, with
// v_rs % 64 == 0, v_rs >= n_kv and zeros in columns [n_kv, v_rs); mask[t][j] at
// mask + t*m_rs + j (or null); out[h][t][c] at O + h*o_hs + t*o_rs + c.
struct FaLaunch {
    const _Float16 *Q = nullptr, *K = nullptr, *Vt = nullptr, *mask = nullptr;
    _Float16 *O = nullptr;
    long q_hs = 0, q_rs = 0, k_hs = 0, k_rs = 0, v_hs = 0, v_rs = 0, o_hs = 0, o_rs = 0, m_rs = 0;
    int T = 0, n_kv = 0, dk = 0, dv = 0, n_head = 0, gqa = 1;
    float scale = 1.f, softcap = 0.f;
    // workspace for key-axis splits (flash_attn_ws_bytes); without it one workgroup walks
    // every key of its queries
    float *ws = nullptr;
    size_t ws_bytes = 0;
};

// Workspace the launch's key-axis split wants (0: none).
size_t flash_attn_ws_bytes(const FaLaunch &L);

// Key / value head dims the kernel supports: multiples of 16 up to 256.
constexpr int kAttnMaxHeadDim = 256;

hipError_t flash_attn(const FaLaunch &L, hipStream_t s, uint64_t *blocks_out);

// dst[r][c] = c < cols ? src[r * src_rs + c] : 0 for r < rows, c < cols_pad (fp16).
hipError_t pad_cols_f16(const _Float16 *src, long src_rs, _Float16 *dst, long rows, int cols, int cols_pad,
                        hipStream_t s);

// Per-head transpose of a token-major [T][n_head * dh] matrix: dst[h][c][t] (row stride
// t_pad, zeros for t >= T).
hipError_t heads_transpose_f16(const _Float16 *src, _Float16 *dst, int T, int n_head, int dh, int t_pad,
                               hipStream_t s);

}  // namespace rk
