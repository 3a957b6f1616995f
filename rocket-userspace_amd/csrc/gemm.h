// gemm.h — internal launch interface of the gfx950 MFMA GEMM kernels.
//
// One kernel template serves every matmul entry of the library. A launch computes up to
// kMaxProblems independent products C_p[M_p, N] = A_p[M_p, K] * B_p[N, K]^T that share
// N, K, the operand formats and the epilogue (a single product is a launch with one
// problem; rocket_matmul_fp16_batch and the MoE grouped entry use several).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rk {

constexpr int kMaxProblems = 16;

// Operand formats as they lie in HBM. Both operands are K-contiguous rows.
enum class Fmt : int {
    I8,      // int8, K bytes per row
    I4P,     // int4 nibble-packed, K/2 bytes per row (B only; layout in pack_int4_kernel)
    I16,     // int16 (clamped to [-32768, 32639] and byte-split on load)
    F16,     // IEEE fp16
    F32BF16, // fp32 in HBM, truncated to bf16 on load
    F32TF32, // fp32 in HBM, truncated to tf32 on load and split exactly into bf16 hi + lo
    BF16,    // bf16, 2K bytes per row (fp32 operands truncated by convert_f32)
    BF16X2,  // tf32 split into bf16 hi/lo by convert_f32: per 8 elements, 8 hi then 8 lo
};

// Epilogues.
enum class Epi : int {
    I32,      // raw int32 (int8 and int4 paths; int4 accumulators carry a x16 factor)
    I64,      // int16_exact: 65536*HH + 256*(HL+LH) + LL, int64
    F16,      // fp32 accumulator rounded to fp16 (RNE)
    F32,      // fp32 accumulator
    GW,       // group-wise: per-group exact int32 partial, fp32 fmaf combine
    GLU,      // gated FFN core: B rows come from two weights (gate B, up B2) of N/2 rows each;
              // C[M, N/2] fp16 = act(gate) * up from the fp32 accumulators (fp16 operands)
    ACT,      // C fp16 = act(acc + bias[n]), bias fp16 [N] in B2 or none (fp16 operands)
};

// Activations of the GLU / ACT epilogues (rocket_activation_kind values).
constexpr int kActSilu = 3, kActGelu = 5;
constexpr int kActIdentity = -1;   // ACT epilogue with the bias alone (internal; no public kind)

struct Problem {
    int M;
    const void *A;        // [M, K] in fmt_a
    const void *B;        // [N, K] in fmt_b
    void *C;              // [M, N] in the epilogue's type
    const float *a_scale; // GW only: [M * nG]
    const float *b_scale; // GW only: [N * nG]
    const void *B2;       // GLU: the up weight [N/2, K]; ACT: fp16 bias [N] (or null)
    // GW debug dump: the exact int32 partial of every K-group for rows [dump_row0,
    // dump_row0 + dump_rows), laid out [row][group][n] (null: none)
    int32_t *dump = nullptr;
    int dump_row0 = 0, dump_rows = 0;
};

struct Launch {
    Fmt fmt_a = Fmt::I8, fmt_b = Fmt::I8;
    Epi epi = Epi::I32;
    int N = 0, K = 0;
    int kbeg = 0, kend = 0;   // K range of this launch (elements); [0, K) unless chunked
    int accum = 0;            // 1: add into C instead of overwriting it (chunked K)
    int group = 0;            // GW: quant group (elements of K)
    int rowscale = 0;         // GW: a_scale is one fp32 per row (Cf = a_scale[m] * sum_g fmaf(b_scale, P_g, .))
    int act = 0;              // GLU / ACT: kActSilu or kActGelu
    int f16out = 0;           // GW: C holds fp16 (each fp32 result rounded once) instead of fp32
    int kt = 0;               // GW: int32 partial period, divides group (== group normally)
    int nprob = 0;
    Problem prob[kMaxProblems];
    // split-K (one problem, int32 / fp16 / fp32 results): device workspace of
    // gemm_ws_bytes() bytes for the slices' partial planes; without it, one slice per tile.
    // Without them the launch runs one slice per tile.
    int32_t *ws = nullptr;
    size_t ws_bytes = 0;
    hipStream_t stream = nullptr;
};

// Workspace bytes the launch's split-K plan needs (0: no split). Reads the formats, epilogue,
// N, K range and the problems' M only.
size_t gemm_ws_bytes(const Launch &L);

// Validates the launch against what the kernels assume (alignment, sizes) and enqueues
// it. Returns hipSuccess or an error; never faults on a rejected launch.
hipError_t gemm_launch(const Launch &L, uint64_t *blocks_out);

// Tile geometry the dispatcher will use for (fmt, epi, M, N): for the planners.
void gemm_tile(Fmt fmt_a, Epi epi, int M, int N, int *bm, int *bn);

// Nibble-pack int8 values in [-8, 7] (one per byte, B[N, K] row-major) into the I4P
// layout (K/2 bytes per row) on the device.
hipError_t pack_int4(const int8_t *src, uint8_t *dst, int N, int K, hipStream_t s);

// prod[i] = act(gate[i]) * up[i] for n fp16 values (fp32 arithmetic, one rounding to fp16).
hipError_t geglu_f16(const _Float16 *gate, const _Float16 *up, _Float16 *prod, long n, int act, hipStream_t s);

// Converts n fp32 values (n % 8 == 0, 16-byte aligned) on the device into `to`: BF16
// (truncation, as Fmt::F32BF16 loads) or BF16X2 (tf32 hi/lo pairs, as Fmt::F32TF32 loads).
// A second array (src2 -> dst2, n2 values, n2 = 0: none) is converted in the same launch.
hipError_t convert_f32(const float *src, void *dst, long n, Fmt to, hipStream_t s,
                       const float *src2 = nullptr, void *dst2 = nullptr, long n2 = 0);

// Per-row int8 quantisation of up to kMaxProblems activation matrices A_p[M_p, K] (fp32,
// or fp16 when f16): row_scale = amax / 127, q = rint(x * (127 / amax)) clamped to int8
// (all zero, scale 0, for an all-zero row). One launch; K % 8 == 0, 16-byte aligned rows.
// act = kActSilu / kActGelu: the rows quantised are act(A_p) * A2_p, element by element in
// fp32 from fp32 (or, f16, fp16) gate and up rows (a gated FFN's hidden rows).
struct QuantRows {
    int n = 0, K = 0;
    bool f16 = false;
    int act = 0;
    int M[kMaxProblems] = {};
    const void *A[kMaxProblems] = {};
    const void *A2[kMaxProblems] = {};
    int8_t *Aq[kMaxProblems] = {};
    float *row_scale[kMaxProblems] = {};
};
hipError_t quant_rows(const QuantRows &q, hipStream_t s, uint64_t *blocks_out);

}  // namespace rk
