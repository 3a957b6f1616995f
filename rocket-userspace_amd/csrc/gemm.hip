// gemm.hip — launch planning for the gfx950 MFMA GEMM kernels (gemm_impl.h, instantiated per
// operand family in gemm_*.hip) and the streaming kernels around them.
//
// The split-K slice sums, per-row activation quantisation, int4 packing, fp32 conversion and
// gated-activation kernels live here; gemm_launch validates a launch, chooses its tile shape
// and K slices, and calls the family's dispatcher.
#include "gemm_impl.h"

namespace rk {
namespace gk {
namespace {

// prod = act(gate) * up over n halves (fp16 in and out, fp32 arithmetic); each thread takes 8 consecutive elements (one
// 16-byte load per operand when VEC, i.e. every pointer is 16-byte aligned).
template <bool VEC, int ACT>
__global__ __launch_bounds__(256) void k_geglu(const _Float16 *__restrict__ g, const _Float16 *__restrict__ u,
                                               _Float16 *__restrict__ p, long n)
{
    const long i0 = ((long)blockIdx.x * 256 + threadIdx.x) * 8;
    if (i0 >= n) return;
    if (VEC && i0 + 8 <= n) {
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
        const h8 gv = __builtin_nontemporal_load(reinterpret_cast<const h8 *>(g + i0));
        const h8 uv = __builtin_nontemporal_load(reinterpret_cast<const h8 *>(u + i0));
        h8 r;
#pragma unroll
        for (int e = 0; e < 8; e++) r[e] = (_Float16)(act_k<ACT>((float)gv[e]) * (float)uv[e]);
        __builtin_nontemporal_store(r, reinterpret_cast<h8 *>(p + i0));
        return;
    }
    const long i1 = i0 + 8 < n ? i0 + 8 : n;
    for (long i = i0; i < i1; i++) p[i] = (_Float16)(act_k<ACT>((float)g[i]) * (float)u[i]);
}

// Small fp16 products (a few 32 x 32 blocks of C and a short K, as configs[0]'s 64 x 256 x 128):
// one wave per 32 x 32 block reads its MFMA operands straight from global memory — lane l takes
// row l % 32 of the block's A and B rows and halves 16 s + 8 (l / 32) .. + 8 of substep s, the
// fragments the tiled kernels read from LDS — 8 substeps at a time, the next 8 in flight under
// this chunk's MFMAs. No LDS and no barrier: one round of load latency and the MFMAs. The
// MFMAs accumulate in the tiled kernels' K order, so the results carry the same bits.
constexpr int kSmallSub = 8;
template <bool F16OUT>
__global__ __launch_bounds__(64) void k_small_f16(const _Float16 *__restrict__ A, const _Float16 *__restrict__ B,
                                                  void *__restrict__ C, int M, int N, int K, int nbn)
{
    const int lane = threadIdx.x, bm = blockIdx.x / nbn, bn = blockIdx.x % nbn;
    const int r = lane & 31, h = lane >> 5;
    const Rsrc ra = rsrc(A + (size_t)bm * 32 * K, (uint32_t)(min(32, M - bm * 32) * K * 2));
    const Rsrc rb = rsrc(B + (size_t)bn * 32 * K, (uint32_t)(min(32, N - bn * 32) * K * 2));
    const uint32_t oa = (uint32_t)(r * K + 8 * h) * 2u;   // rows past M / N lie past the ranges: zeros
    const int nsub = K / 16, nch = (nsub + kSmallSub - 1) / kSmallSub;
    i32x4 fa[2][kSmallSub], fb[2][kSmallSub];
    f32x16 acc = {};
    auto load = [&](auto SET, int c) __attribute__((always_inline)) {
        constexpr int u = decltype(SET)::value;
#pragma unroll
        for (int q = 0; q < kSmallSub; q++) {
            const int sub = c * kSmallSub + q;
            const uint32_t off = sub < nsub ? oa + (uint32_t)sub * 32u : kOOB;   // 16 halves a substep
            fa[u][q] = ld16(ra, off);
            fb[u][q] = ld16(rb, off);
        }
    };
    auto mma = [&](auto SET) __attribute__((always_inline)) {
        constexpr int u = decltype(SET)::value;
#pragma unroll
        for (int q = 0; q < kSmallSub; q++)
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, fa[u][q]),
                                                         __builtin_bit_cast(f16x8, fb[u][q]), acc, 0, 0, 0);
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    load(I0{}, 0);
    for (int c = 0; c < nch; c += 2) {
        if (c + 1 < nch) load(I1{}, c + 1);
        mma(I0{});   // (a chunk's substeps past K read zeros: their MFMAs add nothing)
        if (c + 1 < nch) {
            if (c + 2 < nch) load(I0{}, c + 2);
            mma(I1{});
        }
    }
    // lane holds column 32 bn + l % 32 of rows 32 bm + 8 q + 4 h + e (acc element 4 q + e)
    const int n = bn * 32 + r;
    if (n >= N) return;
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int m = bm * 32 + 8 * q + 4 * h + e;
            if (m >= M) continue;
            if constexpr (F16OUT) static_cast<_Float16 *>(C)[(long)m * N + n] = (_Float16)acc[4 * q + e];
            else static_cast<float *>(C)[(long)m * N + n] = acc[4 * q + e];
        }
}

// C = sum of the fp32 planes ws[0..slices) in slice order (the split-K fp16 / fp32 results):
// 4 elements a thread, 16-byte loads when VEC (n % 4 == 0).
template <bool F16OUT, bool VEC>
__global__ __launch_bounds__(256) void k_sum_slices(const float *__restrict__ ws, void *__restrict__ C, long n,
                                                     int slices)
{
    const long i0 = ((long)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i0 >= n) return;
    if (VEC && i0 + 4 <= n) {
        f32x4 acc = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(ws + i0));
        for (int sp = 1; sp < slices; sp++)
            acc += __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(ws + (size_t)sp * n + i0));
        if constexpr (F16OUT) {
            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
            h4 h;
#pragma unroll
            for (int e = 0; e < 4; e++) h[e] = (_Float16)acc[e];
            __builtin_nontemporal_store(h, reinterpret_cast<h4 *>(static_cast<_Float16 *>(C) + i0));
        } else {
            __builtin_nontemporal_store(acc, reinterpret_cast<f32x4 *>(static_cast<float *>(C) + i0));
        }
        return;
    }
    const long i1 = i0 + 4 < n ? i0 + 4 : n;
    for (long i = i0; i < i1; i++) {
        float a = ws[i];
        for (int sp = 1; sp < slices; sp++) a += ws[(size_t)sp * n + i];
        if constexpr (F16OUT) static_cast<_Float16 *>(C)[i] = (_Float16)a;
        else static_cast<float *>(C)[i] = a;
    }
}

// C[0, n) = 0, for the int32 products whose K slices add into C atomically: 4 elements a
// thread, one 16-byte store where whole (C is 16-byte aligned). Ordinary stores: the slices'
// atomic adds find the lines in L2.
__global__ __launch_bounds__(256) void k_zero_i32(int32_t *__restrict__ C, long n)
{
    const long i0 = ((long)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i0 + 4 <= n) {
        *reinterpret_cast<i32x4 *>(C + i0) = i32x4{};
        return;
    }
    for (long i = i0; i < n; i++) C[i] = 0;
}

// Per-row int8 quantisation (one workgroup per row): the row's amax, then
// q = rint(x * (127 / amax)) clamped to [-128, 127], and row_scale = amax / 127. Both
// divisions are IEEE-rounded fp32 divisions and the product one fp32 multiply, so the
// result is the same bits as the host formula. 8 elements a thread per step.
struct QuantArgs {
    int K, n, act;
    int row_start[kMaxProblems + 1];
    const void *A[kMaxProblems];
    const void *A2[kMaxProblems];   // GLU: the up rows (act(A) * A2 is quantised)
    int8_t *Aq[kMaxProblems];
    float *rs[kMaxProblems];
};

template <bool F16IN>
__device__ __forceinline__ void load8f(const void *base, long i, float (&v)[8])
{
    if constexpr (F16IN) {
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
        const h8 h = *reinterpret_cast<const h8 *>(static_cast<const _Float16 *>(base) + i);
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = (float)h[e];
    } else {
        const f32x4 a = *reinterpret_cast<const f32x4 *>(static_cast<const float *>(base) + i);
        const f32x4 b = *reinterpret_cast<const f32x4 *>(static_cast<const float *>(base) + i + 4);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            v[e] = a[e];
            v[4 + e] = b[e];
        }
    }
}

__device__ __forceinline__ void quant_store8(int8_t *dst, const float (&v)[8], float s)
{
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int e = 0; e < 8; e++) {
        int q = (int)__builtin_rintf(v[e] * s);
        q = q > 127 ? 127 : (q < -128 ? -128 : q);
        w[e >> 2] |= (uint32_t)(q & 0xFF) << (8 * (e & 3));
    }
    typedef uint32_t u2 __attribute__((ext_vector_type(2)));
    *reinterpret_cast<u2 *>(dst) = u2{w[0], w[1]};
}

// The 8 row values at element i of problem p: A's (ACT 0), or act(A) * A2 in fp32 (GLU).
template <bool F16IN, int ACT>
__device__ __forceinline__ void row8(const QuantArgs &qa, int p, long i, float (&v)[8])
{
    load8f<F16IN>(qa.A[p], i, v);
    if constexpr (ACT != 0) {
        float u[8];
        load8f<F16IN>(qa.A2[p], i, u);
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = act_k<ACT>(v[e]) * u[e];
    }
}

// Rows of up to 4 x 2048 elements are read once and kept in registers between the amax and
// the quantisation; longer rows are read twice (the second pass mostly from L2, GLU values
// recomputed with the same bits).
template <bool F16IN, int ACT>
__global__ __launch_bounds__(256) void k_quant_rows(const QuantArgs qa)
{
    constexpr int CACHE = 4;
    const int row = blockIdx.x;
    int p = 0;
    while (p + 1 < qa.n && row >= qa.row_start[p + 1]) p++;
    const long m = row - qa.row_start[p], K = qa.K;
    const long base = m * K;
    const int tid = threadIdx.x;
    const bool cached = K <= (long)CACHE * 2048;
    float v[CACHE][8];
    float mx = 0.f;
    if (cached) {
#pragma unroll
        for (int c = 0; c < CACHE; c++) {
            const long k = (long)c * 2048 + tid * 8;
            if (k < K) {
                row8<F16IN, ACT>(qa, p, base + k, v[c]);
#pragma unroll
                for (int e = 0; e < 8; e++) mx = fmaxf(mx, fabsf(v[c][e]));
            }
        }
    } else {
        for (long k = (long)tid * 8; k < K; k += 2048) {
            float t[8];
            row8<F16IN, ACT>(qa, p, base + k, t);
#pragma unroll
            for (int e = 0; e < 8; e++) mx = fmaxf(mx, fabsf(t[e]));
        }
    }
    // workgroup max: within each wave, then across the 4 waves through LDS
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    __shared__ float wmax[4];
    if ((tid & 63) == 0) wmax[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const float s = mx > 0.f ? 127.0f / mx : 0.0f;
    if (tid == 0) qa.rs[p][m] = mx > 0.f ? mx / 127.0f : 0.0f;
    if (cached) {
#pragma unroll
        for (int c = 0; c < CACHE; c++) {
            const long k = (long)c * 2048 + tid * 8;
            if (k < K) quant_store8(qa.Aq[p] + base + k, v[c], s);
        }
    } else {
        for (long k = (long)tid * 8; k < K; k += 2048) {
            float t[8];
            row8<F16IN, ACT>(qa, p, base + k, t);
            quant_store8(qa.Aq[p] + base + k, t, s);
        }
    }
}

// Rows of at most 2048 elements: one wave a row, four rows a workgroup. Each lane keeps its
// (at most 4) 8-element chunks in registers; the row's amax is reduced by cross-lane shuffles
// alone (no LDS, no barrier: a wave past the last row returns at once). The amax is the same
// maximum and the codes the same formula as k_quant_rows, so the bits are the same.
template <bool F16IN, int ACT>
__global__ __launch_bounds__(256) void k_quant_rows_w(const QuantArgs qa, int rows)
{
    constexpr int CH = 4;
    const int row = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (row >= rows) return;
    const int lane = threadIdx.x & 63;
    int p = 0;
    while (p + 1 < qa.n && row >= qa.row_start[p + 1]) p++;
    const long m = row - qa.row_start[p], K = qa.K;
    const long base = m * K;
    float v[CH][8];
    float mx = 0.f;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const long k = (long)(c * 64 + lane) * 8;
        if (k < K) {
            row8<F16IN, ACT>(qa, p, base + k, v[c]);
#pragma unroll
            for (int e = 0; e < 8; e++) mx = fmaxf(mx, fabsf(v[c][e]));
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    const float s = mx > 0.f ? 127.0f / mx : 0.0f;
    if (lane == 0) qa.rs[p][m] = mx > 0.f ? mx / 127.0f : 0.0f;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const long k = (long)(c * 64 + lane) * 8;
        if (k < K) quant_store8(qa.Aq[p] + base + k, v[c], s);
    }
}

// int4 packing: one thread per packed dword (8 values of K).
__global__ void k_pack_int4(const int8_t *__restrict__ src, uint32_t *__restrict__ dst, long total_words, int words_per_row, int K)
{
    const long w = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (w >= total_words) return;
    const long row = w / words_per_row;
    const int d = (int)(w % words_per_row);
    const int8_t *s = src + row * (long)K + 8L * d;
    uint32_t out = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t hi = (uint32_t)(uint8_t)s[j] & 0xFu, lo = (uint32_t)(uint8_t)s[j + 4] & 0xFu;
        out |= ((hi << 4) | lo) << (8 * j);
    }
    dst[w] = out;
}

// fp32 -> bf16 (SPLIT false: 16 output bytes per 8 values) or tf32 hi/lo bf16 pairs (SPLIT
// true: 32 bytes), one 8-value chunk a lane. The fp32 source is read once: non-temporal.
// Chunks [0, n0) come from the first array, the next n1 from the second (one launch for
// both operands of a product: no second kernel's ramp and drain).
template <bool SPLIT>
__global__ __launch_bounds__(256) void k_cvt_f32(const i32x4 *__restrict__ src0, i32x4 *__restrict__ dst0, long n0,
                                                 const i32x4 *__restrict__ src1, i32x4 *__restrict__ dst1, long n1)
{
    long c = (long)blockIdx.x * 256 + threadIdx.x;
    if constexpr (!SPLIT) {
        // a wave's 64 chunks (2 KB of fp32) inside one array: lane l converts values 4 l .. + 3
        // and 256 + 4 l .. + 3 of the window, so each load instruction reads 1 KB and each
        // store writes 512 B contiguous
        const long w0 = c - (threadIdx.x & 63);
        const int lane = threadIdx.x & 63;
        const bool a0 = w0 + 64 <= n0, a1 = w0 >= n0 && w0 + 64 <= n0 + n1;
        if (a0 || a1) {
            const long base = (a0 ? w0 : w0 - n0) * 2;   // in 16-byte fp32 units
            const i32x4 *sp = (a0 ? src0 : src1) + base;
            int *dp = reinterpret_cast<int *>(a0 ? dst0 : dst1) + base * 2;
            const i32x4 x = __builtin_nontemporal_load(sp + lane), y = __builtin_nontemporal_load(sp + 64 + lane);
            typedef int i2 __attribute__((ext_vector_type(2)));
            *reinterpret_cast<i2 *>(dp + 2 * lane) = i2{bf16pack(x[0], x[1]), bf16pack(x[2], x[3])};
            *reinterpret_cast<i2 *>(dp + 128 + 2 * lane) = i2{bf16pack(y[0], y[1]), bf16pack(y[2], y[3])};
            return;
        }
    }
    const i32x4 *src = src0;
    i32x4 *dst = dst0;
    if (c >= n0) {
        c -= n0;
        if (c >= n1) return;
        src = src1;
        dst = dst1;
    }
    const i32x4 a = __builtin_nontemporal_load(src + 2 * c), b = __builtin_nontemporal_load(src + 2 * c + 1);
    if constexpr (!SPLIT) {
        dst[c] = bf16x8_of(a, b);
    } else {
        i32x4 vh, vl;
        tf32x8_split(a, b, vh, vl);
        dst[2 * c] = vh;
        dst[2 * c + 1] = vl;
    }
}


// Workgroups are renumbered over this many XCDs (MI355X has 8); ROCKET_HIP_XCD overrides,
// 1 keeps the hardware order.
int xcd_count()
{
    static const int n = [] {   // read once (a function-local static initialises thread-safely)
        const char *e = getenv("ROCKET_HIP_XCD");
        const int v = e ? atoi(e) : 8;
        return (v < 1 || v > 64) ? 8 : v;
    }();
    return n;
}

// Row-band height of one-problem launches: ROCKET_HIP_BANDM unset = chosen per launch, 0 =
// plain M-fastest order, n = bands of n row tiles (read per call).
int bandm_override()
{
    const char *e = getenv("ROCKET_HIP_BANDM");
    if (!e) return -1;
    const int n = atoi(e);
    return (n >= 0 && n <= (1 << 20)) ? n : -1;
}

// Upper bound on split-K slices: 4 for fp16 / bf16 products whose tiles leave CUs idle
// (partial planes summed by a second kernel) and for int32 products with few outputs (slices
// add into C with atomics, see choose). ROCKET_HIP_SPLITK sets both (1 = off, 2, 4, 8; read
// per call).
int splitk_cap()
{
    const char *e = getenv("ROCKET_HIP_SPLITK");
    const int n = e ? atoi(e) : 4;
    return (n >= 1 && n <= 8) ? n : 1;
}

// 256 x 256 fp16 / bf16 tiles where they would be chosen; ROCKET_HIP_WIDE=0 keeps 256 x 128
// (read per call).
bool wide_tiles()
{
    const char *e = getenv("ROCKET_HIP_WIDE");
    return !e || atoi(e) != 0;
}

long row_bytes(Fmt f, int K)
{
    switch (f) {
    case Fmt::I8: return K;
    case Fmt::I4P: return K / 2;
    case Fmt::I16: case Fmt::F16: case Fmt::BF16: return 2L * K;
    case Fmt::F32BF16: case Fmt::F32TF32: case Fmt::BF16X2: return 4L * K;
    }
    return 0;
}

int stage_k(Fmt f) { return (f == Fmt::I8 || f == Fmt::I4P || f == Fmt::I16) ? 128 : 64; }

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

uint64_t div_magic(int d) { return ((uint64_t)1 << 38) / (uint64_t)(d >> 5) + 1; }

struct Choice { int bm, bn, splitk; };

// Tile shape and split-K factor. tiles(bm, bn) counts workgroups of one K slice.
// outs: output elements of the launch.
template <class TilesFn>
Choice choose(Fmt fa, Fmt fb, Epi epi, int maxM, int kspan, long outs, bool accum_ok, TilesFn tiles)
{
    // Enough tiles to give every CU a workgroup (256 CUs); a CU needs roughly 64 operand
    // bytes of MFMA work per L2 byte, which 256 x 128 int8 tiles give and 64 x 64 do not.
    const long cus = 256;
    if (epi == Epi::GW) {
        // int32 + fp32 accumulators: 64 x 64 a wave, two waves per SIMD. 256 x 128 (8 waves,
        // one workgroup per CU) when the rows fill it and it still gives most CUs a tile.
        if (maxM > 128 && tiles(256, 128) >= cus * 3 / 4) return {256, 128, 1};
        if (tiles(128, 128) >= cus * 3 / 4) return {128, 128, 1};
        if (tiles(128, 64) >= cus / 2) return {128, 64, 1};
        return {64, 64, 1};
    }
    if (epi == Epi::I32) {
        // int8 / int4 to int32: the largest tile the rows fill, then split K (slices add into
        // C atomically, exact in any order) until every CU has a workgroup — while the atomic
        // adds stay few: at 512 x 4096 x 4096 (4 slices of 256 x 128 tiles, 33.5 M atomic
        // adds) the product took 35.5 us against 18 us whole in 128 x 64 tiles
        Choice c = maxM > 128 ? Choice{256, 128, 1} : (maxM > 64 ? Choice{128, 128, 1} : Choice{64, 64, 1});
        const long t = tiles(c.bm, c.bn);
        if (accum_ok)
            while (c.splitk * 2 <= splitk_cap() && t * c.splitk * 2 <= cus && kspan / (c.splitk * 2) >= 512 &&
                   outs * c.splitk * 2 <= (1L << 20))
                c.splitk *= 2;
        if (t * c.splitk >= cus / 2 || c.bm == 64) return c;
        // too little K to split: smaller tiles instead
        if (tiles(128, 64) >= cus / 2) return {128, 64, 1};
        return {64, 64, 1};
    }
    if (epi == Epi::GLU) {   // gate and up column blocks pair inside 64-row groups of B tile rows
        if (fa == Fmt::F16 && fb == fa && wide_tiles() && tiles(256, 256) >= cus * 15 / 16) return {256, 256, 1};
        return tiles(256, 128) >= cus * 15 / 16 ? Choice{256, 128, 1} : Choice{128, 128, 1};
    }
    const bool two_plane = (fa == Fmt::I16 || fa == Fmt::F32TF32 || fa == Fmt::BF16X2);
    // fp16 / bf16 operands in LDS: 256 x 256 tiles when they alone cover the CUs (a third fewer
    // operand bytes per MFMA than 256 x 128: fp16 512 x 3840 x 30720 172 -> 159 us, 2048 x 3840 x
    // 15360 333 -> 285 us; in K slices (up to 8, 240 workgroups) no faster than 256 x 128 tiles:
    // config 4 341 us a call either way, the FFN's down product within noise, 512 x 3840 x 15360
    // 100 against 85 us)
    const bool wide_ok = fb == fa && ((fa == Fmt::F16 && (epi == Epi::F16 || epi == Epi::F32 || epi == Epi::ACT)) ||
                                      (fa == Fmt::BF16 && epi == Epi::F32));
    if (wide_ok && wide_tiles() && tiles(256, 256) >= cus * 15 / 16) return {256, 256, 1};
    if (!two_plane && tiles(256, 128) >= cus * 15 / 16) return {256, 128, 1};
    if (accum_ok && !two_plane && maxM > 128) {
        // fp16 / bf16 with long K: 256 x 128 tiles in K slices until the CUs are covered
        // (each slice keeps at least 2048 K values)
        Choice c{256, 128, 1};
        const long t = tiles(256, 128);
        while (c.splitk * 2 <= splitk_cap() && t * c.splitk * 2 <= cus && kspan / (c.splitk * 2) >= 2048)
            c.splitk *= 2;
        if (c.splitk > 1 && t * c.splitk >= cus * 3 / 4) return c;
    }
    if (fa != Fmt::I16 && tiles(128, 128) >= cus * 15 / 16) return {128, 128, 1};
    if (tiles(128, 64) >= cus / 2) return {128, 64, 1};
    return {64, 64, 1};
}

// Tile geometry and K slices of a launch whose largest problem has maxM rows. Slices cover
// whole stages and none is empty.
struct Plan {
    int bm, bn, splitk, kper;
    long ntiles;
    bool planes;   // K slices: partial planes summed by a second kernel
    bool atomic;   // K slices of an int32 product: atomic adds into C
    int m0, n;     // the (single) problem's M and N, for the planes
};

Plan plan_of(const Launch &L, int maxM, bool allow_split)
{
    const int kspan = L.kend - L.kbeg;
    auto tiles = [&](int tm, int tn) {
        long t = 0;
        for (int i = 0; i < L.nprob; i++) t += (long)((L.prob[i].M + tm - 1) / tm) * ((L.N + tn - 1) / tn);
        return t;
    };
    // split-K for plain int32 results (any slice count combines exactly) and for fp16 / fp32
    // results of a launch that does not accumulate into C (slices summed in a fixed order)
    const bool fp = (L.epi == Epi::F16 || L.epi == Epi::F32);
    const bool split_ok = allow_split && L.nprob == 1 && (L.epi == Epi::I32 || (fp && !L.accum));
    long outs = 0;
    for (int i = 0; i < L.nprob; i++) outs += (long)L.prob[i].M * L.N;
    const Choice c = choose(L.fmt_a, L.fmt_b, L.epi, maxM, kspan, outs, split_ok, tiles);
    Plan p;
    p.bm = c.bm;
    p.bn = c.bn;
    const int ks = stage_k(L.fmt_a);
    const int nst = (kspan + ks - 1) / ks;
    p.splitk = std::min(c.splitk, nst);
    p.kper = ((nst + p.splitk - 1) / p.splitk) * ks;
    p.splitk = (kspan + p.kper - 1) / p.kper;
    p.ntiles = tiles(p.bm, p.bn);
    p.atomic = p.splitk > 1 && L.epi == Epi::I32;
    p.planes = p.splitk > 1 && !p.atomic;
    p.m0 = L.prob[0].M;
    p.n = L.N;
    return p;
}

// [slice][M][N] planes of fp32 partials
size_t ws_bytes_of(const Plan &p)
{
    return p.planes ? (size_t)p.splitk * p.m0 * p.n * 4 : 0;
}


}  // namespace

// The family of a launch's operand formats and epilogue (one translation unit each).
hipError_t dispatch(int bm, int bn, const Launch &L, const KArgs &ka, int blocks)
{
    if (L.epi == Epi::GW) return L.fmt_b == Fmt::I4P ? dispatch_gw_i4(bm, bn, L, ka, blocks)
                                                     : dispatch_gw_i8(bm, bn, L, ka, blocks);
    if (L.fmt_a == Fmt::I8 || L.fmt_a == Fmt::I16) return dispatch_int(bm, bn, L, ka, blocks);
    if (L.fmt_a == Fmt::F16) return dispatch_f16(bm, bn, L, ka, blocks);
    return dispatch_bf16(bm, bn, L, ka, blocks);
}

}  // namespace gk

using namespace gk;

size_t gemm_ws_bytes(const Launch &L)
{
    if ((L.epi != Epi::I32 && L.epi != Epi::F16 && L.epi != Epi::F32) || L.nprob < 1 || L.nprob > kMaxProblems ||
        L.kend <= L.kbeg)
        return 0;
    int maxM = 0;
    for (int i = 0; i < L.nprob; i++) maxM = std::max(maxM, L.prob[i].M);
    if (maxM <= 0) return 0;
    const Plan p = plan_of(L, maxM, true);
    return ws_bytes_of(p);
}

void gemm_tile(Fmt fmt_a, Epi epi, int M, int N, int *bm, int *bn)
{
    auto tiles = [&](int tm, int tn) { return (long)((M + tm - 1) / tm) * ((N + tn - 1) / tn); };
    const Choice c = choose(fmt_a, fmt_a, epi, M, 0, (long)M * N, false, tiles);
    *bm = c.bm;
    *bn = c.bn;
}

hipError_t gemm_launch(const Launch &L, uint64_t *blocks_out)
{
    if (blocks_out) *blocks_out = 0;
    // what the kernels assume: K in whole 32-element chunks, N in whole 16-column blocks,
    // 16-byte aligned operand rows, a valid K range and problem count
    if (L.nprob < 1 || L.nprob > kMaxProblems || L.N <= 0 || L.K <= 0) return hipErrorInvalidValue;
    if (L.f16out && L.epi != Epi::GW) return hipErrorInvalidValue;
    if (L.K % 32 != 0 && !(L.K % 16 == 0 && (L.fmt_a == Fmt::F32TF32 || L.fmt_a == Fmt::BF16X2)))
        return hipErrorInvalidValue;
    if (L.N % 16 != 0) return hipErrorInvalidValue;
    if (L.kbeg < 0 || L.kend > L.K || L.kbeg >= L.kend || L.kbeg % 128 != 0) return hipErrorInvalidValue;
    if (L.fmt_b == Fmt::I4P && (L.K % 32 != 0)) return hipErrorInvalidValue;
    const long nG = L.group ? L.K / L.group : 0;
    if (L.epi == Epi::GW) {
        if (L.group < 32 || L.group % 32 || L.K % L.group || L.kt < 32 || L.kt % 32 || L.group % L.kt)
            return hipErrorInvalidValue;
        if (L.kbeg != 0 || L.kend != L.K || L.accum) return hipErrorInvalidValue;
        if (L.fmt_a != Fmt::I8) return hipErrorInvalidValue;
        // scale arrays are addressed with 32-bit byte offsets
        if ((long)L.N * nG * 4 >= (1L << 31)) return hipErrorInvalidValue;
    } else if (L.rowscale) {
        return hipErrorInvalidValue;
    }
    if (L.epi == Epi::GLU || L.epi == Epi::ACT) {
        if (L.fmt_a != Fmt::F16 || L.fmt_b != Fmt::F16 || L.kbeg != 0 || L.kend != L.K || L.accum) return hipErrorInvalidValue;
        if (L.act != kActSilu && L.act != kActGelu && !(L.epi == Epi::ACT && L.act == kActIdentity))
            return hipErrorInvalidValue;
        if (L.epi == Epi::GLU && L.N % 64) return hipErrorInvalidValue;   // gate and up of N/2 % 32 columns
    }
    const long lda = row_bytes(L.fmt_a, L.K), ldb = row_bytes(L.fmt_b, L.K);
    if (lda % 16 || ldb % 16) return hipErrorInvalidValue;

    int maxM = 0;
    for (int i = 0; i < L.nprob; i++) {
        const Problem &P = L.prob[i];
        if (P.M < 0) return hipErrorInvalidValue;
        if (P.M == 0) continue;
        if (!P.A || !P.B || !P.C) return hipErrorInvalidValue;
        if (!aligned16(P.A) || !aligned16(P.B) || !aligned16(P.C)) return hipErrorInvalidValue;
        if (L.epi == Epi::GW && (!P.a_scale || !P.b_scale)) return hipErrorInvalidValue;
        if (L.epi == Epi::GLU && (!P.B2 || !aligned16(P.B2))) return hipErrorInvalidValue;
        if (L.epi == Epi::ACT && P.B2 && ((uintptr_t)P.B2 & 1u)) return hipErrorInvalidValue;
        if (L.epi == Epi::GW && !L.rowscale && (long)P.M * nG * 4 >= (1L << 31)) return hipErrorInvalidValue;
        if (P.dump) {   // group-wise partials of whole groups, rows inside the problem, 32-bit offsets
            if (L.epi != Epi::GW || L.kt != L.group || ((uintptr_t)P.dump & 3u)) return hipErrorInvalidValue;
            if (P.dump_row0 < 0 || P.dump_rows < 1 || P.dump_row0 + P.dump_rows > P.M) return hipErrorInvalidValue;
            if ((long)(P.M + 256) * nG * L.N * 4 >= (1L << 31)) return hipErrorInvalidValue;
        }
        maxM = std::max(maxM, P.M);
    }
    if (maxM == 0) return hipSuccess;

    // a small fp16 product (whole K, one problem, few 32 x 32 blocks): the direct kernel
    if (L.fmt_a == Fmt::F16 && L.fmt_b == Fmt::F16 && (L.epi == Epi::F16 || L.epi == Epi::F32) && L.nprob == 1 &&
        !L.accum && L.kbeg == 0 && L.kend == L.K && L.K <= 1024) {
        const Problem &P = L.prob[0];
        const int nbm = (P.M + 31) / 32, nbn = (L.N + 31) / 32;
        if ((long)nbm * nbn <= 64) {
            const auto *A = static_cast<const _Float16 *>(P.A), *B = static_cast<const _Float16 *>(P.B);
            if (L.epi == Epi::F16)
                hipLaunchKernelGGL(k_small_f16<true>, dim3(nbm * nbn), dim3(64), 0, L.stream, A, B, P.C, P.M, L.N, L.K, nbn);
            else
                hipLaunchKernelGGL(k_small_f16<false>, dim3(nbm * nbn), dim3(64), 0, L.stream, A, B, P.C, P.M, L.N, L.K, nbn);
            if (blocks_out) *blocks_out = (uint64_t)nbm * nbn;
            return hipGetLastError();
        }
    }

    Plan pl = plan_of(L, maxM, true);
    if (pl.planes && (!L.ws || L.ws_bytes < ws_bytes_of(pl)))
        pl = plan_of(L, maxM, false);   // no workspace: the best plan with one slice per tile
    const int bm = pl.bm, bn = pl.bn;
    // every operand tile is addressed with 32-bit byte offsets
    if ((long)bm * lda >= (1L << 31) || (long)bn * ldb >= (1L << 31)) return hipErrorInvalidValue;

    KArgs ka;
    ka.N = L.N; ka.K = L.K; ka.kbeg = L.kbeg; ka.kend = L.kend; ka.accum = L.accum;
    ka.group = L.group; ka.kt = L.kt; ka.nG = (int)nG;
    ka.gmag = L.group ? div_magic(L.group) : 0;
    ka.tmag = L.kt ? div_magic(L.kt) : 0;
    ka.lda = (uint32_t)lda; ka.ldb = (uint32_t)ldb;
    ka.nprob = L.nprob;
    ka.xcds = xcd_count();
    ka.act = L.act;
    ka.f16out = L.f16out;
    ka.splitk = pl.splitk;
    ka.kper = pl.kper;
    ka.ws = L.ws;
    ka.atomic = pl.atomic ? 1 : 0;
    const int nbn = (L.N + bn - 1) / bn;
    // Group-wise kernels with short groups skip the waves whose rows lie past M, so a last
    // row tile with at most half its rows costs little: such "light" tiles run after all
    // the others (see k_gemm). At Gemma MoE shapes (experts of 1024 +- 30 rows) they took
    // 12-19% of the gate/up launch and 30% of the down launch as a round of their own.
    const int cad = L.epi == Epi::GW ? gw_cadence(L) : 0;
    const bool order = ka.splitk == 1 && (cad == 1 || cad == 2);
    // Problems that read the same activations (the gate and up products of one expert) are
    // numbered next to each other (first appearance order otherwise kept), so their tiles run
    // as consecutive workgroups of one XCD and its L2 serves the shared rows to both.
    int ord[kMaxProblems];
    {
        int n = 0;
        bool used[kMaxProblems] = {};
        for (int i = 0; i < L.nprob; i++) {
            if (used[i]) continue;
            for (int j = i; j < L.nprob; j++)
                if (!used[j] && L.prob[j].A == L.prob[i].A) {
                    used[j] = true;
                    ord[n++] = j;
                }
        }
    }
    long ntiles = 0, nlight = 0;
    for (int i = 0; i < L.nprob; i++) {
        ka.prob[i] = L.prob[ord[i]];
        const int M = ka.prob[i].M, rem = M % bm;
        const bool light = order && rem != 0 && rem <= bm / 2;
        ka.tile_start[i] = (int)ntiles;
        ka.light_start[i] = (int)nlight;
        ntiles += (long)((M + bm - 1) / bm - (light ? 1 : 0)) * nbn;
        nlight += light ? nbn : 0;
    }
    ka.tile_start[L.nprob] = (int)ntiles;
    ka.light_start[L.nprob] = (int)nlight;
    const long blocks = ntiles * ka.splitk + nlight;
    ka.nheavy = (int)(ntiles * ka.splitk);
    // Row bands (one problem): an XCD's consecutive tiles cover h row blocks of A and about
    // per / h column blocks of B, per = its share of the tiles. Plain M-fastest order is
    // h = all heavy row tiles, which at M >= 1024 makes every XCD stream all of A; the band
    // height minimising h * (A row-block bytes) + ceil(per / h) * (B column-block bytes) is
    // taken where it beats that (M = 2048 bf16 with 256 x 128 tiles: 4 of 8 row tiles).
    ka.bandm = 0;
    ka.nbn = nbn;
    if (L.nprob == 1 && ntiles > 0) {
        const long nbh = ntiles / nbn, per = (ntiles + ka.xcds - 1) / ka.xcds;
        const int ov = bandm_override();
        if (ov >= 0) {
            if (ov < nbh) ka.bandm = ov;
        } else if (ka.xcds > 1) {
            const auto cost = [&](long h) { return h * bm * (double)lda + (double)((per + h - 1) / h) * bn * (double)ldb; };
            long best = nbh;
            for (long h = nbh - 1; h >= 1; h--)
                if (cost(h) < cost(best)) best = h;
            if (best < nbh) ka.bandm = (int)best;
        }
    }
    if (blocks > 0x7FFFFFFFL) return hipErrorInvalidValue;
    if (blocks_out) *blocks_out = (uint64_t)blocks;

    if (pl.atomic && !L.accum) {   // the slices add into C: it starts from zero
        const long n = (long)L.prob[0].M * L.N, zblocks = (n / 4 + 255) / 256 + 1;
        if (zblocks > 0x7FFFFFFFL) return hipErrorInvalidValue;
        hipLaunchKernelGGL(k_zero_i32, dim3((unsigned)zblocks), dim3(256), 0, L.stream,
                           static_cast<int32_t *>(L.prob[0].C), n);
        if (blocks_out) *blocks_out += (uint64_t)zblocks;
    }
    hipError_t e = dispatch(bm, bn, L, ka, (int)blocks);
    if (e != hipSuccess || !pl.planes) return e;
    // sum the slices' planes into C
    const long n = (long)pl.m0 * pl.n, rblocks = (n + 1023) / 1024;
    if (rblocks > 0x7FFFFFFFL) return hipErrorInvalidValue;
    const float *wsf = reinterpret_cast<const float *>(L.ws);
    void *C = const_cast<void *>(L.prob[0].C);
    const bool vec = n % 4 == 0;
    if (L.epi == Epi::F16) {
        if (vec) hipLaunchKernelGGL((k_sum_slices<true, true>), dim3((unsigned)rblocks), dim3(256), 0, L.stream, wsf, C, n, pl.splitk);
        else hipLaunchKernelGGL((k_sum_slices<true, false>), dim3((unsigned)rblocks), dim3(256), 0, L.stream, wsf, C, n, pl.splitk);
    } else {
        if (vec) hipLaunchKernelGGL((k_sum_slices<false, true>), dim3((unsigned)rblocks), dim3(256), 0, L.stream, wsf, C, n, pl.splitk);
        else hipLaunchKernelGGL((k_sum_slices<false, false>), dim3((unsigned)rblocks), dim3(256), 0, L.stream, wsf, C, n, pl.splitk);
    }
    if (blocks_out) *blocks_out += (uint64_t)rblocks;
    return hipGetLastError();
}

hipError_t pack_int4(const int8_t *src, uint8_t *dst, int N, int K, hipStream_t s)
{
    if (N <= 0 || K <= 0 || K % 8) return hipErrorInvalidValue;
    const long words = (long)N * (K / 8);
    const int tpb = 256;
    hipLaunchKernelGGL(k_pack_int4, dim3((unsigned)((words + tpb - 1) / tpb)), dim3(tpb), 0, s,
                       src, reinterpret_cast<uint32_t *>(dst), words, K / 8, K);
    return hipGetLastError();
}

hipError_t quant_rows(const QuantRows &q, hipStream_t s, uint64_t *blocks_out)
{
    if (blocks_out) *blocks_out = 0;
    if (q.n < 1 || q.n > kMaxProblems || q.K <= 0 || q.K % 8) return hipErrorInvalidValue;
    const bool glu = q.act != 0;
    if (glu && q.act != kActSilu && q.act != kActGelu) return hipErrorInvalidValue;
    QuantArgs qa;
    qa.K = q.K;
    qa.n = q.n;
    qa.act = q.act;
    long rows = 0;
    for (int p = 0; p < q.n; p++) {
        if (q.M[p] < 0) return hipErrorInvalidValue;
        if (q.M[p] && (!aligned16(q.A[p]) || ((uintptr_t)q.Aq[p] & 7) || !q.row_scale[p])) return hipErrorInvalidValue;
        if (q.M[p] && glu && !aligned16(q.A2[p])) return hipErrorInvalidValue;
        qa.row_start[p] = (int)rows;
        qa.A[p] = q.A[p];
        qa.A2[p] = glu ? q.A2[p] : nullptr;
        qa.Aq[p] = q.Aq[p];
        qa.rs[p] = q.row_scale[p];
        rows += q.M[p];
    }
    for (int p = q.n; p <= kMaxProblems; p++) qa.row_start[p] = (int)rows;
    if (rows == 0) return hipSuccess;
    if (rows > 0x7FFFFFFFL) return hipErrorInvalidValue;
    // rows of up to 2048 elements: a wave each (a 256-thread workgroup per row would leave
    // threads idle and pay a barrier per row: the MoE down products' 1408-element gated rows
    // took 27 us for 104 MB)
    const bool wave = q.K <= 2048;
    const long blocks = wave ? (rows + 3) / 4 : rows;
    const int nr = (int)rows;
    // one instantiation per (fp16 input, activation kind)
    auto launch = [&](auto F16T, auto ACTT) {
        constexpr bool F = decltype(F16T)::value;
        constexpr int A = decltype(ACTT)::value;
        if (wave) hipLaunchKernelGGL((k_quant_rows_w<F, A>), dim3((unsigned)blocks), dim3(256), 0, s, qa, nr);
        else hipLaunchKernelGGL((k_quant_rows<F, A>), dim3((unsigned)rows), dim3(256), 0, s, qa);
    };
    auto by_act = [&](auto F16T) {
        if (q.act == kActSilu) launch(F16T, std::integral_constant<int, kActSilu>{});
        else if (q.act == kActGelu) launch(F16T, std::integral_constant<int, kActGelu>{});
        else launch(F16T, std::integral_constant<int, 0>{});
    };
    if (q.f16) by_act(std::true_type{});
    else by_act(std::false_type{});
    if (blocks_out) *blocks_out = (uint64_t)blocks;
    return hipGetLastError();
}

hipError_t convert_f32(const float *src, void *dst, long n, Fmt to, hipStream_t s, const float *src2, void *dst2,
                       long n2)
{
    if (n <= 0 || n % 8 || !aligned16(src) || !aligned16(dst) || (to != Fmt::BF16 && to != Fmt::BF16X2))
        return hipErrorInvalidValue;
    if (n2 < 0 || n2 % 8 || (n2 && (!aligned16(src2) || !aligned16(dst2)))) return hipErrorInvalidValue;
    const long c0 = n / 8, c1 = n2 / 8, blocks = (c0 + c1 + 255) / 256;
    if (blocks > 0x7FFFFFFFL) return hipErrorInvalidValue;
    const i32x4 *in0 = reinterpret_cast<const i32x4 *>(src), *in1 = reinterpret_cast<const i32x4 *>(src2);
    i32x4 *out0 = static_cast<i32x4 *>(dst), *out1 = static_cast<i32x4 *>(dst2);
    if (to == Fmt::BF16)
        hipLaunchKernelGGL(k_cvt_f32<false>, dim3((unsigned)blocks), dim3(256), 0, s, in0, out0, c0, in1, out1, c1);
    else
        hipLaunchKernelGGL(k_cvt_f32<true>, dim3((unsigned)blocks), dim3(256), 0, s, in0, out0, c0, in1, out1, c1);
    return hipGetLastError();
}

hipError_t geglu_f16(const _Float16 *gate, const _Float16 *up, _Float16 *prod, long n, int act, hipStream_t s)
{
    if (n <= 0 || (act != kActSilu && act != kActGelu)) return hipErrorInvalidValue;
    const long blocks = (n + 2047) / 2048;
    if (blocks > 0x7FFFFFFFL) return hipErrorInvalidValue;
    const bool vec = ((reinterpret_cast<uintptr_t>(gate) | reinterpret_cast<uintptr_t>(up) |
                       reinterpret_cast<uintptr_t>(prod)) & 15) == 0;
    if (act == kActGelu) {
        if (vec) hipLaunchKernelGGL((k_geglu<true, kActGelu>), dim3((unsigned)blocks), dim3(256), 0, s, gate, up, prod, n);
        else hipLaunchKernelGGL((k_geglu<false, kActGelu>), dim3((unsigned)blocks), dim3(256), 0, s, gate, up, prod, n);
    } else {
        if (vec) hipLaunchKernelGGL((k_geglu<true, kActSilu>), dim3((unsigned)blocks), dim3(256), 0, s, gate, up, prod, n);
        else hipLaunchKernelGGL((k_geglu<false, kActSilu>), dim3((unsigned)blocks), dim3(256), 0, s, gate, up, prod, n);
    }
    return hipGetLastError();
}


}  // namespace rk
