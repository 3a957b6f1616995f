// gemm_impl.h — the gfx950 MFMA GEMM kernel template shared by the translation units that
// instantiate it (gemm_int.hip, gemm_gw8.hip, gemm_gw4.hip, gemm_f16.hip, gemm_bf16.hip; one
// operand family each, so the instantiations compile in parallel) and by gemm.hip, which
// plans launches and holds the streaming kernels.
//
// C[M,N] = A[M,K] * B[N,K]^T with both operands K-contiguous. One workgroup owns a
// BM x BN output tile (optionally one K slice of it: split-K); its waves own sub-tiles
// built from MFMA result blocks: 32x32 (v_mfma_i32_32x32x32_i8, v_mfma_f32_32x32x16_{f16,bf16})
// or, for fp16 / bf16 on 256-row tiles, 16x16 (v_mfma_f32_16x16x32_{f16,bf16}; the same
// rate and operand bytes per flop for a given wave tile, measured 7% faster there; the int8
// 16x16x64 shape measured slower: config 3 53.9 against 47.9 us, int8 at its shape 40.4
// against 38.6 us). K
// advances in stages of 128 LDS bytes per tile row; each stage goes global -> LDS (by DMA,
// or through registers) while earlier stages feed the MFMAs, one barrier per stage.
//
// Global loads are buffer loads: each lane's offsets inside the tile are computed once,
// the K position and the valid byte range of a stage live in the (scalar) buffer
// descriptor, and the hardware range check returns zeros for rows past M / N and for
// stages past the end of K. Only a partial last stage masks chunks per lane.
//
// MFMA operand convention: the A fragment is the instruction's first operand and the B
// fragment its second, so in each 32x32 result block lane l holds column n = l % 32 and
// rows 8q + 4(l/32) + r in register 4q + r (q, r = 0..3): one output column per lane,
// which makes every C store a pair of 128-byte row segments and gives group-wise
// epilogues one B scale per lane and block. Lane l supplies row l % 32 of each fragment
// and bytes [16*(l/32), +16) of the 32-byte K substep, identically for both operands.
// In a 16x16 block lane l holds column l % 16 and rows 4(l/16) + r in register r, and
// supplies row l % 16 and bytes [16*(l/16), +16) of a 64-byte K substep.
#pragma once

#include "gemm.h"

#include <stdlib.h>

#include <algorithm>
#include <atomic>
#include <type_traits>

namespace rk {
namespace gk {


typedef int      i32x4  __attribute__((ext_vector_type(4)));
typedef float    f32x4  __attribute__((ext_vector_type(4)));
typedef float    f32x16 __attribute__((ext_vector_type(16)));
typedef int      i32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8  __attribute__((ext_vector_type(8)));
typedef __bf16   bf16x8 __attribute__((ext_vector_type(8)));
typedef long long i64;
typedef __amdgpu_buffer_rsrc_t Rsrc;

constexpr int ROWB = 128;                 // LDS bytes per tile row per plane per stage
constexpr uint32_t kOOB = 0x80000000u;    // an offset past every operand range: loads return 0

// Chunk c of row r sits at slot c ^ ((r >> 1) & 7): the sixteen lanes an LDS cycle serves
// (sixteen consecutive rows, one chunk) cover all 64 banks once.
__device__ __forceinline__ int swz(int row, int chunk) { return row * ROWB + ((chunk ^ ((row >> 1) & 7)) << 4); }

// Buffer descriptor over [base, base + bytes). Word 3 selects the raw 32-bit data format
// of the gfx9 family (a zero format would make every access out of range).
__device__ __forceinline__ Rsrc rsrc(const void *base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
// The same over a base and size that every lane holds alike, read from the first lane: the
// descriptor then stays in SGPRs even where the compiler cannot prove the values uniform
// (a descriptor in VGPRs wraps each buffer access in a readfirstlane loop).
__device__ __forceinline__ Rsrc rsrc_u(const void *base, uint32_t bytes)
{
    const uint64_t a = (uint64_t)(uintptr_t)base;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
    return rsrc(reinterpret_cast<const void *>(((uint64_t)hi << 32) | lo),
                (uint32_t)__builtin_amdgcn_readfirstlane((int)bytes));
}
__device__ __forceinline__ i32x4 ld16(Rsrc r, uint32_t off)
{
    return __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ float ld4f(Rsrc r, uint32_t off)
{
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

// floor(k / d) for a divisor d that is a multiple of 32 (d < 2^24, 0 <= k < 2^24 + 2^12):
// (k / 32) * mag >> 38 with mag = 2^38 / (d / 32) + 1 (host: div_magic). Exact on that range.
__device__ __forceinline__ int div32m(int k, uint64_t mag)
{
    return (int)(((uint64_t)((uint32_t)k >> 5) * mag) >> 38);
}

// ------------------------------------------------------------------------------------
// Kernel arguments (passed by value: the problem table travels in the kernarg segment).
// ------------------------------------------------------------------------------------
struct KArgs {
    int N, K, kbeg, kend, accum, group, kt, nG;
    uint32_t lda, ldb;                   // bytes per row of A and of B
    uint64_t gmag, tmag;                 // div32m magics for group and kt
    int splitk, kper;                    // K slices per tile and the K elements of one slice
    int32_t *ws;                         // fp split-K: [slice][M][N] fp32 partial planes
    int nprob;
    int tile_start[kMaxProblems + 1];    // prefix sums of per-problem heavy tile counts
    int light_start[kMaxProblems + 1];   // prefix sums of per-problem light tile counts
    int nheavy;                          // workgroups of heavy tiles (x K slices); light ones follow
    Problem prob[kMaxProblems];
    int xcds;                            // XCDs to renumber workgroups over (1: keep order)
    int bandm, nbn;                      // one problem: heavy tiles M-fastest in bands of bandm row tiles (0: one band); column blocks
    int act;                             // GLU / ACT activation (kActSilu, kActGelu)
    int f16out;                          // GW: fp16 results
    int atomic;                          // int32 K slices: each adds its sums into C atomically
};

// Workgroup w is dispatched to XCD w % 8. Renumber so the workgroups of one XCD get
// consecutive logical ids, then walk split-K slices, then M fastest (inside a band of row
// tiles, for one-problem launches whose XCDs would otherwise each read all of A): the slices
// of a tile and the M tiles of one B column block then run on one XCD, whose own L2 serves
// them.
__device__ __forceinline__ int xcd_remap(int w, int G, int X)
{
    if (X <= 1) return w;
    const int xcd = w % X, idx = w / X, per = G / X, rem = G % X;
    return xcd * per + (xcd < rem ? xcd : rem) + idx;
}

// ------------------------------------------------------------------------------------
// Operand loaders: global -> registers (load) and registers -> LDS planes (store).
// R rows of the tile, NT threads. A stage covers KPS elements of K, SB bytes of a row.
// voff(i): byte offset of chunk i of this thread inside the tile (fixed for the kernel);
// lane_kb: the byte offset of this thread's chunks inside a stage row (the same for
// every i, since NT is a multiple of the chunks per row).
// ------------------------------------------------------------------------------------
template <Fmt F, int R, int NT> struct Loader;

template <int R, int NT> struct Loader<Fmt::I8, R, NT> {
    static constexpr int PLANES = 1, KPS = 128, SB = 128, NCH = R * 8, CH = (NCH + NT - 1) / NT, BYTES = R * 128;
    static constexpr int VM = CH;   // vector-memory instructions per stage
    __device__ static uint32_t kbytes(int k) { return (uint32_t)k; }
    __device__ static uint32_t lane_kb(int tid) { return (uint32_t)(tid & 7) * 16u; }
    __device__ static uint32_t voff(int i, uint32_t ld, int tid)
    {
        const int q = tid + i * NT;
        return (NCH % NT == 0 || q < NCH) ? (uint32_t)(q >> 3) * ld + (uint32_t)(q & 7) * 16u : kOOB;
    }
    i32x4 r[CH];
    __device__ __forceinline__ void load(Rsrc rs, const uint32_t *vo, uint32_t pz)
    {
#pragma unroll
        for (int i = 0; i < CH; i++) r[i] = ld16(rs, vo[i] | pz);
    }
    __device__ __forceinline__ void store(char *lds, int pstride, int tid) const
    {
        (void)pstride;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT;
            if (NCH % NT == 0 || q < NCH) *reinterpret_cast<i32x4 *>(lds + swz(q >> 3, q & 7)) = r[i];
        }
    }
};

// int4 nibble-packed rows (K/2 bytes). Packed dword d of a row holds k = 8d..8d+7 as
// byte j = (k_{8d+j} << 4) | (k_{8d+4+j} & 0xF). Unpacking keeps each nibble in the HIGH
// half of its byte, so every int8 lane value is exactly 16*k: the int32 accumulators then
// carry a factor 16 that the epilogues remove exactly (shift, or a 1/16 folded into the
// fp32 scale).
__device__ __forceinline__ int nib_hi(int w) { return w & (int)0xF0F0F0F0u; }
__device__ __forceinline__ int nib_lo(int w) { return (int)(((unsigned)w << 4) & 0xF0F0F0F0u); }

template <int R, int NT> struct Loader<Fmt::I4P, R, NT> {
    static constexpr int PLANES = 1, KPS = 128, SB = 64, NCH = R * 4, CH = (NCH + NT - 1) / NT, BYTES = R * 64;
    static constexpr int VM = CH;   // vector-memory instructions per stage
    __device__ static uint32_t kbytes(int k) { return (uint32_t)k >> 1; }
    __device__ static uint32_t lane_kb(int tid) { return (uint32_t)(tid & 3) * 16u; }
    __device__ static uint32_t voff(int i, uint32_t ld, int tid)
    {
        const int q = tid + i * NT;
        return (NCH % NT == 0 || q < NCH) ? (uint32_t)(q >> 2) * ld + (uint32_t)(q & 3) * 16u : kOOB;
    }
    i32x4 r[CH];
    __device__ __forceinline__ void load(Rsrc rs, const uint32_t *vo, uint32_t pz)
    {
#pragma unroll
        for (int i = 0; i < CH; i++) r[i] = ld16(rs, vo[i] | pz);
    }
    __device__ __forceinline__ void store(char *lds, int pstride, int tid) const
    {
        (void)pstride;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT, row = q >> 2, pc = q & 3;
            if (NCH % NT == 0 || q < NCH) {
                const i32x4 w = r[i];
                *reinterpret_cast<i32x4 *>(lds + swz(row, 2 * pc)) =
                    i32x4{nib_hi(w[0]), nib_lo(w[0]), nib_hi(w[1]), nib_lo(w[1])};
                *reinterpret_cast<i32x4 *>(lds + swz(row, 2 * pc + 1)) =
                    i32x4{nib_hi(w[2]), nib_lo(w[2]), nib_hi(w[3]), nib_lo(w[3])};
            }
        }
    }
};

// int16 -> two int8 planes. Balanced split of x clamped to [-32768, 32639]:
// lo = x mod 256 as a signed byte, hi = (x + 128) >> 8 (both in [-128, 127], x = 256 hi + lo).
// On two int16 halves at once: y = min(x, 32639) and z = y + 128 per half (no half overflows:
// z <= 32767), so lo is byte 0 of each half of y and hi byte 1 of each half of z. Four
// int16 values (dwords w0, w1) give four lo bytes and four hi bytes in value order.
typedef short s16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void split4(int w0, int w1, int &lo4, int &hi4)
{
    const s16x2 cap = {32639, 32639}, bias = {128, 128};
    const s16x2 y0 = __builtin_elementwise_min(__builtin_bit_cast(s16x2, w0), cap);
    const s16x2 y1 = __builtin_elementwise_min(__builtin_bit_cast(s16x2, w1), cap);
    const s16x2 z0 = y0 + bias, z1 = y1 + bias;
    // perm(S0, S1, sel): byte i of the result is byte sel_i of {S0:S1} (S1 = bytes 0-3)
    lo4 = (int)__builtin_amdgcn_perm(__builtin_bit_cast(unsigned, y1), __builtin_bit_cast(unsigned, y0), 0x06040200u);
    hi4 = (int)__builtin_amdgcn_perm(__builtin_bit_cast(unsigned, z1), __builtin_bit_cast(unsigned, z0), 0x07050301u);
}

template <int R, int NT> struct Loader<Fmt::I16, R, NT> {
    static constexpr int PLANES = 2, KPS = 128, SB = 256, NCH = R * 8, CH = (NCH + NT - 1) / NT, BYTES = R * 256;
    static constexpr int VM = 2 * CH;   // vector-memory instructions per stage
    __device__ static uint32_t kbytes(int k) { return 2u * (uint32_t)k; }
    __device__ static uint32_t lane_kb(int tid) { return (uint32_t)(tid & 7) * 32u; }
    __device__ static uint32_t voff(int i, uint32_t ld, int tid)
    {
        const int q = tid + i * NT;
        return (NCH % NT == 0 || q < NCH) ? (uint32_t)(q >> 3) * ld + (uint32_t)(q & 7) * 32u : kOOB;
    }
    i32x4 r[CH][2];
    __device__ __forceinline__ void load(Rsrc rs, const uint32_t *vo, uint32_t pz)
    {
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const uint32_t o = vo[i] | pz;
            r[i][0] = ld16(rs, o);
            r[i][1] = ld16(rs, o + 16);
        }
    }
    __device__ __forceinline__ void store(char *lds, int pstride, int tid) const
    {
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT;
            if (NCH % NT == 0 || q < NCH) {
                int l4[4], h4[4];
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    split4(r[i][h][0], r[i][h][1], l4[2 * h], h4[2 * h]);
                    split4(r[i][h][2], r[i][h][3], l4[2 * h + 1], h4[2 * h + 1]);
                }
                const i32x4 vl = {l4[0], l4[1], l4[2], l4[3]}, vh = {h4[0], h4[1], h4[2], h4[3]};
                const int off = swz(q >> 3, q & 7);
                *reinterpret_cast<i32x4 *>(lds + off) = vh;             // plane 0: hi
                *reinterpret_cast<i32x4 *>(lds + pstride + off) = vl;   // plane 1: lo
            }
        }
    }
};

template <int R, int NT> struct Loader<Fmt::F16, R, NT> {
    static constexpr int PLANES = 1, KPS = 64, SB = 128, NCH = R * 8, CH = (NCH + NT - 1) / NT, BYTES = R * 128;
    static constexpr int VM = CH;   // vector-memory instructions per stage
    __device__ static uint32_t kbytes(int k) { return 2u * (uint32_t)k; }
    __device__ static uint32_t lane_kb(int tid) { return (uint32_t)(tid & 7) * 16u; }
    __device__ static uint32_t voff(int i, uint32_t ld, int tid)
    {
        const int q = tid + i * NT;
        return (NCH % NT == 0 || q < NCH) ? (uint32_t)(q >> 3) * ld + (uint32_t)(q & 7) * 16u : kOOB;
    }
    i32x4 r[CH];
    __device__ __forceinline__ void load(Rsrc rs, const uint32_t *vo, uint32_t pz)
    {
#pragma unroll
        for (int i = 0; i < CH; i++) r[i] = ld16(rs, vo[i] | pz);
    }
    // Rows from two sources in 32-row halves (the GLU pairing: tile rows 64 p .. 64 p + 31
    // from rs0, 64 p + 32 .. 64 p + 63 from rs1); chunk i covers tile rows i NT/8 .. + NT/8,
    // so with NT = 256 each chunk lies in one half and one descriptor serves it.
    __device__ __forceinline__ void load_pair(Rsrc rs0, Rsrc rs1, const uint32_t *vo, uint32_t pz)
    {
        static_assert(NT == 256, "one 32-row half per chunk");
#pragma unroll
        for (int i = 0; i < CH; i++) r[i] = ld16((i & 1) ? rs1 : rs0, vo[i] | pz);
    }
    // Source row offset of chunk i in the GLU pairing (tile row r -> row (r / 64) * 32 + r % 32).
    __device__ static uint32_t voff_pair(int i, uint32_t ld, int tid)
    {
        const int q = tid + i * NT, row = q >> 3;
        return (NCH % NT == 0 || q < NCH) ? (uint32_t)((row >> 6) * 32 + (row & 31)) * ld + (uint32_t)(q & 7) * 16u
                                          : kOOB;
    }
    __device__ __forceinline__ void store(char *lds, int pstride, int tid) const
    {
        (void)pstride;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT;
            if (NCH % NT == 0 || q < NCH) *reinterpret_cast<i32x4 *>(lds + swz(q >> 3, q & 7)) = r[i];
        }
    }
};

// erfc(z) = t exp(-z^2 + P(t)) with t = 1 / (1 + |z| / 2) and the degree-9 Chebyshev fit P of
// Press et al., Numerical Recipes in C (2nd ed., section 6.2, "erfcc"): fractional error below
// 1.2e-7 for z >= 0; erfc(-z) = 2 - erfc(z). Branch-free, 27 VALU operations with the hardware
// reciprocal and exp2 (the math library's erfcf took 57).
__device__ __forceinline__ float erfc_fit(float z)
{
    const float a = fabsf(z);
    const float t = __builtin_amdgcn_rcpf(1.0f + 0.5f * a);
    float p = 0.17087277f;
    p = __builtin_fmaf(p, t, -0.82215223f);
    p = __builtin_fmaf(p, t, 1.48851587f);
    p = __builtin_fmaf(p, t, -1.13520398f);
    p = __builtin_fmaf(p, t, 0.27886807f);
    p = __builtin_fmaf(p, t, -0.18628806f);
    p = __builtin_fmaf(p, t, 0.09678418f);
    p = __builtin_fmaf(p, t, 0.37409196f);
    p = __builtin_fmaf(p, t, 1.00002368f);
    p = __builtin_fmaf(p, t, -1.26551223f);
    const float r = t * __builtin_amdgcn_exp2f((p - a * a) * 1.4426950408889634f);
    return z >= 0.f ? r : 2.0f - r;
}

// Gated-FFN, MLP and pre-pass activations in fp32, the reference's forms (GELU with erf; SiLU
// x * sigmoid(x)) to a few fp32 ulp: every result is rounded to fp16 or quantised to int8
// next. The kind is a template argument so that no element carries a branch on it.
// GELU as 0.5 x erfc(-x/sqrt2): equal to 0.5 x (1 + erf(x/sqrt2)), without the cancellation
// of 1 + erf in the negative tail, where fp32 would lose every digit. SiLU with the hardware
// exp and reciprocal: x * rcp(1 + 2^(-x log2 e)) (1 + e^-x rounds to 1 for x >= 17.4, where it
// gives x exactly; for x <= -88 the exp2 is +inf and the result -0).
template <int K> __device__ __forceinline__ float act_k(float x)
{
    if constexpr (K == kActGelu) return 0.5f * x * erfc_fit(x * -0.70710678118654752f);
    else if constexpr (K == kActSilu) return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
    else return x;   // kActIdentity
}

// fp32 -> bf16 by truncation: the high halves of two fp32 words packed into one word.
__device__ __forceinline__ int bf16pack(int f0, int f1)
{
    return (int)(((unsigned)f0 >> 16) | ((unsigned)f1 & 0xFFFF0000u));
}

// fp32 -> tf32 (13 low mantissa bits cleared) -> hi = its bf16 truncation, lo = t - hi.
// lo carries the remaining 3 significant bits, so it is exact in bf16 as well.
__device__ __forceinline__ void tf32split(int f, unsigned &hi16, unsigned &lo16)
{
    const unsigned t = (unsigned)f & 0xFFFFE000u, h = t & 0xFFFF0000u;
    const float lo = __uint_as_float(t) - __uint_as_float(h);
    hi16 = h >> 16;
    lo16 = __float_as_uint(lo) >> 16;
}

// Eight fp32 values (a, then b) -> eight bf16 (truncated).
__device__ __forceinline__ i32x4 bf16x8_of(i32x4 a, i32x4 b)
{
    return i32x4{bf16pack(a[0], a[1]), bf16pack(a[2], a[3]), bf16pack(b[0], b[1]), bf16pack(b[2], b[3])};
}

// Eight fp32 values (a, then b) -> eight tf32 hi bf16 (vh) and eight lo bf16 (vl).
__device__ __forceinline__ void tf32x8_split(i32x4 a, i32x4 b, i32x4 &vh, i32x4 &vl)
{
    unsigned h[8], l[8];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        tf32split(a[e], h[e], l[e]);
        tf32split(b[e], h[4 + e], l[4 + e]);
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
        vh[e] = (int)(h[2 * e] | (h[2 * e + 1] << 16));
        vl[e] = (int)(l[2 * e] | (l[2 * e + 1] << 16));
    }
}

// fp32 rows (truncated to bf16, or split into tf32 hi/lo bf16 planes, on the way to LDS).
template <int R, int NT, bool TF32> struct LoaderF32 {
    static constexpr int PLANES = TF32 ? 2 : 1, KPS = 64, SB = 256, NCH = R * 8, CH = (NCH + NT - 1) / NT,
                         BYTES = R * 256;
    static constexpr int VM = 2 * CH;
    __device__ static uint32_t kbytes(int k) { return 4u * (uint32_t)k; }
    __device__ static uint32_t lane_kb(int tid) { return (uint32_t)(tid & 7) * 32u; }
    __device__ static uint32_t voff(int i, uint32_t ld, int tid)
    {
        const int q = tid + i * NT;
        return (NCH % NT == 0 || q < NCH) ? (uint32_t)(q >> 3) * ld + (uint32_t)(q & 7) * 32u : kOOB;
    }
    i32x4 r[CH][2];
    __device__ __forceinline__ void load(Rsrc rs, const uint32_t *vo, uint32_t pz)
    {
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const uint32_t o = vo[i] | pz;
            r[i][0] = ld16(rs, o);
            r[i][1] = ld16(rs, o + 16);
        }
    }
    __device__ __forceinline__ void store(char *lds, int pstride, int tid) const
    {
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT;
            if (!(NCH % NT == 0 || q < NCH)) continue;
            const int off = swz(q >> 3, q & 7);
            if constexpr (!TF32) {
                (void)pstride;
                *reinterpret_cast<i32x4 *>(lds + off) = bf16x8_of(r[i][0], r[i][1]);
            } else {
                i32x4 vh, vl;
                tf32x8_split(r[i][0], r[i][1], vh, vl);
                *reinterpret_cast<i32x4 *>(lds + off) = vh;
                *reinterpret_cast<i32x4 *>(lds + pstride + off) = vl;
            }
        }
    }
};
template <int R, int NT> struct Loader<Fmt::F32BF16, R, NT> : LoaderF32<R, NT, false> {};
template <int R, int NT> struct Loader<Fmt::F32TF32, R, NT> : LoaderF32<R, NT, true> {};

// bf16 rows: moved like fp16 (the MFMA reads the same 16-bit lanes as bf16).
template <int R, int NT> struct Loader<Fmt::BF16, R, NT> : Loader<Fmt::F16, R, NT> {};

// tf32 hi/lo rows from convert_f32 (per 8 elements, 16 bytes of hi then 16 of lo): the two
// halves of a 32-byte chunk go to the hi and lo planes unchanged.
template <int R, int NT> struct Loader<Fmt::BF16X2, R, NT> : LoaderF32<R, NT, true> {
    using Base = LoaderF32<R, NT, true>;
    __device__ __forceinline__ void store(char *lds, int pstride, int tid) const
    {
#pragma unroll
        for (int i = 0; i < Base::CH; i++) {
            const int q = tid + i * NT;
            if (!(Base::NCH % NT == 0 || q < Base::NCH)) continue;
            const int off = swz(q >> 3, q & 7);
            *reinterpret_cast<i32x4 *>(lds + off) = this->r[i][0];
            *reinterpret_cast<i32x4 *>(lds + pstride + off) = this->r[i][1];
        }
    }
};

// int8 rows straight from HBM into LDS (gfx950 buffer_load_dwordx4 ... lds): no staging
// registers and no LDS store instructions. One wave instruction moves 1 KB = 8 tile rows and
// lane l's 16 bytes land at byte 16 l of the block, so each lane fetches the chunk the LDS
// swizzle puts there. R rows, NW waves: each wave owns R / NW consecutive rows.
template <int R, int NW> struct DmaA {
    static constexpr int RW = R / NW, INS = RW / 8;
    static_assert(RW % 8 == 0, "whole 8-row blocks per wave");
    uint32_t vo[INS], cb[INS];
    __device__ __forceinline__ void init(uint32_t ld, int wave, int lane)
    {
#pragma unroll
        for (int i = 0; i < INS; i++) {
            const int row = wave * RW + i * 8 + (lane >> 3), c = (lane & 7) ^ ((row >> 1) & 7);
            vo[i] = (uint32_t)row * ld + (uint32_t)c * 16u;
            cb[i] = (uint32_t)c * 16u;
        }
    }
    // The GLU pairing (tile rows 64 p .. 64 p + 31 from the gate source, 64 p + 32 .. 64 p + 63
    // from the up source, both from source row 32 p on): a wave's rows lie in one 32-row
    // half, so one wave-uniform descriptor serves all of them (pair_half picks it).
    __device__ __forceinline__ void init_pair(uint32_t ld, int wave, int lane)
    {
        static_assert(RW <= 32 && 32 % RW == 0, "a wave's rows in one 32-row half");
#pragma unroll
        for (int i = 0; i < INS; i++) {
            const int row = wave * RW + i * 8 + (lane >> 3), c = (lane & 7) ^ ((row >> 1) & 7);
            vo[i] = (uint32_t)((row >> 6) * 32 + (row & 31)) * ld + (uint32_t)c * 16u;
            cb[i] = (uint32_t)c * 16u;
        }
    }
    __device__ static bool pair_half(int wave) { return ((wave * RW) >> 5) & 1; }
    // plane: the A slot; wave must be wave-uniform (it forms the LDS address in M0).
    // MASK: chunks at or past kenda read as zero; without it they read whatever lies there
    // inside the descriptor's range (for integer operands whose partner is masked: any
    // finite value times a zero partner adds nothing).
    // (The LDS-pointer builtin exists in the device pass only; the host pass, which also
    // instantiates kernel templates to emit their launch stubs, must not see it.)
    template <bool MASK = true>
    __device__ __forceinline__ void issue(Rsrc rs, char *plane, uint32_t ka, uint32_t kenda, int wave) const
    {
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
        for (int i = 0; i < INS; i++) {
            const uint32_t pz = (!MASK || ka + cb[i] < kenda) ? 0u : kOOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rs, (__attribute__((address_space(3))) void *)(plane + (wave * RW + i * 8) * ROWB), 16, vo[i] | pz, 0,
                0, 0);
        }
#endif
    }
};

// s_waitcnt for at most n outstanding vector-memory operations (lgkm and exp untouched).
template <int N> __device__ __forceinline__ void wait_vm()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
#endif
}

// ------------------------------------------------------------------------------------
// MFMA math. BS x BS result blocks (32 x 32, or 16 x 16 for the MathF16x16 / MathBF16x16
// fp16 and bf16 shapes); a substep consumes KSB LDS bytes per row; KEL = K elements per
// substep. A fragments are the first MFMA operand (see the file header). Lane l supplies
// fragment row l % BS and the 16-byte chunk l / BS of the substep's KSB bytes; in a result
// block it holds column l % BS and NE elements, element e at row 4 (l / BS) + row_of(e).
// ------------------------------------------------------------------------------------
template <class MATH> __device__ __forceinline__ i32x4 lds_frag(const char *plane, int row, int sub, int lane)
{
    return *reinterpret_cast<const i32x4 *>(plane + swz(row, (MATH::KSB / 16) * sub + lane / MATH::BS));
}

// 32 x 32 result blocks: 16 elements a lane, element e = 4 q + r at row 8 q + r (+ 4 (l / 32)).
struct Block32 {
    static constexpr int BS = 32, NE = 16;
    using AccF = f32x16;   // fp32 sums of one block (group-wise epilogues)
    __device__ static constexpr int row_of(int e) { return 8 * (e >> 2) + (e & 3); }
};
// 16 x 16 result blocks: 4 elements a lane, element e at row e (+ 4 (l / 16)).
struct Block16 {
    static constexpr int BS = 16, NE = 4;
    using AccF = f32x4;
    __device__ static constexpr int row_of(int e) { return e; }
};

struct MathI8 : Block32 {  // v_mfma_i32_32x32x32_i8
    using Acc = i32x16;
    static constexpr int NACC = 1, PA = 1, PB = 1, KSB = 32, KEL = 32;
    __device__ static void mma(Acc *acc, const i32x4 *a, const i32x4 *b)
    {
        acc[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[0], b[0], acc[0], 0, 0, 0);
    }
    // first product of a quant group: the accumulator input is the constant 0
    __device__ static void mma0(Acc *acc, const i32x4 *a, const i32x4 *b)
    {
        acc[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[0], b[0], i32x16{}, 0, 0, 0);
    }
};

struct MathI16 : Block32 { // byte planes (0 = hi, 1 = lo): acc0 = hh, acc1 = hl + lh, acc2 = ll
    using Acc = i32x16;
    static constexpr int NACC = 3, PA = 2, PB = 2, KSB = 32, KEL = 32;
    __device__ static void mma(Acc *acc, const i32x4 *a, const i32x4 *b)
    {
        acc[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[0], b[0], acc[0], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[0], b[1], acc[1], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[1], b[0], acc[1], 0, 0, 0);
        acc[2] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[1], b[1], acc[2], 0, 0, 0);
    }
    __device__ static void mma0(Acc *acc, const i32x4 *a, const i32x4 *b)
    {
#pragma unroll
        for (int n = 0; n < NACC; n++) acc[n] = Acc{};
        mma(acc, a, b);
    }
};

struct MathF16 : Block32 { // v_mfma_f32_32x32x16_f16
    using Acc = f32x16;
    static constexpr int NACC = 1, PA = 1, PB = 1, KSB = 32, KEL = 16;
    __device__ static void mma(Acc *acc, const i32x4 *a, const i32x4 *b)
    {
        acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a[0]),
                                                        __builtin_bit_cast(f16x8, b[0]), acc[0], 0, 0, 0);
    }
    __device__ static void mma0(Acc *acc, const i32x4 *a, const i32x4 *b)
    {
#pragma unroll
        for (int n = 0; n < NACC; n++) acc[n] = Acc{};
        mma(acc, a, b);
    }
};

struct MathBF16 : Block32 {   // v_mfma_f32_32x32x16_bf16
    using Acc = f32x16;
    static constexpr int NACC = 1, PA = 1, PB = 1, KSB = 32, KEL = 16;
    __device__ static void mma(Acc *acc, const i32x4 *a, const i32x4 *b)
    {
        acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a[0]),
                                                         __builtin_bit_cast(bf16x8, b[0]), acc[0], 0, 0, 0);
    }
    __device__ static void mma0(Acc *acc, const i32x4 *a, const i32x4 *b)
    {
#pragma unroll
        for (int n = 0; n < NACC; n++) acc[n] = Acc{};
        mma(acc, a, b);
    }
};

struct MathTF32 : Block32 {   // bf16 hi/lo planes: hi*hi + lo*hi + hi*lo (lo*lo dropped)
    using Acc = f32x16;
    static constexpr int NACC = 1, PA = 2, PB = 2, KSB = 32, KEL = 16;
    __device__ static void mma(Acc *acc, const i32x4 *a, const i32x4 *b)
    {
        const bf16x8 ah = __builtin_bit_cast(bf16x8, a[0]), al = __builtin_bit_cast(bf16x8, a[1]);
        const bf16x8 bh = __builtin_bit_cast(bf16x8, b[0]), bl = __builtin_bit_cast(bf16x8, b[1]);
        acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh, acc[0], 0, 0, 0);
        acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh, acc[0], 0, 0, 0);
        acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl, acc[0], 0, 0, 0);
    }
    __device__ static void mma0(Acc *acc, const i32x4 *a, const i32x4 *b)
    {
#pragma unroll
        for (int n = 0; n < NACC; n++) acc[n] = Acc{};
        mma(acc, a, b);
    }
};

struct MathF16x16 : Block16 {    // v_mfma_f32_16x16x32_f16: 8 halves of K a lane, 64 LDS bytes a substep
    using Acc = f32x4;
    static constexpr int NACC = 1, PA = 1, PB = 1, KSB = 64, KEL = 32;
    __device__ static void mma(Acc *acc, const i32x4 *a, const i32x4 *b)
    {
        acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a[0]),
                                                        __builtin_bit_cast(f16x8, b[0]), acc[0], 0, 0, 0);
    }
    __device__ static void mma0(Acc *acc, const i32x4 *a, const i32x4 *b)
    {
        acc[0] = Acc{};
        mma(acc, a, b);
    }
};

struct MathBF16x16 : Block16 {   // v_mfma_f32_16x16x32_bf16
    using Acc = f32x4;
    static constexpr int NACC = 1, PA = 1, PB = 1, KSB = 64, KEL = 32;
    __device__ static void mma(Acc *acc, const i32x4 *a, const i32x4 *b)
    {
        acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[0]),
                                                         __builtin_bit_cast(bf16x8, b[0]), acc[0], 0, 0, 0);
    }
    __device__ static void mma0(Acc *acc, const i32x4 *a, const i32x4 *b)
    {
        acc[0] = Acc{};
        mma(acc, a, b);
    }
};

// ------------------------------------------------------------------------------------
// Group-wise scales. Every stage carries NGS slots of scales, gathered from the
// caller's [rows][nG] arrays into registers with the operand prefetch and written to LDS
// with the stage. NGS == 1 when every group is a whole number of stages: a stage then
// closes at most one group, the one its first element lies in. NGS == 4 otherwise: slot ss
// holds the group of the last element of substep ss.
// LDS layout of a stage's scales: B [NGS][BN], then (per-group activation scales) A [NGS][BM].
// ------------------------------------------------------------------------------------
// MODE 0: 4-byte gathers; 4: a 16-byte load per row and stage (NGS == 4), for the tiles with
// per-group activation scales (with per-row ones the gathers measured faster: MoE forward
// 244-247 against 250-253 us). One-group stages keep the gathers: windows of four groups
// loaded every fourth stage into LDS measured slower (config 3 through the reference entry
// 58.5-58.9 against 55.7-56.3 us; 56.8 with the window loads taken out, 53.5 with the gathers
// taken out: the window bookkeeping cost more than the gathers).
template <int NGS, bool ROWSCALE> constexpr int scale_mode() { return (!ROWSCALE && NGS == 4) ? 4 : 0; }
template <int BM, int BN, int NGS, bool ROWSCALE, bool B_I4, int NT, int MODE = scale_mode<NGS, ROWSCALE>()>
struct ScaleLoader;

// Whether tile row r has a group scale that differs from its first, from the per-thread
// verdicts rowmis[sub * BM + r] of the NT / BM threads that checked it.
template <int BM, int NT> __device__ __forceinline__ bool row_mis(const int *rowmis, int r)
{
    int m = 0;
#pragma unroll
    for (int sub = 0; sub < NT / BM; sub++) m |= rowmis[sub * BM + r];
    return m != 0;
}

// Rows of the 16-byte form: thread q (q = tid + i NT) takes row q of the tile's BN B rows
// followed by its BM A rows; BN is a multiple of 64, so every wave reads from one of the two
// arrays and picks its descriptor once. A window of four groups starts at g0 and is moved
// back to end inside the row when nG >= 4 (no load reaches past its row, nor past the
// array); with nG < 4 (g0 = 0) a row's window runs into the next row, and the array's last
// row starts its window 4 - nG groups early (last).
template <int BM, int BN, int NT> struct ScaleRows {
    static constexpr int R = BN + BM, NB = (R + NT - 1) / NT;
    uint32_t off[NB];   // byte offset of the row in its array (kOOB: no row)
    int last[NB];       // 4 - nG for the array's last row when nG < 4, else 0
    uint32_t aunit = 0; // bit i: A row of load i folds in the row-scale order (staged as 1.0)
    // rowmis[sub * BM + r]: some scale of tile row r differs from its first (one entry per
    // checking thread of the row); a row folds in the row-scale order when none does
    __device__ void set_unit(const int *rowmis, bool check, int tid)
    {
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const int q = tid + i * NT;
            if (q >= BN && q < R && check && !row_mis<BM, NT>(rowmis, q - BN)) aunit |= 1u << i;
        }
    }
    __device__ void init(int nG, int n0, int N, int m0, int M, int tid)
    {
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const int q = tid + i * NT;
            const bool isb = q < BN;
            const int row = isb ? n0 + q : m0 + (q - BN), rows = isb ? N : M;
            const bool ok = q < R && row < rows;
            off[i] = ok ? (uint32_t)row * (uint32_t)nG * 4u : kOOB;
            last[i] = (ok && nG < 4 && row == rows - 1) ? 4 - nG : 0;
        }
    }
    __device__ static int window_start(int g, int nG) { return nG >= 4 ? min(g, nG - 4) : 0; }
    // element e (group g0 + e) of a window row; e + last > 3 only for groups past nG (unused)
    __device__ static float pick(const i32x4 &r, int e, int last)
    {
        const int x = e + last;
        return __int_as_float(x == 0 ? r[0] : (x == 1 ? r[1] : (x == 2 ? r[2] : r[3])));
    }
};

// One 4-byte gather per (slot, row) and stage.
template <int BM, int BN, int NGS, bool ROWSCALE, bool B_I4, int NT> struct ScaleLoader<BM, BN, NGS, ROWSCALE, B_I4, NT, 0> {
    static constexpr int NB = (NGS * BN + NT - 1) / NT;
    static constexpr int NA = ROWSCALE ? 0 : (NGS * BM + NT - 1) / NT;
    // per thread, fixed for the kernel: the row offsets (bytes) of the scales it gathers
    struct Cols {
        uint32_t b[NB], a[NA > 0 ? NA : 1];
        uint32_t aunit = 0;   // bit i: A row of gather i folds in the row-scale order (staged as 1.0)
        __device__ void set_unit(const int *rowmis, bool check, int tid)
        {
#pragma unroll
            for (int i = 0; i < NA; i++) {
                const int q = tid + i * NT;
                if (q < NGS * BM && check && !row_mis<BM, NT>(rowmis, q % BM)) aunit |= 1u << i;
            }
        }
        __device__ void init(int nG, int n0, int N, int m0, int M, int tid)
        {
#pragma unroll
            for (int i = 0; i < NB; i++) {
                const int q = tid + i * NT, n = n0 + q % BN;
                b[i] = (q < NGS * BN && n < N) ? (uint32_t)n * (uint32_t)nG * 4u : kOOB;
            }
#pragma unroll
            for (int i = 0; i < NA; i++) {
                const int q = tid + i * NT, m = m0 + q % BM;
                a[i] = (q < NGS * BM && m < M) ? (uint32_t)m * (uint32_t)nG * 4u : kOOB;
            }
        }
    };
    float rb[NB], ra[NA > 0 ? NA : 1];
    __device__ __forceinline__ void load(Rsrc sb, Rsrc sa, const Cols &c, int k, uint64_t gmag, int nG, bool noa, int tid)
    {
        (void)nG;
        int gs[NGS];
#pragma unroll
        for (int s = 0; s < NGS; s++) gs[s] = div32m(NGS == 1 ? k : k + 32 * s + 31, gmag);
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const int slot = (tid + i * NT) / BN;
            int g = gs[0];
#pragma unroll
            for (int s = 1; s < NGS; s++) g = slot == s ? gs[s] : g;
            rb[i] = ld4f(sb, c.b[i] + (uint32_t)g * 4u);   // kOOB + a small offset stays out of range
        }
#pragma unroll
        for (int i = 0; i < NA; i++) {
            const int slot = (tid + i * NT) / BM;
            int g = gs[0];
#pragma unroll
            for (int s = 1; s < NGS; s++) g = slot == s ? gs[s] : g;
            ra[i] = ld4f(sa, noa ? kOOB : c.a[i] + (uint32_t)g * 4u);
        }
    }
    __device__ __forceinline__ void store(float *sc, int tid, const Cols &c) const
    {
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const int q = tid + i * NT;
            // 1/16 is exact: it removes the x16 that unpacked int4 weights carry
            if (q < NGS * BN) sc[q] = B_I4 ? rb[i] * 0.0625f : rb[i];
        }
#pragma unroll
        for (int i = 0; i < NA; i++) {
            const int q = tid + i * NT;
            if (q < NGS * BM) sc[NGS * BN + q] = ((c.aunit >> i) & 1u) ? 1.0f : ra[i];
        }
    }
};

// NGS == 4 (groups that are not whole stages) with per-group activation scales: the four
// slots' groups are consecutive groups of one row, so each row is one 16-byte load of four
// groups (one L2 request per row and stage, against four 4-byte gathers from four waves; the
// reference's MoE entry at config 5: 576 -> 554 us a forward).
template <int BM, int BN, int NGS, bool ROWSCALE, bool B_I4, int NT> struct ScaleLoader<BM, BN, NGS, ROWSCALE, B_I4, NT, 4> {
    static_assert(NGS == 4 && !ROWSCALE && BN % 64 == 0, "one array per wave");
    using Cols = ScaleRows<BM, BN, NT>;
    static constexpr int R = Cols::R, NB = Cols::NB, NA = 0;   // 16-byte loads per thread and stage
    i32x4 r[NB];
    int d[NGS];   // element of the loaded window that each slot takes
    __device__ __forceinline__ void load(Rsrc sb, Rsrc sa, const Cols &c, int k, uint64_t gmag, int nG, bool noa, int tid)
    {
        int gs[NGS];
#pragma unroll
        for (int s = 0; s < NGS; s++) gs[s] = div32m(k + 32 * s + 31, gmag);
        const int g0 = Cols::window_start(gs[0], nG);
#pragma unroll
        for (int s = 0; s < NGS; s++) d[s] = gs[s] - g0;
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const int q0 = __builtin_amdgcn_readfirstlane(tid + i * NT);   // the wave's first row
            const Rsrc rs = q0 < BN ? sb : sa;
            const uint32_t off = (noa && q0 >= BN) ? kOOB : c.off[i] + (uint32_t)(g0 - c.last[i]) * 4u;
            r[i] = ld16(rs, off);   // kOOB + a small offset stays out of range
        }
    }
    __device__ __forceinline__ void store(float *sc, int tid, const Cols &c) const
    {
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const int q = tid + i * NT;
            if (q < R) {
#pragma unroll
                for (int s = 0; s < NGS; s++) {
                    const float x = Cols::pick(r[i], d[s], c.last[i]);
                    // 1/16 is exact: it removes the x16 that unpacked int4 weights carry
                    if (q < BN) sc[s * BN + q] = B_I4 ? x * 0.0625f : x;
                    else sc[NGS * BN + s * BM + (q - BN)] = ((c.aunit >> i) & 1u) ? 1.0f : x;
                }
            }
        }
    }
};

// f(0), f(1), ..., f(N-1) with compile-time indices.
template <int N, class F> __device__ __forceinline__ void static_for(F &&f)
{
    if constexpr (N > 0) {
        static_for<N - 1>(f);
        f(std::integral_constant<int, N - 1>{});
    }
}

// Workgroup barrier that orders LDS only. __syncthreads() is a workgroup release fence,
// which on gfx9 also waits for every outstanding global load (vmcnt(0)) and so would
// drain the prefetch pipeline at each stage.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// ------------------------------------------------------------------------------------
// Tile configuration. BM x BN tile of 32x32 MFMA blocks; WGM x WGN waves, each owning a
// (BM/WGM) x (BN/WGN) sub-tile. Dynamic LDS: 2 stages x (operand planes [+ scale slots])
// [+ the tile's per-row activation scales].
//
// GM, the group-wise cadence: 1, 2, 4 = quant groups of 32, 64, 128 elements (a group
// closes after every GM-th substep, known at compile time: the first MFMA of a group takes
// a zero accumulator input); 8 = groups of whole stages found at run time; 0 = any other
// group found at run time. NGS scale slots per stage: one when groups are whole stages.
// ------------------------------------------------------------------------------------
template <int BM, int BN, Fmt FA, Fmt FB, class MATH, Epi EPI, bool ROWSCALE, int GM>
struct KCfg {
    using MT = MATH;
    static constexpr bool GW = (EPI == Epi::GW);
    // substeps per quant group when groups are compile-time (GM = group / 32)
    static constexpr int GMS = (GM >= 1 && GM <= 4) ? (GM * 32 / MATH::KEL > 0 ? GM * 32 / MATH::KEL : 1) : GM;
    // 256 x 128 tiles with an int8 A operand and a group-wise (per-row or per-group activation
    // scales) or a plain int32 epilogue: 8 waves (4 x 2) of 64 x 64, two per SIMD, one
    // workgroup per CU (W8). Others: 4 waves (2 x 2).
    // Group-wise 256 x 128 tiles with int8 B and per-row activation scales whose groups close
    // every substep or two (fold-bound: the fold's two VALU operations per element and group
    // outweigh the MFMAs): 16 waves (4 x 4) of 64 x 32, four per SIMD at most 128 registers
    // each (W16). The extra waves keep the matrix pipe and the VALU fed while others wait on
    // LDS or the barrier: the MoE forward (config 5) takes 241 us against 270 us with 8 waves
    // of 64 x 64. (Per-group activation scales would spill at 128 registers. The group-128
    // int4 kernel fits, in 125, but measured slower: config 3 52.9-54.3 against 48.5 us.)
    static constexpr bool W16 = BM == 256 && BN == 128 && GW && ROWSCALE && FA == Fmt::I8 && FB == Fmt::I8 &&
                                (GM == 1 || GM == 2);
    static constexpr bool W8 = !W16 && BM == 256 && ((FA == Fmt::I8 && (GW || EPI == Epi::I32)) ||
                                             ((FA == Fmt::BF16 || FA == Fmt::F16) && FB == FA &&
                                              (EPI == Epi::F16 || EPI == Epi::F32 || EPI == Epi::GLU ||
                                               EPI == Epi::ACT)));
    // 128 x 64 tiles of int8 -> int32, of group-wise products with int8 B and of fp16 / bf16
    // products (the shapes whose 256 x 128 tiles leave most CUs idle): 8 waves (4 x 2) of
    // 32 x 32, both operands by LDS DMA like the 256 x 128 8-wave tiles (W4D; 4 waves of
    // 64 x 32 measured slower: int8 512 x 4096 x 4096 19.2 against 18.0 us, fp16 same shape
    // 33.9 against 30.2 us; the per-expert calls of the reference's MoE entry, ~1024 x 2048 x
    // 1408 group 32: 790 against 577 us a forward).
    static constexpr bool W4D = BM == 128 && BN == 64 && FB == FA &&
                                ((FA == Fmt::I8 && (EPI == Epi::I32 || EPI == Epi::GW)) ||
                                 ((FA == Fmt::F16 || FA == Fmt::BF16) &&
                                  (EPI == Epi::F16 || EPI == Epi::F32 || EPI == Epi::ACT)));
    // 256 x 256 fp16 / bf16 tiles (W8W, the 8-wave layout with 64 x 128 wave tiles): a third
    // fewer operand bytes per MFMA than 256 x 128. Both operands by DMA into two 32 KB slots
    // each (128 KB of LDS), one stage in flight. (B staged in registers beside three A slots,
    // two stages in flight in 160 KB, measured 3% faster and spills 7 VGPRs.)
    static constexpr bool W8W = W8 && BN == 256;
    static constexpr bool DMA = W8 || W4D || W16;
    // Two-plane products whose 4-wave tiles run one wave per SIMD (their LDS ring admits one
    // workgroup per CU): 8 waves (4 x 2) with register-staged loads, two per SIMD. int16-exact
    // 128 x 64 tiles (config 2b: 65.5 against 76.1 us) and tf32 128 x 128 tiles on hi/lo bf16
    // pairs converted ahead (config 4 tf32: 848 against 956 us; A converted inside the loads
    // would spill).
    static constexpr bool I16W = (BM == 128 && BN == 64 && FA == Fmt::I16 && FB == Fmt::I16) ||
                                 (BM == 128 && BN == 128 && FA == Fmt::BF16X2);
    static constexpr int WGM = (DMA || I16W) ? 4 : 2, WGN = W16 ? 4 : 2, NT = 64 * WGM * WGN;
    static constexpr int WTM = BM / WGM, WTN = BN / WGN, TM = WTM / MATH::BS, TN = WTN / MATH::BS;
    static constexpr int PLA = BM * ROWB, PLB = BN * ROWB;
    // (a stage holds KPS / 32 chunks of 32 K values, each within one group)
    static constexpr int NGS = (GM == 4 || GM == 8) ? 1 : Loader<FA, BM, NT>::KPS / 32;
    static constexpr int SCB = GW ? NGS * (BN + (ROWSCALE ? 0 : BM)) * 4 : 0;
    static constexpr int STAGE = MATH::PA * PLA + MATH::PB * PLB + SCB;
    // the tile's row scales (and, per-group activation scales, one flag word per wave)
    // (per-group activation scales: + one verdict per checking thread and one flag per wave)
    static constexpr int RSB = GW ? BM * 4 + (ROWSCALE ? 0 : NT * 4 + 64) : 0;
    static constexpr int LDS_RING = 2 * STAGE + RSB;
    static constexpr int REGS = (Loader<FA, BM, NT>::BYTES + Loader<FB, BN, NT>::BYTES) / (4 * NT);
    // Group-wise tiles with per-row activation scales and the DMA tiles run two waves per
    // SIMD (at most 256 registers a wave), so that one wave's LDS waits and scale epilogue
    // overlap the other's MFMAs: two stages in flight. Per-group activation scales need more
    // registers: one wave per SIMD.
    // Other tiles run one wave per SIMD with as many stages in flight as ~128 VGPRs of
    // staging registers hold.
    static constexpr int WPE = W16 ? 4 : ((DMA || I16W || (GW && ROWSCALE)) ? 2 : 1);
    // (Six W4D slots, five stages in flight, measured the same as three: 19.3 us at
    // 512 x 4096 x 4096.)
    static constexpr int D = W8W ? 1 : ((GW || DMA) ? 2 : (REGS <= 32 ? 4 : (REGS <= 48 ? 3 : (REGS <= 64 ? 2 : 1))));
    // DMA tiles load the A operand straight into a ring of D + 1 LDS slots. With B by DMA too
    // they hold a whole stage of fragments in registers one stage ahead; the group-wise
    // tiles (int4 B) keep two fragment sets (the next substep's reads overlap this
    // substep's MFMAs).
    static constexpr bool ADMA = DMA;
    static constexpr int ASL = ADMA ? D + 1 : 0;
    // B operands that need no unpacking (int8, bf16, fp16) take the same DMA path into D + 1
    // slots; int4 B is unpacked in registers and stored (two slots).
    static constexpr bool BDMA = DMA && FB != Fmt::I4P;
    static constexpr int BSL = BDMA ? D + 1 : 2;
    static constexpr int BSTAGE = MATH::PB * PLB;
    // group scales are stored from registers, so two slots suffice beside a deeper B ring
    static constexpr int LDS_ADMA = ASL * PLA + BSL * BSTAGE + 2 * SCB + RSB;
};

// Group-wise fold of one 32x32 block's int32 partials into its fp32 accumulators:
// fmaf(a*b, P, acc), or fmaf(b, P, acc) with per-row activation scales applied at the end
// (ROWSCALE; also the order of tiles whose per-group activation scales are constant along
// each row).
// sbj: the block's B scale for this lane's column; sc / slot: the stage's staged scales
// (per-group activation scales of the block's rows follow the B scales).
template <class CF, bool ROWSCALE, class PG, class AF>
__device__ __forceinline__ void gw_fold_block(const PG &pg, AF &af, float sbj, const float *sc, int slot, int i,
                                              int wm, int lane)
{
    constexpr int BM = CF::WTM * CF::WGM, BN = CF::WTN * CF::WGN, NGS = CF::NGS;
    using MT = typename CF::MT;
    constexpr int BS = MT::BS, NE = MT::NE;
    if constexpr (ROWSCALE) {
#pragma unroll
        for (int e = 0; e < NE; e++) af[e] = __builtin_fmaf(sbj, (float)pg[e], af[e]);
    } else {
        // elements 4 q .. 4 q + 3 lie on four consecutive rows: one 16-byte read of their scales
#pragma unroll
        for (int q = 0; q < NE / 4; q++) {
            const f32x4 sa = *reinterpret_cast<const f32x4 *>(sc + NGS * BN + slot * BM + wm * CF::WTM + BS * i +
                                                              MT::row_of(4 * q) + 4 * (lane / BS));
#pragma unroll
            for (int r = 0; r < 4; r++) af[4 * q + r] = __builtin_fmaf(sa[r] * sbj, (float)pg[4 * q + r], af[4 * q + r]);
        }
    }
}

// This lane's B scale of column block j for the staged group `slot`.
template <class CF>
__device__ __forceinline__ float gw_bscale(const float *sc, int slot, int wn, int j, int lane)
{
    constexpr int BN = CF::WTN * CF::WGN;
    return sc[slot * BN + wn * CF::WTN + CF::MT::BS * j + lane % CF::MT::BS];
}

// A problem's dump window, read from the kernel arguments once before the main loop (the
// LDS barriers' memory clobbers would otherwise reload it at every group).
struct DumpWin {
    int32_t *ptr;
    int row0, rows;
};

// Copies the partials of the group that ends at K position kpos out to the problem's dump
// buffer, when the launch carries one (a wave-uniform branch: the dump comes from the same
// instantiation as every other call).
template <class CF, bool B_I4, class AccArr>
__device__ __forceinline__ void gw_dump(const KArgs &args, const DumpWin &P, const AccArr &acc, int kpos, int mrow,
                                        int ncol, int N)
{
    constexpr int TM = CF::TM, TN = CF::TN, BS = CF::MT::BS;
    if (P.ptr) {
        // [row][group][n] window of rows [dump_row0, + dump_rows): this lane's byte offset for
        // column block j at row mrow, then a scalar offset per row. Rows above the window wrap
        // to offsets at or past 2^31 and rows below it (including rows past M) lie past its
        // end, so the buffer range check drops their stores; columns past N start past the
        // range (the host keeps (M + 256) * nG * N * 4 below 2^31).
        const int g = div32m(kpos - 1, args.gmag);
        const uint32_t rstride = (uint32_t)args.nG * (uint32_t)N * 4u;
        const Rsrc rd = rsrc(P.ptr, (uint32_t)P.rows * rstride);
        uint32_t dmo[TN];
#pragma unroll
        for (int j = 0; j < TN; j++)
            dmo[j] = ncol + BS * j < N ? (uint32_t)(mrow - P.row0) * rstride + (uint32_t)(g * N + ncol + BS * j) * 4u
                                       : kOOB;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int e = 0; e < CF::MT::NE; e++) {
                const uint32_t so = (uint32_t)(BS * i + CF::MT::row_of(e)) * rstride;
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    int v = acc[i][j][0][e];
                    if (B_I4) v >>= 4;
                    __builtin_amdgcn_raw_buffer_store_b32(v, rd, dmo[j] + so, 0, 0);
                }
            }
    }
}

// Group-wise epilogue at the end of an int32 partial period: fold every block (sb: this
// lane's B scale of each column block), dump, and clear the partials when the next group's
// first MFMA does not start from zero itself.
template <class CF, bool ROWSCALE, bool B_I4, bool ZERO, bool DUMP, class AccT>
__device__ __forceinline__ void gw_group(const KArgs &args, const DumpWin &dw, AccT (&acc)[CF::TM][CF::TN][1],
                                         typename CF::MT::AccF (&accf)[CF::TM][CF::TN], const float (&sb)[CF::TN], const float *sc,
                                         int slot, int kpos, int wm, int lane, int mrow, int ncol, int N)
{
    constexpr int TM = CF::TM, TN = CF::TN;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) gw_fold_block<CF, ROWSCALE>(acc[i][j][0], accf[i][j], sb[j], sc, slot, i, wm, lane);
    if constexpr (DUMP) gw_dump<CF, B_I4>(args, dw, acc, kpos, mrow, ncol, N);
    if constexpr (ZERO) {   // otherwise the next group's first MFMA starts from a zero input
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) acc[i][j][0] = AccT{};
    }
}

// ------------------------------------------------------------------------------------
// The kernel.
// ------------------------------------------------------------------------------------
template <int BM, int BN, Fmt FA, Fmt FB, class MATH, Epi EPI, bool ROWSCALE, int GM>
__global__ __launch_bounds__((KCfg<BM, BN, FA, FB, MATH, EPI, ROWSCALE, GM>::NT))
__attribute__((amdgpu_waves_per_eu(KCfg<BM, BN, FA, FB, MATH, EPI, ROWSCALE, GM>::WPE)))
void k_gemm(const KArgs args)
{
    using CF = KCfg<BM, BN, FA, FB, MATH, EPI, ROWSCALE, GM>;
    constexpr int NGS = CF::NGS;
    constexpr int NT = CF::NT, WGN = CF::WGN, WTM = CF::WTM, WTN = CF::WTN, TM = CF::TM, TN = CF::TN;
    constexpr int PLA = CF::PLA, PLB = CF::PLB, STAGE = CF::STAGE;
    constexpr bool GW = CF::GW;
    using LA = Loader<FA, BM, NT>;
    using LB = Loader<FB, BN, NT>;
    using SL = ScaleLoader<BM, BN, NGS, ROWSCALE, FB == Fmt::I4P, NT>;
    static_assert(!GW || GM == 0 || GM == 1 || GM == 2 || GM == 4 || GM == 8, "group cadence");
    static_assert(LA::KPS == LB::KPS, "operand stage K mismatch");
    static_assert(LA::KPS == MATH::KEL * (ROWB / MATH::KSB), "stage K vs MFMA substeps");
    static_assert(LA::PLANES == MATH::PA && LB::PLANES == MATH::PB, "plane count");
    static_assert(TM >= 1 && TN >= 1, "wave tile below one MFMA block");
    static_assert(NT % 8 == 0, "lane_kb assumes whole rows of chunks per pass");
    constexpr int KPS = LA::KPS, NSUB = ROWB / MATH::KSB;
    constexpr bool B_I4 = (FB == Fmt::I4P);
    constexpr bool ADMA = CF::ADMA;
    constexpr int ASL = ADMA ? CF::ASL : 1;

    extern __shared__ __attribute__((aligned(16))) char smem[];

    // ---- which problem / tile / K slice ----
    // Heavy tiles come first (workgroups [0, nheavy), renumbered over the XCDs), then the
    // light ones: a problem's last row tile when it holds at most half of the tile's rows and
    // the waves past M skip their work. Light tiles then fill the CUs that the heavy tiles'
    // last round leaves idle, round-robin over the XCDs, instead of stretching a round of
    // their own. (Launches that order nothing have no light tiles.)
    const int wg = (int)blockIdx.x;
    const bool heavy = wg < args.nheavy;
    int split = 0, tile, p = 0;
    if (heavy) {
        const int lid = xcd_remap(wg, args.nheavy, args.xcds);
        split = lid % args.splitk;
        tile = lid / args.splitk;   // heavy tile index over all problems
#pragma unroll 1
        while (p + 1 < args.nprob && tile >= args.tile_start[p + 1]) p++;
        tile -= args.tile_start[p];
    } else {
        tile = wg - args.nheavy;
#pragma unroll 1
        while (p + 1 < args.nprob && tile >= args.light_start[p + 1]) p++;
        tile -= args.light_start[p];
    }
    const Problem &P = args.prob[p];
    const DumpWin dwin{P.dump, P.dump_row0, P.dump_rows};
    const int M = P.M, N = args.N;
    const int nbm = (M + BM - 1) / BM;
    // a problem with a light tile has nbm - 1 heavy row tiles (column block bn: tile / rows)
    const int nbh = nbm - (args.light_start[p + 1] > args.light_start[p] ? 1 : 0);
    int bm = nbm - 1, bn = tile;
    if (heavy) {
        if (args.bandm > 0 && args.bandm < nbh) {
            // row bands of bandm row tiles (the last may be shorter), M fastest inside a band
            const int full = args.bandm * args.nbn, band = tile / full, r = tile - band * full;
            const int rows = min(args.bandm, nbh - band * args.bandm);
            bm = band * args.bandm + r % rows;
            bn = r / rows;
        } else {
            bm = tile % nbh;
            bn = tile / nbh;
        }
    }
    const int kbeg = args.kbeg + split * args.kper;
    const int kend = min(args.kend, kbeg + args.kper);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    constexpr int BS = MATH::BS;
    const int rowA = wm * WTM + lane % BS;   // A-tile row of block i: rowA + BS i
    const int rowB = wn * WTN + lane % BS;   // B-tile row of block j: rowB + BS j

    typename MATH::Acc acc[TM][TN][MATH::NACC];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int a = 0; a < MATH::NACC; a++) acc[i][j][a] = typename MATH::Acc{};

    constexpr int TMG = GW ? TM : 1, TNG = GW ? TN : 1;
    typename MATH::AccF accf[TMG][TNG];
#pragma unroll
    for (int i = 0; i < TMG; i++)
#pragma unroll
        for (int j = 0; j < TNG; j++) accf[i][j] = typename MATH::AccF{};

    // output coordinates of this lane: column ncol + 32 j, rows mrow + 32 i + 8 q + r
    const int mrow = bm * BM + wm * WTM + 4 * (lane / BS);
    const int ncol = bn * BN + wn * WTN + lane % BS;

    // ---- operand streams ----
    const uint32_t lda = args.lda, ldb = args.ldb;
    const int ra0 = bm * BM, rb0 = bn * BN;
    const char *At = static_cast<const char *>(P.A) + (size_t)ra0 * lda;
    // GLU: the tile's B rows pair gate rows (P.B) and up rows (P.B2) of the same BN / 2
    // output columns, from source row rb0 / 2 on
    constexpr bool GLU = (EPI == Epi::GLU);
    const int brow0 = GLU ? rb0 / 2 : rb0, bvalid = GLU ? min(BN / 2, N / 2 - rb0 / 2) : min(BN, N - rb0);
    const char *Bt = static_cast<const char *>(P.B) + (size_t)brow0 * ldb;
    const char *Bt2 = GLU ? static_cast<const char *>(P.B2) + (size_t)brow0 * ldb : Bt;
    const uint32_t Va = (uint32_t)min(BM, M - ra0) * lda, Vb = (uint32_t)bvalid * ldb;
    const uint32_t kenda = LA::kbytes(kend), kendb = LB::kbytes(kend);
    const uint32_t lka = LA::lane_kb(tid), lkb = LB::lane_kb(tid);
    uint32_t voa[LA::CH], vob[LB::CH];
#pragma unroll
    for (int i = 0; i < LA::CH; i++) voa[i] = LA::voff(i, lda, tid);
#pragma unroll
    for (int i = 0; i < LB::CH; i++) {
        if constexpr (GLU) vob[i] = LB::voff_pair(i, ldb, tid);
        else vob[i] = LB::voff(i, ldb, tid);
    }

    // LDS of stage s: A plane(s) at a_at(s), B plane(s) at b_at(s), its group scales at
    // sc_at(s). Ring layout: two stages of [A | B | scales]. A-DMA layout: ASL A slots, BSL
    // B slots, then two scale slots. The tile's row scales follow either.
    auto a_at = [&](int s) __attribute__((always_inline)) -> char * {
        if constexpr (ADMA) return smem + (s % ASL) * PLA;
        else return smem + (s & 1) * STAGE;
    };
    auto b_at = [&](int s) __attribute__((always_inline)) -> char * {
        if constexpr (ADMA) return smem + ASL * PLA + (s % CF::BSL) * CF::BSTAGE;
        else return smem + (s & 1) * STAGE + MATH::PA * PLA;
    };
    auto sc_at = [&](int s) __attribute__((always_inline)) -> float * {
        if constexpr (ADMA) return reinterpret_cast<float *>(smem + ASL * PLA + CF::BSL * CF::BSTAGE + (s & 1) * CF::SCB);
        else return reinterpret_cast<float *>(smem + (s & 1) * STAGE + MATH::PA * PLA + MATH::PB * PLB);
    };
    float *rsl = reinterpret_cast<float *>(ADMA ? smem + ASL * PLA + CF::BSL * CF::BSTAGE + 2 * CF::SCB
                                                : smem + 2 * STAGE);
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    // Group-wise tiles with groups of 32 or 64 (fold-bound): a wave whose rows all lie past M
    // (the last M tile of a short problem, e.g. an expert's few rows beyond a multiple of BM)
    // skips its fragment reads, MFMAs and fold; it still issues its part of every stage's
    // loads and meets every barrier. (Grouped MoE launch at group 32: 270 -> 266 us per
    // forward. The test costs the group-128 int4 kernel 3% at 512 x 3840 x 15360, whose tiles
    // are never short: left out there.)
    constexpr bool SKIP = GW && (GM == 1 || GM == 2);
    const bool live = !SKIP || ra0 + (wave_u / WGN) * WTM < M;
    DmaA<BM, NT / 64> dma;
    if constexpr (ADMA) dma.init(lda, wave_u, lane);
    constexpr bool BDMA = CF::BDMA;
    DmaA<BN, NT / 64> dmb;
    if constexpr (BDMA && GLU) dmb.init_pair(ldb, wave_u, lane);
    else if constexpr (BDMA) dmb.init(ldb, wave_u, lane);
    // GLU with B by DMA: this wave's B rows come from the gate or the up source only
    const char *Btw = (BDMA && GLU && DmaA<BN, NT / 64>::pair_half(wave_u)) ? Bt2 : Bt;
    // vector-memory instructions one stage issues (the DMA waits count them): exactly those
    // load_stage issues, so scale loads only for group-wise tiles. A count above the issued
    // loads would let the next stage's last DMA loads still be in flight at the barrier.
    constexpr int NVM = (ADMA ? DmaA<BM, NT / 64>::INS : 0) + (BDMA ? DmaA<BN, NT / 64>::INS : LB::VM) +
                        (GW ? SL::NB + SL::NA : 0);

    typename SL::Cols scols;
    Rsrc srb = rsrc(P.b_scale, 0u), sra = rsrc(P.a_scale, 0u);
    if constexpr (GW) {
        scols.init(args.nG, rb0, N, ra0, M, tid);
        srb = rsrc(P.b_scale, (uint32_t)N * (uint32_t)args.nG * 4u);
        if constexpr (!ROWSCALE) sra = rsrc(P.a_scale, (uint32_t)M * (uint32_t)args.nG * 4u);
    }

    // Per-group activation scales that are the same for every group of a row (a per-row scale
    // passed in the reference's [M][nG] layout): that row folds in the row-scale order,
    // fmaf(b_scale, P_g, acc) and the row's scale at the store, and any other row in the
    // reference order; the choice depends on the row's own scales only (4 <= nG <= 64; other
    // nG keep the reference order everywhere), so a row's bits do not depend on the rows
    // batched with it (oracle: matmul_gw_rowscale_f32 with the row's first scale, or
    // matmul_gw_f32). In a tile that mixes both kinds, the row-scale rows run the reference
    // loop with their staged activation scales replaced by 1.0 (fmaf(1 * b, P, acc) is
    // fmaf(b, P, acc)) and their scale applied at the store. A tile whose rows are all of the
    // row kind runs a loop that folds in the row-scale order directly, one VALU operation
    // less per output and group (config 3 through the reference entry ~57 -> ~49 us), and
    // stops loading the per-group A scales. The check reads every scale of the tile's rows
    // once, 16 bytes at a time, issued ahead of the first stages and compared after them.
    [[maybe_unused]] bool rowc = false;
    constexpr bool PGS = GW && !ROWSCALE;
    // threads per row, and 16-byte chunks per thread for nG <= 64 (16 chunks a row)
    constexpr int RC_TPR = NT / BM, RC_MAX = (16 + RC_TPR - 1) / RC_TPR;
    static_assert(!PGS || (NT % BM == 0 && BM % 64 == 0), "whole waves per row sub-range");
    [[maybe_unused]] i32x4 rcv[PGS ? RC_MAX : 1];
    [[maybe_unused]] float rc0 = 0.f;
    [[maybe_unused]] bool rcheck = false;
    [[maybe_unused]] const int rc_row = tid % BM, rc_sub = tid / BM, rc_nc = (args.nG + 3) / 4;
    if constexpr (PGS) {
        const int nG = args.nG;
        rcheck = nG >= 4 && nG <= 64;
        const int m = ra0 + rc_row;
        const uint32_t roff = m < M ? (uint32_t)m * (uint32_t)nG * 4u : kOOB;
        rc0 = ld4f(sra, roff);
        if (rcheck) {
#pragma unroll
            for (int c = 0; c < RC_MAX; c++) {
                const int ci = rc_sub + c * RC_TPR;   // this thread's chunk ci of the row
                if (ci < rc_nc)   // the row's last chunk moved back to end at the row's end
                    rcv[c] = ld16(sra, roff + (uint32_t)min(4 * ci, nG - 4) * 4u);
            }
        }
    }

    // Stage at element k: descriptors start at byte k of the tile's rows and end with the
    // tile's valid rows (none past kend); a partial last stage masks this lane's chunks.
    // Integer products need only one operand's K tail zeroed: K and every slice end are
    // multiples of 32, so B's masked chunks cover exactly the tail, and the A bytes read
    // there instead (the row's next bytes, or zero past the tile's rows) are finite
    // integers multiplied by zero. 8-wave integer tiles skip the A mask (VALU per stage).
    constexpr bool AMASK = !(ADMA && (FA == Fmt::I8 || FA == Fmt::I16) &&
                             (FB == Fmt::I8 || FB == Fmt::I4P || FB == Fmt::I16));
    auto load_stage = [&](LA &la, LB &lb, SL &ls, int k, int st) __attribute__((always_inline)) {
        // k is the same in every lane: said so, its offsets stay scalar
        k = __builtin_amdgcn_readfirstlane(k);
        const uint32_t ka = LA::kbytes(k), kb = LB::kbytes(k);
        // (256x256 tiles: descriptors read from the first lane, see rsrc_u)
        const auto mk = [](const char *b, uint32_t n) __attribute__((always_inline)) {
            if constexpr (CF::W8W) return rsrc_u(b, n);
            else return rsrc(b, n);
        };
        const Rsrc rA = mk(At + ka, ka < kenda ? Va - ka : 0u);
        if constexpr (ADMA) dma.template issue<AMASK>(rA, a_at(st), ka, kenda, wave_u);
        else la.load(rA, voa, ka + lka < kenda ? 0u : kOOB);
        const Rsrc rB = mk((BDMA && GLU ? Btw : Bt) + kb, kb < kendb ? Vb - kb : 0u);
        if constexpr (BDMA) dmb.issue(rB, b_at(st), kb, kendb, wave_u);
        else if constexpr (GLU) lb.load_pair(rB, rsrc(Bt2 + kb, kb < kendb ? Vb - kb : 0u), vob, kb + lkb < kendb ? 0u : kOOB);
        else lb.load(rB, vob, kb + lkb < kendb ? 0u : kOOB);
        if constexpr (GW) ls.load(srb, sra, scols, k, args.gmag, args.nG, rowc, tid);
    };

    // Plain tiles with both operands by DMA keep a whole stage of fragments in registers,
    // read one stage ahead: the MFMAs of stage s run from registers while stage s + 1's
    // fragments come from LDS, so the first MFMA after each barrier waits for no LDS read.
    // The RS LDS slots hold stages s + 1 (complete) to s + RS (in flight); the register set
    // is one more buffer.
    constexpr bool FULLREG = ADMA && BDMA && !GW && !CF::W8W;
    if constexpr (FULLREG) {
        constexpr int RS = CF::ASL;
        static_assert(MATH::PA == 1 && MATH::PB == 1 && CF::BSL == RS && RS >= 3 && (RS - 1) * NVM < 64, "ring");
        LA la0;
        LB lb0;
        SL ls0;
        const int nst = (kend - kbeg + KPS - 1) / KPS;
        i32x4 fr[2][NSUB][TM + TN];
        auto read_stage = [&](auto FS, int s) __attribute__((always_inline)) {
            constexpr int f = decltype(FS)::value;
            const char *ca = a_at(s), *cb = b_at(s);
            static_for<NSUB>([&](auto SS) __attribute__((always_inline)) {
                constexpr int ss = decltype(SS)::value;
#pragma unroll
                for (int i = 0; i < TM; i++) fr[f][ss][i] = lds_frag<MATH>(ca, rowA + BS * i, ss, lane);
#pragma unroll
                for (int j = 0; j < TN; j++) fr[f][ss][TM + j] = lds_frag<MATH>(cb, rowB + BS * j, ss, lane);
            });
        };
        // stages 0 .. RS - 1 in flight; stage 0 read into set 0 once every wave's part landed
#pragma unroll
        for (int u = 0; u < RS; u++) load_stage(la0, lb0, ls0, kbeg + u * KPS, u);
        __builtin_amdgcn_sched_barrier(0);
        wait_vm<(RS - 1) * NVM>();
        lds_barrier();
        read_stage(std::integral_constant<int, 0>{}, 0);
        __builtin_amdgcn_sched_barrier(0);
        wait_vm<(RS - 2) * NVM>();
        lds_barrier();
        // Stage s: slot s % RS was read into registers before the last barrier, so stage
        // s + RS's DMA may overwrite it; stage s + 1 landed before that barrier.
        auto stage = [&](auto FS, int s) __attribute__((always_inline)) {
            constexpr int f = decltype(FS)::value;
            load_stage(la0, lb0, ls0, kbeg + (s + RS) * KPS, s + RS);
            read_stage(std::integral_constant<int, f ^ 1>{}, s + 1);
            static_for<NSUB>([&](auto SS) __attribute__((always_inline)) {
                constexpr int ss = decltype(SS)::value;
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++) MATH::mma(acc[i][j], &fr[f][ss][i], &fr[f][ss][TM + j]);
            });
            // each substep's TM + TN fragment reads spread over its TM * TN MFMAs, and the
            // stage's DMA issued after half of them: issued first, right after the barrier,
            // its address arithmetic and M0 set-ups kept both waves of a SIMD away from the
            // matrix pipe at the same moment (the config-4 bf16 GEMM 331 -> 317 us a call,
            // the FFN block 229 -> 222 us; after a quarter or three quarters of the MFMAs, or
            // split between the two, measured in between)
            static_for<NSUB * TM * TN>([&](auto M) __attribute__((always_inline)) {
                constexpr int mi = decltype(M)::value;
                constexpr int m = mi % (TM * TN), R = TM + TN, MM = TM * TN;
                constexpr int nr = (m + 1) * R / MM - m * R / MM;
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if constexpr (nr > 0) __builtin_amdgcn_sched_group_barrier(0x100, nr, 0);
                if constexpr (mi == NSUB * TM * TN / 2 - 1) __builtin_amdgcn_sched_group_barrier(0x020, NVM, 0);
            });
            __builtin_amdgcn_sched_barrier(0);
            wait_vm<(RS - 2) * NVM>();
            lds_barrier();
        };
        const int npair = nst / 2 * 2;
#pragma unroll 1
        for (int s = 0; s < npair; s += 2) {
            stage(std::integral_constant<int, 0>{}, s);
            stage(std::integral_constant<int, 1>{}, s + 1);
        }
        if (npair < nst) stage(std::integral_constant<int, 0>{}, npair);
    } else {
        // D register sets keep loads for D stages in flight; the LDS holds two stages (A-DMA:
        // D + 1 A slots). Stage t lives in set t % D from its load until it is written to LDS
        // during stage t - 1; the K loop is unrolled by D so every set index is a constant.
        constexpr int D = CF::D;
        LA la[D];
        LB lb[D];
        SL ls[D];
        const int nst = (kend - kbeg + KPS - 1) / KPS;
    #pragma unroll
        for (int u = 0; u < D; u++) load_stage(la[u], lb[u], ls[u], kbeg + u * KPS, u);
        if constexpr (!ADMA) la[0].store(a_at(0), PLA, tid);
        if constexpr (!BDMA) lb[0].store(b_at(0), PLB, tid);
        // (per-group activation scales: stage 0's scales are stored once the rows' orders are known)
        if constexpr (GW && !PGS) ls[0].store(sc_at(0), tid, scols);
        if constexpr (GW && ROWSCALE)
            if (tid < BM) rsl[tid] = ra0 + tid < M ? P.a_scale[ra0 + tid] : 0.f;
        [[maybe_unused]] int *rowmis = reinterpret_cast<int *>(rsl + BM);   // [NT / BM][BM]
        [[maybe_unused]] int *wflag = rowmis + NT;                          // [NT / 64]
        if constexpr (PGS) {
            bool mis = false;
            if (rcheck) {
#pragma unroll
                for (int c = 0; c < RC_MAX; c++)
                    if (rc_sub + c * RC_TPR < rc_nc)
#pragma unroll
                        for (int e = 0; e < 4; e++) mis |= rcv[c][e] != __float_as_int(rc0);
            }
            rowmis[rc_sub * BM + rc_row] = mis;
        }
        if constexpr (ADMA) {   // stage 0's DMA data is in LDS once only the later stages' loads remain
            __builtin_amdgcn_sched_barrier(0);
            wait_vm<NVM * (D - 1)>();
        }
        lds_barrier();
        if constexpr (PGS) {
            // each row's order: its scale at the store (1.0 for reference-order rows, whose
            // activation scales enter the fold), its staged activation scales, and whether the
            // whole tile is of the row kind
            bool rm = true;
            if (tid < BM) {
                rm = !rcheck || row_mis<BM, NT>(rowmis, tid);
                rsl[tid] = rm ? 1.0f : rc0;   // rows past M (scales read as 0): never stored
            }
            const bool wmis = __builtin_amdgcn_ballot_w64(tid < BM && rm) != 0;
            if (lane == 0) wflag[wave_u] = wmis;
            scols.set_unit(rowmis, rcheck, tid);
            ls[0].store(sc_at(0), tid, scols);
            lds_barrier();
            int any = 0;
#pragma unroll
            for (int w = 0; w < NT / 64; w++) any |= wflag[w];
            rowc = __builtin_amdgcn_readfirstlane(rcheck && !any) != 0;
        }

        // One stage: prefetch stage s + D into set u, run the MFMAs of stage s from LDS slot
        // s % 2, write stage s + 1 (set (u + 1) % D) into slot (s + 1) % 2, then one barrier.
        // Slot (s + 1) % 2 was last read in stage s - 1, which every wave finished at the
        // previous barrier, so its writes may go anywhere in the stage: fp32-operand formats
        // (whose conversion VALU work then overlaps the MFMAs) write at the start, the integer
        // formats at the end (measured faster for each).
        constexpr bool EARLY_STORE = (FA == Fmt::F32BF16 || FA == Fmt::F32TF32 || FB == Fmt::F32BF16 ||
                                      FB == Fmt::F32TF32);
        auto store_next = [&](auto U, int s) __attribute__((always_inline)) {
            constexpr int v = (decltype(U)::value + 1) % D;
            if constexpr (!ADMA) la[v].store(a_at(s + 1), PLA, tid);
            if constexpr (!BDMA) lb[v].store(b_at(s + 1), PLB, tid);
            if constexpr (GW) ls[v].store(sc_at(s + 1), tid, scols);
        };
        // Block-row order (8-wave group-wise tiles whose groups are single stages, folding in the
        // row-scale order): a stage runs its MFMAs one block row at a time (row i: the TN blocks
        // (i, j), all NSUB substeps), so block row i's partials are whole after its phase, and
        // their fold runs among the MFMAs of row i + 1 — the last row's among the first row's of
        // the next stage — instead of every wave folding all its blocks after all its MFMAs
        // while the matrix pipe idles. The zero-input MFMA that opens a block's next group comes
        // after its fold in program order. The stage's B fragments stay in registers for all
        // rows; A fragments are read per row. pend_sb: the B scales of the last row's pending
        // fold (0 before the first stage: the zero partials then add exactly 0). Config 3:
        // 48.6 -> 46.5 us on one box. Left to the scheduler inside each phase: one MFMA per 2, 4
        // or 8 fold operations forced with sched_group_barrier measured 1-4 us slower, and the
        // B unpack and store moved between the phases 2-3 us slower.
        constexpr bool BMJ_OK = GW && CF::W8 && !CF::W16 && GM == 4 && NGS == 1 && MATH::NACC == 1 && TM >= 2;
        [[maybe_unused]] float pend_sb[TN];
#pragma unroll
        for (int j = 0; j < TN; j++) pend_sb[j] = 0.f;
        // Deferred folds for one-block waves whose groups close every substep (groups of 32,
        // row-scale order): a second set of partials takes the groups of odd substeps, so each
        // substep issues its MFMA first and then folds the previous substep's group while the
        // MFMA runs (the one-block wave otherwise waits out every MFMA's latency before its
        // fold). The last substep's group of a stage folds at the next stage's first substep;
        // the second set starts at zero, so the first stage's fold of it adds exactly 0.
        constexpr bool DFR_OK = GW && GM == 1 && TM == 1 && TN == 1 && MATH::NACC == 1 && NGS == NSUB && NSUB % 2 == 0;
        [[maybe_unused]] typename MATH::Acc accq[TM][TN][1];
        accq[0][0][0] = typename MATH::Acc{};
        // RC: the row-scale fold order of a tile whose per-group activation scales are constant
        // along every row (the K loop runs in one of two copies, one per order)
        auto stage = [&](auto U, int s, auto RCT, auto CHKT) __attribute__((always_inline)) {
            constexpr int u = decltype(U)::value;
            constexpr bool RC = decltype(RCT)::value;
            constexpr bool BMJ = BMJ_OK && (ROWSCALE || RC);
            const char *ca = a_at(s), *cb = b_at(s);
            const int k0 = kbeg + s * KPS;
            // set u is free: its stage went to LDS during the previous stage
            load_stage(la[u], lb[u], ls[u], k0 + D * KPS, s + D);
            if constexpr (EARLY_STORE) store_next(U, s);
            // fragments: with A-DMA two sets, the next substep's read issued before this
            // substep's MFMAs; otherwise one set, read at its substep
            constexpr int NFB = ADMA ? 2 : 1;
            i32x4 fa[NFB][TM][MATH::PA], fb[NFB][TN][MATH::PB];
            auto ldfr = [&](auto FSET, int ss) __attribute__((always_inline)) {
                constexpr int f = decltype(FSET)::value;
    #pragma unroll
                for (int i = 0; i < TM; i++)
    #pragma unroll
                    for (int pl = 0; pl < MATH::PA; pl++) fa[f][i][pl] = lds_frag<MATH>(ca + pl * PLA, rowA + BS * i, ss, lane);
    #pragma unroll
                for (int j = 0; j < TN; j++)
    #pragma unroll
                    for (int pl = 0; pl < MATH::PB; pl++) fb[f][j][pl] = lds_frag<MATH>(cb + pl * PLB, rowB + BS * j, ss, lane);
            };
            // B scales of the groups that close at compile-time substeps in this stage, read
            // before any fragment: the fold then waits for no LDS read issued after them
            constexpr bool CT = GW && GM >= 1 && GM <= 4;
            constexpr int GMS = CF::GMS;   // substeps per group (compile-time cadence)
            static_assert(!CT || (GM * 32) % MATH::KEL == 0, "a substep inside one group");
            constexpr int NGC = CT ? NSUB / (GMS > 0 ? GMS : 1) : 1;
            float sbs[NGC][TN];
            // CHK: the stage may reach past kend or dumps partials (run-time group checks and
            // the dump branch); without, every compile-time group closes and the stage's body
            // has no branch, so the scheduler can place each fold among the MFMAs around it
            auto compute = [&](auto CHKT) __attribute__((always_inline)) {
            constexpr bool CHK = decltype(CHKT)::value;
            if constexpr (CT) {
#pragma unroll
                for (int g = 0; g < NGC; g++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        sbs[g][j] = gw_bscale<CF>(sc_at(s), NGS == 1 ? 0 : ((g + 1) * GMS - 1) * MATH::KEL / 32, wn, j, lane);
            }
            if constexpr (ADMA) ldfr(std::integral_constant<int, 0>{}, 0);
            static_for<NSUB>([&](auto SS) __attribute__((always_inline)) {
                constexpr int ss = decltype(SS)::value;
                constexpr int f = ADMA ? (ss & 1) : 0;
                // compile-time group cadence: this substep opens / closes a quant group
                constexpr bool opens = GW && GM >= 1 && GM <= 4 && ss % (GMS > 0 ? GMS : 1) == 0;
                constexpr bool closes = GW && GM >= 1 && GM <= 4 && ss % (GMS > 0 ? GMS : 1) == (GMS > 0 ? GMS : 1) - 1;
                if constexpr (!ADMA) ldfr(std::integral_constant<int, 0>{}, ss);
                else if constexpr (ss + 1 < NSUB) {
                    ldfr(std::integral_constant<int, (ss + 1) & 1>{}, ss + 1);
                    // Plain products (here those with int4 B, which keep this one-substep
                    // scheme): keep the next substep's LDS reads ahead of this substep's MFMAs
                    // (left to itself the scheduler sinks them below, and each substep's first
                    // MFMA waits out a full LDS latency with the matrix pipe idle; measured on
                    // int8 at 512 x 3840 x 15360 before its whole-stage scheme: 42.3 -> 38.4 us).
                    // Group-wise tiles measured faster with the reads left to the scheduler
                    // among their fold VALU (47 against 50 us).
                    if constexpr (!GW) __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++) {
                        if constexpr (opens) MATH::mma0(acc[i][j], fa[f][i], fb[f][j]);
                        else MATH::mma(acc[i][j], fa[f][i], fb[f][j]);
                    }

                if constexpr (GW) {
                    const int kpos = k0 + (ss + 1) * MATH::KEL;   // K consumed so far
                    const float *sc = sc_at(s);
                    constexpr bool rt = (GM == 0 || (GM == 8 && ss == NSUB - 1));   // run-time cadence
                    if constexpr (closes || rt) {
                        const bool close =
                            (CHK || rt) ? (kpos <= kend && (closes || div32m(kpos, args.tmag) * args.kt == kpos)) : true;
                        if (close) {
                            const int slot = NGS == 1 ? 0 : ss * MATH::KEL / 32;
                            if constexpr (CT) {
                                gw_group<CF, ROWSCALE || RC, B_I4, rt, CHK>(args, dwin, acc, accf, sbs[ss / GMS], sc, slot,
                                                                            kpos, wm, lane, mrow, ncol, N);

                            } else {
                                float sb[TN];
#pragma unroll
                                for (int j = 0; j < TN; j++) sb[j] = gw_bscale<CF>(sc, slot, wn, j, lane);
                                gw_group<CF, ROWSCALE || RC, B_I4, rt, true>(args, dwin, acc, accf, sb, sc, slot, kpos, wm,
                                                                             lane, mrow, ncol, N);
                            }
                        }
                    }
                }
            });
            };
            auto compute_dfr = [&](auto CHKT) __attribute__((always_inline)) {
                constexpr bool CHK = decltype(CHKT)::value;
                if constexpr (DFR_OK) {
                // this lane's B scale of each of the stage's groups (slot g: substep g)
                float sbg[NSUB];
#pragma unroll
                for (int g = 0; g < NSUB; g++) sbg[g] = gw_bscale<CF>(sc_at(s), g, wn, 0, lane);
                // fragments: with A-DMA two sets, the next substep's read issued ahead; otherwise
                // one set, read at its substep
                if constexpr (ADMA) ldfr(std::integral_constant<int, 0>{}, 0);
                static_for<NSUB>([&](auto SS) __attribute__((always_inline)) {
                    constexpr int ss = decltype(SS)::value, f = ss & 1, fs = ADMA ? f : 0;
                    if constexpr (!ADMA) ldfr(std::integral_constant<int, 0>{}, ss);
                    else if constexpr (ss + 1 < NSUB) ldfr(std::integral_constant<int, f ^ 1>{}, ss + 1);
                    auto &cur = f ? accq : acc;
                    auto &prv = f ? acc : accq;
                    MATH::mma0(cur[0][0], fa[fs][0], fb[fs][0]);
                    // the previous substep's group: K through it is kp (the zeros before the
                    // first stage fold as 0 with pend_sb = 0; groups past kend never close)
                    const int kp = k0 + ss * MATH::KEL;
                    if (!CHK || ss == 0 || kp <= kend) {
                        gw_fold_block<CF, true>(prv[0][0][0], accf[0][0], ss == 0 ? pend_sb[0] : sbg[ss > 0 ? ss - 1 : 0], nullptr, 0,
                                                0, wm, lane);
#if defined(__HIP_DEVICE_COMPILE__)
                        asm volatile("" ::"v"(accf[0][0]));
#endif
                        if constexpr (CHK)
                            if (kp > kbeg) gw_dump<CF, B_I4>(args, dwin, prv, kp, mrow, ncol, N);
                    }
                });
                pend_sb[0] = sbg[NSUB - 1];
                }
            };
            auto compute_bmj = [&]() __attribute__((always_inline)) {
                if constexpr (BMJ_OK) {
                float sbn[TN];
#pragma unroll
                for (int j = 0; j < TN; j++) sbn[j] = gw_bscale<CF>(sc_at(s), 0, wn, j, lane);
                i32x4 fbv[NSUB][TN], fav[TM][NSUB];
                static_for<TM>([&](auto I) __attribute__((always_inline)) {
                    constexpr int i = decltype(I)::value;
                    static_for<NSUB>([&](auto SS) __attribute__((always_inline)) {
                        constexpr int ss = decltype(SS)::value;
                        fav[i][ss] = lds_frag<MATH>(ca, rowA + BS * i, ss, lane);
                        if constexpr (i == 0)
#pragma unroll
                            for (int j = 0; j < TN; j++) fbv[ss][j] = lds_frag<MATH>(cb, rowB + BS * j, ss, lane);
                    });
                    static_for<NSUB>([&](auto SS) __attribute__((always_inline)) {
                        constexpr int ss = decltype(SS)::value;
#pragma unroll
                        for (int j = 0; j < TN; j++) {
                            if constexpr (ss == 0) MATH::mma0(acc[i][j], &fav[i][ss], &fbv[ss][j]);
                            else MATH::mma(acc[i][j], &fav[i][ss], &fbv[ss][j]);
                        }
                    });
                    // the previous block row's fold: row TM - 1 of the previous group in the
                    // first phase, row i - 1 of this group in the others
                    constexpr int fi = i == 0 ? TM - 1 : i - 1;
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        gw_fold_block<CF, true>(acc[fi][j][0], accf[fi][j], i == 0 ? pend_sb[j] : sbn[j], nullptr, 0, fi,
                                                wm, lane);
                    // keep the fold in this phase (left alone, the compiler sinks it to the loop
                    // latch, keeping every partial alive and renaming the next group's)
                    // (device pass only: the host pass, which also instantiates kernel templates
                    // to emit their launch stubs, has no VGPR constraint and would drop the stub)
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
                    for (int j = 0; j < TN; j++) asm volatile("" ::"v"(accf[fi][j]));
#endif
                });
                // every block now holds this group's partials (row 0's are overwritten only by
                // the next stage's first phase)
                gw_dump<CF, B_I4>(args, dwin, acc, k0 + KPS, mrow, ncol, N);
#pragma unroll
                for (int j = 0; j < TN; j++) pend_sb[j] = sbn[j];
                }
            };
            if (live) {
                if constexpr (BMJ) {
                    compute_bmj();
                } else if constexpr (DFR_OK && (ROWSCALE || RC)) {
                    compute_dfr(CHKT);
                } else {
                    compute(CHKT);
                }
            }
            if constexpr (!EARLY_STORE) store_next(U, s);
            if constexpr (ADMA) {   // stage s + 1's DMA data is in LDS once only later stages' loads remain
                __builtin_amdgcn_sched_barrier(0);
                wait_vm<NVM * (D - 1)>();
            }
            lds_barrier();
        };

        // The steady state runs whole groups of D stages with no branch around a memory access
        // (a loop exit between stages would make the loop head wait for every prefetch); the
        // last nst % D stages run after it.
        // Every wave folds a group's partials at the end of the substep that closes it. (Two
        // waves of a SIMD folding in opposite halves of a stage, so that one's fold VALU runs
        // under the other's MFMAs, measured slower: 50 against 47 us at 512 x 3840 x 15360.)
        // Group-wise tiles with compile-time group cadence run their whole stages in a K loop
        // whose stages carry no group checks and no dump branch (CHK false: every group in
        // them closes, so a stage's body has no branch and the scheduler can place each fold
        // among the MFMAs around it); the stages that may reach past kend, and every stage of a
        // launch that dumps partials, run the checked body. (Chosen per loop, not per stage:
        // a checked and an unchecked body side by side in one loop spill the 16-wave tiles.)
        const int nwhole = (kend - kbeg) / KPS;
        auto kloop = [&](auto RCT, auto CHKT) __attribute__((always_inline)) {
            constexpr bool CHK = decltype(CHKT)::value;
            const int nloop = (CHK ? nst : nwhole) / D * D;
    #pragma unroll 1
            for (int s0 = 0; s0 < nloop; s0 += D)
                static_for<D>([&](auto U) __attribute__((always_inline)) { stage(U, s0 + decltype(U)::value, RCT, CHKT); });
            static_for<D>([&](auto U) __attribute__((always_inline)) {
                if (nloop + decltype(U)::value < nst) stage(U, nloop + decltype(U)::value, RCT, std::true_type{});
            });
        };
        // (DMA tiles only: the register-staged 128 x 128 group-wise tiles spill without the
        // checked body's branches)
        constexpr bool SPLITCHK = GW && GM >= 1 && GM <= 4 && !BMJ_OK && ADMA;
        auto kloop2 = [&](auto RCT) __attribute__((always_inline)) {
            if constexpr (SPLITCHK) {
                if (dwin.ptr != nullptr) kloop(RCT, std::true_type{});
                else kloop(RCT, std::false_type{});
            } else {
                kloop(RCT, std::true_type{});
            }
        };
        if constexpr (PGS) {
            if (rowc) kloop2(std::true_type{});
            else kloop2(std::false_type{});
        } else {
            kloop2(std::false_type{});
        }
        // deferred folds: the last stage's last substep closes a group only when the K range
        // is whole stages (otherwise its last group closed, and folded, inside the stage)
        if constexpr (DFR_OK) {
            if (live && (ROWSCALE || rowc) && (kend - kbeg) % KPS == 0) {
                gw_fold_block<CF, true>(accq[0][0][0], accf[0][0], pend_sb[0], nullptr, 0, 0, wm, lane);
                gw_dump<CF, B_I4>(args, dwin, accq, kend, mrow, ncol, N);
            }
        }
        // block-row order: the last group's last block row is still to fold
        if constexpr (BMJ_OK) {
            if (live && (ROWSCALE || rowc)) {
#pragma unroll
                for (int j = 0; j < TN; j++)
                    gw_fold_block<CF, true>(acc[TM - 1][j][0], accf[TM - 1][j], pend_sb[j], nullptr, 0, TM - 1, wm, lane);
            }
        }
        // the stages past the end still have (zero-filled) DMA loads in flight into LDS: drain
        // them before the workgroup's LDS can be handed to another
        if constexpr (ADMA) wait_vm<0>();
    }

    // ---- epilogue: lane holds column ncol + BS j of rows mrow + BS i + row_of(e) ----
    // Results in K slices: int32 slices add their sums into C with device-scope atomic adds
    // (exact in any order; C starts from zero, or from the sums being accumulated into);
    // fp32 slices store theirs into plane s of the workspace ([slice][M][N], one problem)
    // and a second kernel adds the planes in slice order (the same fp32 bits whichever slice
    // finishes first). No workgroup waits for another.
    float *const plane = ((EPI == Epi::F16 || EPI == Epi::F32) && args.splitk > 1)
                             ? reinterpret_cast<float *>(args.ws) + (size_t)split * M * N
                             : nullptr;
    // (GLU / ACT: the activation kind dispatched once, each kind's stores a loop of their own.
    // The flags are read into registers first: inside the store loop the compiler cannot
    // tell that the result stores leave the kernel arguments alone, and reloaded them from
    // kernarg memory at every element.)
    const bool st_atomic = args.atomic != 0, st_accum = args.accum != 0, st_f16 = args.f16out != 0;
    void *const Cout = P.C;
    const _Float16 *const bias = static_cast<const _Float16 *>(P.B2);
    auto store_all = [&](auto ACTC) __attribute__((always_inline)) {
        [[maybe_unused]] constexpr int AK = decltype(ACTC)::value;
    #pragma unroll
        for (int i = 0; i < TM; i++)
    #pragma unroll
            for (int e = 0; e < MATH::NE; e++) {
                    const int m = mrow + BS * i + MATH::row_of(e);
                    if (m >= M) continue;
                    if constexpr (GLU) {
                        // each 64-row group of B tile rows holds 32 gate then 32 up columns: G = 32 / BS
                        // blocks of each, gate block 2 G g + t pairing with up block 2 G g + G + t
                        constexpr int G = 32 / BS;
                        static_assert(TN % (2 * G) == 0, "GLU pairs gate and up column blocks");
                        const int NO = N / 2;
    #pragma unroll
                        for (int jp = 0; jp < TN / 2; jp++) {
                            const int g = jp / G, t = jp % G, jg = 2 * G * g + t;
                            const int no = bn * (BN / 2) + wn * (WTN / 2) + 32 * g + BS * t + lane % BS;
                            if (no < NO)
                                static_cast<_Float16 *>(Cout)[(long)m * NO + no] =
                                    (_Float16)(act_k<AK>(acc[i][jg][0][e]) * acc[i][jg + G][0][e]);
                        }
                        continue;
                    }
                    const float rs = GW ? rsl[m - ra0] : 1.f;
    #pragma unroll
                    for (int j = 0; j < TN; j++) {
                        const int n = ncol + BS * j;
                        if (n >= N) continue;
                        const long off = (long)m * N + n;
                        if constexpr (EPI == Epi::I32) {
                            int v = acc[i][j][0][e];
                            if (B_I4) v >>= 4;   // exact: every int4 product carries x16
                            int32_t *c = static_cast<int32_t *>(Cout) + off;
                            if (st_atomic) {
                                __hip_atomic_fetch_add(c, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            } else if (st_accum) {
                                *c = v + *c;
                            } else {
                                __builtin_nontemporal_store(v, c);
                            }
                        } else if constexpr (EPI == Epi::I64) {
                            i64 *c = static_cast<i64 *>(Cout) + off;
                            i64 v = (i64)acc[i][j][0][e] * 65536 + (i64)acc[i][j][1][e] * 256 + (i64)acc[i][j][2][e];
                            if (st_accum) v += *c;
                            *c = v;
                        } else if constexpr (EPI == Epi::F16) {
                            if (plane) __builtin_nontemporal_store(acc[i][j][0][e], plane + off);
                            else static_cast<_Float16 *>(Cout)[off] = (_Float16)acc[i][j][0][e];
                        } else if constexpr (EPI == Epi::ACT) {
                            const float b = bias ? (float)bias[n] : 0.f;
                            static_cast<_Float16 *>(Cout)[off] = (_Float16)act_k<AK>(acc[i][j][0][e] + b);
                        } else if constexpr (EPI == Epi::F32) {   // results are not re-read: non-temporal
                            __builtin_nontemporal_store(acc[i][j][0][e], (plane ? plane : static_cast<float *>(Cout)) + off);
                        } else {   // GW
                            const float v = accf[i < TMG ? i : 0][j < TNG ? j : 0][e] * rs;
                            if (st_f16) static_cast<_Float16 *>(Cout)[off] = (_Float16)v;
                            else __builtin_nontemporal_store(v, static_cast<float *>(Cout) + off);
                        }
                    }
                }
    };
    if constexpr (GLU || EPI == Epi::ACT) {
        if (args.act == kActGelu) store_all(std::integral_constant<int, kActGelu>{});
        else if (args.act == kActSilu) store_all(std::integral_constant<int, kActSilu>{});
        else store_all(std::integral_constant<int, kActIdentity>{});
    } else {
        store_all(std::integral_constant<int, 0>{});
    }
}

// ------------------------------------------------------------------------------------
// Launch of one instantiation.
// ------------------------------------------------------------------------------------
template <int BM, int BN, Fmt FA, Fmt FB, class MATH, Epi EPI, bool RS, int GM = 0>
hipError_t launch_one(const KArgs &ka, int blocks, hipStream_t s)
{
    using CF = KCfg<BM, BN, FA, FB, MATH, EPI, RS, GM>;
    constexpr int lds = CF::ADMA ? CF::LDS_ADMA : CF::LDS_RING;
    static_assert(lds <= 160 * 1024, "LDS budget");
    auto kern = k_gemm<BM, BN, FA, FB, MATH, EPI, RS, GM>;
    // dynamic LDS above 64 KiB needs an opt-in, once per device (bit d of the mask; any
    // thread may launch, so the mask is atomic)
    static std::atomic<uint64_t> opted{0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return hipGetLastError();
    const uint64_t bit = dev >= 0 && dev < 64 ? (uint64_t)1 << dev : 0;
    if (!bit || !(opted.load(std::memory_order_acquire) & bit)) {
        if (hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                lds) != hipSuccess)
            return hipGetLastError();
        opted.fetch_or(bit, std::memory_order_release);
    }
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(CF::NT), lds, s, ka);
    return hipGetLastError();
}

// Group cadence of a group-wise launch (see KCfg): compile-time for 32, 64 and 128.
inline int gw_cadence(const Launch &L)
{
    if (L.kt == L.group && (L.group == 32 || L.group == 64 || L.group == 128)) return L.group / 32;
    return (L.group % 128 == 0 && L.kt % 128 == 0) ? 8 : 0;
}

template <int BM, int BN, Fmt FA, Fmt FB, bool RS>
hipError_t launch_gw_rs(const Launch &L, const KArgs &ka, int blocks)
{
    hipStream_t s = L.stream;
    switch (gw_cadence(L)) {
    case 1: return launch_one<BM, BN, FA, FB, MathI8, Epi::GW, RS, 1>(ka, blocks, s);
    case 2: return launch_one<BM, BN, FA, FB, MathI8, Epi::GW, RS, 2>(ka, blocks, s);
    case 4: return launch_one<BM, BN, FA, FB, MathI8, Epi::GW, RS, 4>(ka, blocks, s);
    case 8: return launch_one<BM, BN, FA, FB, MathI8, Epi::GW, RS, 8>(ka, blocks, s);
    default: return launch_one<BM, BN, FA, FB, MathI8, Epi::GW, RS, 0>(ka, blocks, s);
    }
}

template <int BM, int BN, Fmt FA, Fmt FB>
hipError_t launch_gw(const Launch &L, const KArgs &ka, int blocks)
{
    return L.rowscale ? launch_gw_rs<BM, BN, FA, FB, true>(L, ka, blocks)
                      : launch_gw_rs<BM, BN, FA, FB, false>(L, ka, blocks);
}

// The tile shapes the planner picks, as template arguments: f(BM, BN) with
// std::integral_constant arguments.
template <class F> hipError_t by_tile(int bm, int bn, F &&f)
{
    using std::integral_constant;
    if (bm == 256) return f(integral_constant<int, 256>{}, integral_constant<int, 128>{});
    if (bm == 128 && bn == 128) return f(integral_constant<int, 128>{}, integral_constant<int, 128>{});
    if (bm == 128) return f(integral_constant<int, 128>{}, integral_constant<int, 64>{});
    return f(integral_constant<int, 64>{}, integral_constant<int, 64>{});
}

// One operand family per translation unit.
hipError_t dispatch_int(int bm, int bn, const Launch &L, const KArgs &ka, int blocks);    // int8 / int4 -> int32, int16
hipError_t dispatch_gw_i8(int bm, int bn, const Launch &L, const KArgs &ka, int blocks);  // group-wise, int8 B
hipError_t dispatch_gw_i4(int bm, int bn, const Launch &L, const KArgs &ka, int blocks);  // group-wise, int4 B
hipError_t dispatch_f16(int bm, int bn, const Launch &L, const KArgs &ka, int blocks);    // fp16 operands
hipError_t dispatch_bf16(int bm, int bn, const Launch &L, const KArgs &ka, int blocks);   // fp32 / bf16 / tf32 operands

}  // namespace gk
}  // namespace rk
