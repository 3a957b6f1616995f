// gemm.hip — gfx950 MFMA GEMM kernels for every matmul entry of the library.
//
// C[M,N] = A[M,K] * B[N,K]^T with both operands K-contiguous. One workgroup owns a
// BM x BN output tile; its 4 waves (2 x 2) own (BM/2) x (BN/2) sub-tiles built from
// 32x32 MFMA blocks (v_mfma_i32_32x32x32_i8, v_mfma_f32_32x32x16_{f16,bf16}: the 16x16
// shapes issue at half rate on gfx950). K advances in stages of 128 LDS bytes per tile
// row; each stage goes global -> registers -> LDS (double-buffered, one barrier per
// stage) while the previous stage feeds the MFMAs.
//
// MFMA operand convention: the B fragment is the instruction's first operand and the A
// fragment its second, so in each 32x32 result block lane l holds row m = l % 32 and the
// columns 8q + 4(l/32) + {0..3}, q = 0..3: four 16-byte vector stores per lane per block.
// Lane l supplies row l % 32 of each fragment and bytes [16*(l/32), +16) of the 32-byte
// K substep, identically for both operands.
#include "gemm.h"

#include <stdlib.h>

#include <algorithm>
#include <type_traits>

namespace rk {
namespace {

typedef int      i32x4  __attribute__((ext_vector_type(4)));
typedef int      i32x2  __attribute__((ext_vector_type(2)));
typedef float    f32x4  __attribute__((ext_vector_type(4)));
typedef float    f32x16 __attribute__((ext_vector_type(16)));
typedef int      i32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8  __attribute__((ext_vector_type(8)));
typedef __bf16   bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4  __attribute__((ext_vector_type(4)));
typedef long long i64;

constexpr int ROWB = 128;   // LDS bytes per tile row per plane per stage

// Chunk c of row r sits at slot c ^ ((r >> 1) & 7): the sixteen lanes an LDS cycle serves
// (sixteen consecutive rows, one chunk) cover all 64 banks once.
__device__ __forceinline__ int swz(int row, int chunk) { return row * ROWB + ((chunk ^ ((row >> 1) & 7)) << 4); }

// ------------------------------------------------------------------------------------
// Kernel arguments (passed by value: the problem table travels in the kernarg segment).
// ------------------------------------------------------------------------------------
struct KArgs {
    int N, K, kbeg, kend, accum, group, kt, nG;
    long lda, ldb;                       // bytes per row of A and of B
    int nprob;
    int tile_start[kMaxProblems + 1];    // prefix sums of per-problem tile counts
    Problem prob[kMaxProblems];
    int32_t *dump;
    int dump_row0, dump_rows;
    int xcds;                            // XCDs to renumber workgroups over (1: keep order)
};

// Workgroup w is dispatched to XCD w % 8. Renumber so the workgroups of one XCD get
// consecutive logical ids, then walk M fastest: an XCD's tiles share B column blocks,
// which its own L2 then serves.
__device__ __forceinline__ int xcd_remap(int w, int G, int X)
{
    if (X <= 1) return w;
    const int xcd = w % X, idx = w / X, per = G / X, rem = G % X;
    return xcd * per + (xcd < rem ? xcd : rem) + idx;
}

// ------------------------------------------------------------------------------------
// Operand loaders: global -> registers (load) and registers -> LDS planes (store).
// R rows of the tile, NT threads; a stage covers KPS elements of K.
// ------------------------------------------------------------------------------------
// Loads are issued unconditionally (an invalid chunk reads element 0 of the operand,
// which always exists) and zeroed when they reach LDS: no branch sits between a load and
// the instructions that follow it, so the compiler keeps several stages in flight.
__device__ __forceinline__ i32x4 keep(i32x4 v, unsigned ok, int i)
{
    const bool on = (ok >> i) & 1u;
    return i32x4{on ? v[0] : 0, on ? v[1] : 0, on ? v[2] : 0, on ? v[3] : 0};
}

template <Fmt F, int R, int NT> struct Loader;

template <int R, int NT> struct Loader<Fmt::I8, R, NT> {
    static constexpr int PLANES = 1, KPS = 128, NCH = R * 8, CH = (NCH + NT - 1) / NT, BYTES = R * 128;
    i32x4 r[CH];
    unsigned ok;
    __device__ __forceinline__ void load(const char *base, long ld, int row0, int rows,
                                         int k0, int kend, int tid)
    {
        ok = 0;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT, row = q >> 3, c = q & 7;
            const int gr = row0 + row, kk = k0 + c * 16;
            const bool v = (NCH % NT == 0 || q < NCH) && gr < rows && kk < kend;
            r[i] = *reinterpret_cast<const i32x4 *>(base + (v ? (long)gr * ld + kk : 0L));
            ok |= (unsigned)v << i;
        }
    }
    __device__ __forceinline__ void store(char *lds, int pstride, int tid) const
    {
        (void)pstride;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT;
            if (NCH % NT == 0 || q < NCH)
                *reinterpret_cast<i32x4 *>(lds + swz(q >> 3, q & 7)) = keep(r[i], ok, i);
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
    static constexpr int PLANES = 1, KPS = 128, NCH = R * 4, CH = (NCH + NT - 1) / NT, BYTES = R * 64;
    i32x4 r[CH];
    unsigned ok;
    __device__ __forceinline__ void load(const char *base, long ld, int row0, int rows,
                                         int k0, int kend, int tid)
    {
        ok = 0;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT, row = q >> 2, pc = q & 3;
            const int gr = row0 + row, kk = k0 + pc * 32;
            const bool v = (NCH % NT == 0 || q < NCH) && gr < rows && kk < kend;
            r[i] = *reinterpret_cast<const i32x4 *>(base + (v ? (long)gr * ld + (kk >> 1) : 0L));
            ok |= (unsigned)v << i;
        }
    }
    __device__ __forceinline__ void store(char *lds, int pstride, int tid) const
    {
        (void)pstride;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT, row = q >> 2, pc = q & 3;
            if (NCH % NT == 0 || q < NCH) {
                const i32x4 w = keep(r[i], ok, i);
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
// two int16 in w -> (lo bytes, hi bytes) of the CLAMPED values as 16-bit halves
__device__ __forceinline__ void split2(int w, unsigned &lo2, unsigned &hi2)
{
    int x0 = (int)(short)(w & 0xFFFF), x1 = w >> 16;
    x0 = x0 > 32639 ? 32639 : x0;
    x1 = x1 > 32639 ? 32639 : x1;
    lo2 = ((unsigned)x0 & 0xFFu) | (((unsigned)x1 & 0xFFu) << 8);
    hi2 = ((unsigned)((x0 + 128) >> 8) & 0xFFu) | (((unsigned)((x1 + 128) >> 8) & 0xFFu) << 8);
}

template <int R, int NT> struct Loader<Fmt::I16, R, NT> {
    static constexpr int PLANES = 2, KPS = 128, NCH = R * 8, CH = (NCH + NT - 1) / NT, BYTES = R * 256;
    i32x4 r[CH][2];
    unsigned ok;
    __device__ __forceinline__ void load(const char *base, long ld, int row0, int rows,
                                         int k0, int kend, int tid)
    {
        ok = 0;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT, row = q >> 3, c = q & 7;
            const int gr = row0 + row, kk = k0 + c * 16;
            const bool v = (NCH % NT == 0 || q < NCH) && gr < rows && kk < kend;
            const i32x4 *p = reinterpret_cast<const i32x4 *>(base + (v ? (long)gr * ld + 2L * kk : 0L));
            r[i][0] = p[0];
            r[i][1] = p[1];
            ok |= (unsigned)v << i;
        }
    }
    __device__ __forceinline__ void store(char *lds, int pstride, int tid) const
    {
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT;
            if (NCH % NT == 0 || q < NCH) {
                unsigned lo[8], hi[8];
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const i32x4 x = keep(r[i][h], ok, i);
#pragma unroll
                    for (int e = 0; e < 4; e++) split2(x[e], lo[h * 4 + e], hi[h * 4 + e]);
                }
                i32x4 vl, vh;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    vl[e] = (int)(lo[2 * e] | (lo[2 * e + 1] << 16));
                    vh[e] = (int)(hi[2 * e] | (hi[2 * e + 1] << 16));
                }
                const int off = swz(q >> 3, q & 7);
                *reinterpret_cast<i32x4 *>(lds + off) = vh;             // plane 0: hi
                *reinterpret_cast<i32x4 *>(lds + pstride + off) = vl;   // plane 1: lo
            }
        }
    }
};

template <int R, int NT> struct Loader<Fmt::F16, R, NT> {
    static constexpr int PLANES = 1, KPS = 64, NCH = R * 8, CH = (NCH + NT - 1) / NT, BYTES = R * 128;
    i32x4 r[CH];
    unsigned ok;
    __device__ __forceinline__ void load(const char *base, long ld, int row0, int rows,
                                         int k0, int kend, int tid)
    {
        ok = 0;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT, row = q >> 3, c = q & 7;
            const int gr = row0 + row, kk = k0 + c * 8;
            const bool v = (NCH % NT == 0 || q < NCH) && gr < rows && kk < kend;
            r[i] = *reinterpret_cast<const i32x4 *>(base + (v ? (long)gr * ld + 2L * kk : 0L));
            ok |= (unsigned)v << i;
        }
    }
    __device__ __forceinline__ void store(char *lds, int pstride, int tid) const
    {
        (void)pstride;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT;
            if (NCH % NT == 0 || q < NCH)
                *reinterpret_cast<i32x4 *>(lds + swz(q >> 3, q & 7)) = keep(r[i], ok, i);
        }
    }
};

// fp32 -> bf16 by truncation: the high halves of two fp32 words packed into one word.
__device__ __forceinline__ int bf16pack(int f0, int f1)
{
    return (int)(((unsigned)f0 >> 16) | ((unsigned)f1 & 0xFFFF0000u));
}

template <int R, int NT> struct Loader<Fmt::F32BF16, R, NT> {
    static constexpr int PLANES = 1, KPS = 64, NCH = R * 8, CH = (NCH + NT - 1) / NT, BYTES = R * 256;
    i32x4 r[CH][2];
    unsigned ok;
    __device__ __forceinline__ void load(const char *base, long ld, int row0, int rows,
                                         int k0, int kend, int tid)
    {
        ok = 0;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT, row = q >> 3, c = q & 7;
            const int gr = row0 + row, kk = k0 + c * 8;
            const bool v = (NCH % NT == 0 || q < NCH) && gr < rows && kk < kend;
            const i32x4 *p = reinterpret_cast<const i32x4 *>(base + (v ? (long)gr * ld + 4L * kk : 0L));
            r[i][0] = p[0];
            r[i][1] = p[1];
            ok |= (unsigned)v << i;
        }
    }
    __device__ __forceinline__ void store(char *lds, int pstride, int tid) const
    {
        (void)pstride;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT;
            if (NCH % NT == 0 || q < NCH) {
                const i32x4 a = keep(r[i][0], ok, i), b = keep(r[i][1], ok, i);
                *reinterpret_cast<i32x4 *>(lds + swz(q >> 3, q & 7)) =
                    i32x4{bf16pack(a[0], a[1]), bf16pack(a[2], a[3]),
                          bf16pack(b[0], b[1]), bf16pack(b[2], b[3])};
            }
        }
    }
};

// fp32 -> tf32 (13 low mantissa bits cleared) -> hi = its bf16 truncation, lo = t - hi.
// lo carries the remaining 3 significant bits, so it is exact in bf16 as well.
__device__ __forceinline__ void tf32split(int f, unsigned &hi16, unsigned &lo16)
{
    const unsigned t = (unsigned)f & 0xFFFFE000u, h = t & 0xFFFF0000u;
    const float lo = __uint_as_float(t) - __uint_as_float(h);
    hi16 = h >> 16;
    lo16 = __float_as_uint(lo) >> 16;
}

template <int R, int NT> struct Loader<Fmt::F32TF32, R, NT> {
    static constexpr int PLANES = 2, KPS = 64, NCH = R * 8, CH = (NCH + NT - 1) / NT, BYTES = R * 256;
    i32x4 r[CH][2];
    unsigned ok;
    __device__ __forceinline__ void load(const char *base, long ld, int row0, int rows,
                                         int k0, int kend, int tid)
    {
        ok = 0;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT, row = q >> 3, c = q & 7;
            const int gr = row0 + row, kk = k0 + c * 8;
            const bool v = (NCH % NT == 0 || q < NCH) && gr < rows && kk < kend;
            const i32x4 *p = reinterpret_cast<const i32x4 *>(base + (v ? (long)gr * ld + 4L * kk : 0L));
            r[i][0] = p[0];
            r[i][1] = p[1];
            ok |= (unsigned)v << i;
        }
    }
    __device__ __forceinline__ void store(char *lds, int pstride, int tid) const
    {
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT;
            if (NCH % NT == 0 || q < NCH) {
                unsigned h[8], l[8];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    tf32split(keep(r[i][0], ok, i)[e], h[e], l[e]);
                    tf32split(keep(r[i][1], ok, i)[e], h[4 + e], l[4 + e]);
                }
                i32x4 vh, vl;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    vh[e] = (int)(h[2 * e] | (h[2 * e + 1] << 16));
                    vl[e] = (int)(l[2 * e] | (l[2 * e + 1] << 16));
                }
                const int off = swz(q >> 3, q & 7);
                *reinterpret_cast<i32x4 *>(lds + off) = vh;
                *reinterpret_cast<i32x4 *>(lds + pstride + off) = vl;
            }
        }
    }
};

// ------------------------------------------------------------------------------------
// MFMA math (32x32 shapes: the 16x16 ones issue at half rate on gfx950). A substep
// consumes KSB = 32 LDS bytes per row; lane l supplies row l % 32 and the 16 bytes
// [16*(l/32), +16) of the substep, identically for both operands. KEL = K elements per
// substep.
// ------------------------------------------------------------------------------------
__device__ __forceinline__ i32x4 lds_frag(const char *plane, int row, int sub, int lane)
{
    return *reinterpret_cast<const i32x4 *>(plane + swz(row, 2 * sub + (lane >> 5)));
}

struct MathI8 {            // v_mfma_i32_32x32x32_i8
    using Acc = i32x16;
    static constexpr int NACC = 1, PA = 1, PB = 1, KSB = 32, KEL = 32;
    __device__ static void mma(Acc *acc, const i32x4 *a, const i32x4 *b)
    {
        acc[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b[0], a[0], acc[0], 0, 0, 0);
    }
};

struct MathI16 {           // byte planes: acc0 = hi*hi, acc1 = hi*lo + lo*hi, acc2 = lo*lo
    using Acc = i32x16;
    static constexpr int NACC = 3, PA = 2, PB = 2, KSB = 32, KEL = 32;
    __device__ static void mma(Acc *acc, const i32x4 *a, const i32x4 *b)
    {
        acc[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b[0], a[0], acc[0], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b[0], a[1], acc[1], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b[1], a[0], acc[1], 0, 0, 0);
        acc[2] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b[1], a[1], acc[2], 0, 0, 0);
    }
};

struct MathF16 {           // v_mfma_f32_32x32x16_f16
    using Acc = f32x16;
    static constexpr int NACC = 1, PA = 1, PB = 1, KSB = 32, KEL = 16;
    __device__ static void mma(Acc *acc, const i32x4 *a, const i32x4 *b)
    {
        acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, b[0]),
                                                        __builtin_bit_cast(f16x8, a[0]), acc[0], 0, 0, 0);
    }
};

struct MathBF16 {          // v_mfma_f32_32x32x16_bf16
    using Acc = f32x16;
    static constexpr int NACC = 1, PA = 1, PB = 1, KSB = 32, KEL = 16;
    __device__ static void mma(Acc *acc, const i32x4 *a, const i32x4 *b)
    {
        acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, b[0]),
                                                         __builtin_bit_cast(bf16x8, a[0]), acc[0], 0, 0, 0);
    }
};

struct MathTF32 {          // bf16 hi/lo planes: hi*hi + lo*hi + hi*lo (lo*lo dropped)
    using Acc = f32x16;
    static constexpr int NACC = 1, PA = 2, PB = 2, KSB = 32, KEL = 16;
    __device__ static void mma(Acc *acc, const i32x4 *a, const i32x4 *b)
    {
        const bf16x8 ah = __builtin_bit_cast(bf16x8, a[0]), al = __builtin_bit_cast(bf16x8, a[1]);
        const bf16x8 bh = __builtin_bit_cast(bf16x8, b[0]), bl = __builtin_bit_cast(bf16x8, b[1]);
        acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bh, ah, acc[0], 0, 0, 0);
        acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bl, ah, acc[0], 0, 0, 0);
        acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bh, al, acc[0], 0, 0, 0);
    }
};

// ------------------------------------------------------------------------------------
// Group-wise scale slots: every stage carries the scales of the (at most NGS) quant
// groups that intersect its K range, staged through LDS with the operand tiles.
// ------------------------------------------------------------------------------------
constexpr int NGS = 4;   // a 128-element stage meets at most 4 groups of >= 32

template <int BM, int BN, bool ROWSCALE, bool B_I4, int NT> struct ScaleLoader {
    static constexpr int NA = ROWSCALE ? 0 : (NGS * BM + NT - 1) / NT;
    static constexpr int NB = (NGS * BN + NT - 1) / NT;
    float ra[NA > 0 ? NA : 1], rb[NB];
    unsigned oka, okb;
    __device__ __forceinline__ void load(const KArgs &args, const Problem &P, int m0, int M, int n0, int N,
                                         int k0, int tid)
    {
        const int g0 = k0 / args.group, nG = args.nG;
        oka = okb = 0;
#pragma unroll
        for (int i = 0; i < NA; i++) {
            const int q = tid + i * NT, slot = q / BM, r = q % BM, g = g0 + slot, m = m0 + r;
            const bool v = q < NGS * BM && m < M && g < nG;
            ra[i] = P.a_scale[v ? (long)m * nG + g : 0L];
            oka |= (unsigned)v << i;
        }
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const int q = tid + i * NT, slot = q / BN, c = q % BN, g = g0 + slot, n = n0 + c;
            const bool v = q < NGS * BN && n < N && g < nG;
            rb[i] = P.b_scale[v ? (long)n * nG + g : 0L];
            okb |= (unsigned)v << i;
        }
    }
    // layout in LDS: b-scales [NGS][BN] then a-scales [NGS][BM]
    __device__ __forceinline__ void store(float *sc, int tid) const
    {
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const int q = tid + i * NT;
            // 1/16 is exact: it removes the x16 that unpacked int4 weights carry
            if (q < NGS * BN) sc[q] = ((okb >> i) & 1u) ? (B_I4 ? rb[i] * 0.0625f : rb[i]) : 0.f;
        }
#pragma unroll
        for (int i = 0; i < NA; i++) {
            const int q = tid + i * NT;
            if (q < NGS * BM) sc[NGS * BN + q] = ((oka >> i) & 1u) ? ra[i] : 0.f;
        }
    }
};

// Workgroup barrier that orders LDS only. __syncthreads() is a workgroup release fence,
// which on gfx9 also waits for every outstanding global load (vmcnt(0)) and so would
// drain the prefetch pipeline at each stage.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Group-wise epilogue at the end of quant group g: fold the int32 partials of every
// block into the fp32 accumulators (fmaf(a*b, P, acc), or fmaf(b, P, acc) with per-row
// activation scales applied at the end), optionally dump them, and clear them.
template <int TM, int TN, int BM, int BN, int WTN, bool ROWSCALE, bool B_I4, bool DUMP>
__device__ __forceinline__ void gw_epilogue(const KArgs &args, i32x16 (&acc)[TM][TN][1], f32x16 (&accf)[TM][TN],
                                            const float *sc, int g, int g_first, int rowA, int wn, int lane,
                                            int m0, int n0, int M, int N, int p)
{
    const int slot = g - g_first, nG = args.nG;
    float sa[TM];
#pragma unroll
    for (int i = 0; i < TM; i++) sa[i] = ROWSCALE ? 1.f : sc[NGS * BN + slot * BM + rowA + 32 * i];
#pragma unroll
    for (int j = 0; j < TN; j++) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const f32x4 sb = *reinterpret_cast<const f32x4 *>(sc + slot * BN + wn * WTN + 32 * j + 8 * q + 4 * (lane >> 5));
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float s = ROWSCALE ? sb[r] : sa[i] * sb[r];
                    accf[i][j][4 * q + r] = __builtin_fmaf(s, (float)acc[i][j][0][4 * q + r], accf[i][j][4 * q + r]);
                }
        }
    }
    if (DUMP && p == 0 && args.kt == args.group) {
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int m = m0 + 32 * i;
            if (m < args.dump_row0 || m >= args.dump_row0 + args.dump_rows || m >= M) continue;
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int n = n0 + 32 * j + 8 * q;
                    if (n >= N) continue;
                    i32x4 v = {acc[i][j][0][4 * q], acc[i][j][0][4 * q + 1], acc[i][j][0][4 * q + 2], acc[i][j][0][4 * q + 3]};
                    if (B_I4) v = v >> 4;
                    *reinterpret_cast<i32x4 *>(args.dump + ((long)(m - args.dump_row0) * nG + g) * N + n) = v;
                }
        }
    }
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j][0] = i32x16{};
}

// ------------------------------------------------------------------------------------
// The kernel. BM x BN tile, 4 waves as 2 x 2, each wave (BM/2) x (BN/2) of 32x32 MFMA
// blocks. Dynamic LDS: 2 stages x (operand planes [+ scale slots]).
// ------------------------------------------------------------------------------------
template <int BM, int BN, Fmt FA, Fmt FB, class MATH, Epi EPI, bool ROWSCALE>
struct KCfg {
    static constexpr int NT = 256, WGM = 2, WGN = 2;
    static constexpr int WTM = BM / WGM, WTN = BN / WGN, TM = WTM / 32, TN = WTN / 32;
    static constexpr int PLA = BM * ROWB, PLB = BN * ROWB;
    static constexpr bool GW = (EPI == Epi::GW);
    static constexpr int SCB = GW ? NGS * (BN + (ROWSCALE ? 0 : BM)) * 4 : 0;
    static constexpr int STAGE = MATH::PA * PLA + MATH::PB * PLB + SCB;
    static constexpr int LDS = 2 * STAGE;
    // prefetch depth: as many in-flight stages as fit in ~128 VGPRs of staging registers
    static constexpr int REGS = (Loader<FA, BM, NT>::BYTES + Loader<FB, BN, NT>::BYTES) / (4 * NT);
    static constexpr int D = REGS <= 32 ? 4 : (REGS <= 48 ? 3 : (REGS <= 64 ? 2 : 1));
};

template <int BM, int BN, Fmt FA, Fmt FB, class MATH, Epi EPI, bool ROWSCALE, bool DUMP>
__global__ __launch_bounds__(256) void k_gemm(const KArgs args)
{
    using CF = KCfg<BM, BN, FA, FB, MATH, EPI, ROWSCALE>;
    constexpr int NT = CF::NT, WGN = CF::WGN, WTM = CF::WTM, WTN = CF::WTN, TM = CF::TM, TN = CF::TN;
    constexpr int PLA = CF::PLA, PLB = CF::PLB, STAGE = CF::STAGE;
    constexpr bool GW = CF::GW;
    using LA = Loader<FA, BM, NT>;
    using LB = Loader<FB, BN, NT>;
    static_assert(LA::KPS == LB::KPS, "operand stage K mismatch");
    static_assert(LA::KPS == MATH::KEL * (ROWB / MATH::KSB), "stage K vs MFMA substeps");
    static_assert(LA::PLANES == MATH::PA && LB::PLANES == MATH::PB, "plane count");
    static_assert(TM >= 1 && TN >= 1, "wave tile below one MFMA block");
    constexpr int KPS = LA::KPS, NSUB = ROWB / MATH::KSB;
    constexpr bool B_I4 = (FB == Fmt::I4P);
    constexpr int OFFSC = MATH::PA * PLA + MATH::PB * PLB;   // scale slots within a stage

    extern __shared__ __attribute__((aligned(16))) char smem[];

    // ---- which problem / tile ----
    int tile = xcd_remap((int)blockIdx.x, (int)gridDim.x, args.xcds);
    int p = 0;
#pragma unroll 1
    while (p + 1 < args.nprob && tile >= args.tile_start[p + 1]) p++;
    tile -= args.tile_start[p];
    const Problem &P = args.prob[p];
    const int M = P.M, N = args.N;
    const int nbm = (M + BM - 1) / BM;
    const int bm = tile % nbm, bn = tile / nbm;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    const int rowA = wm * WTM + (lane & 31);   // A-tile row of block i: rowA + 32 i
    const int rowB = wn * WTN + (lane & 31);   // B-tile row of block j: rowB + 32 j

    typename MATH::Acc acc[TM][TN][MATH::NACC];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int a = 0; a < MATH::NACC; a++) acc[i][j][a] = typename MATH::Acc{};

    constexpr int TMG = GW ? TM : 1, TNG = GW ? TN : 1;
    f32x16 accf[TMG][TNG];
#pragma unroll
    for (int i = 0; i < TMG; i++)
#pragma unroll
        for (int j = 0; j < TNG; j++) accf[i][j] = f32x16{};

    // output coordinates of this lane: row m0 + 32 i, columns n0 + 32 j + 8 q + {0..3}
    const int m0 = bm * BM + rowA;
    const int n0 = bn * BN + wn * WTN + 4 * (lane >> 5);

    const char *Ab = static_cast<const char *>(P.A);
    const char *Bb = static_cast<const char *>(P.B);
    const int kbeg = args.kbeg, kend = args.kend;

    // D register sets keep loads for D stages in flight; the LDS holds two stages. Stage t
    // lives in set t % D from its load until it is written to LDS slot t % 2 at the end of
    // iteration t - 1; the K loop is unrolled by D so every set index is a constant.
    constexpr int D = CF::D;
    LA la[D];
    LB lb[D];
    ScaleLoader<BM, BN, ROWSCALE, B_I4, NT> ls[D];
    const int nst = (kend - kbeg + KPS - 1) / KPS;
#pragma unroll
    for (int u = 0; u < D; u++) {
        la[u].load(Ab, args.lda, bm * BM, M, kbeg + u * KPS, kend, tid);
        lb[u].load(Bb, args.ldb, bn * BN, N, kbeg + u * KPS, kend, tid);
        if constexpr (GW) ls[u].load(args, P, bm * BM, M, bn * BN, N, kbeg + u * KPS, tid);
    }
    la[0].store(smem, PLA, tid);
    lb[0].store(smem + MATH::PA * PLA, PLB, tid);
    if constexpr (GW) ls[0].store(reinterpret_cast<float *>(smem + OFFSC), tid);
    lds_barrier();

    // The steady state has no branch around a memory access: the loop runs whole groups
    // of D stages, and stages past kend load zero-masked data that adds nothing.
#pragma unroll 1
    for (int s0 = 0; s0 < nst; s0 += D) {
#pragma unroll
        for (int u = 0; u < D; u++) {
            const int s = s0 + u;
            const char *cur = smem + (s & 1) * STAGE;
            const int k0 = kbeg + s * KPS;
            // set u is free: its stage went to LDS at the end of the previous iteration
            la[u].load(Ab, args.lda, bm * BM, M, k0 + D * KPS, kend, tid);
            lb[u].load(Bb, args.ldb, bn * BN, N, k0 + D * KPS, kend, tid);
            if constexpr (GW) ls[u].load(args, P, bm * BM, M, bn * BN, N, k0 + D * KPS, tid);
#pragma unroll
            for (int ss = 0; ss < NSUB; ss++) {
                i32x4 fa[TM][MATH::PA], fb[TN][MATH::PB];
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int pl = 0; pl < MATH::PA; pl++)
                        fa[i][pl] = lds_frag(cur + pl * PLA, rowA + 32 * i, ss, lane);
#pragma unroll
                for (int j = 0; j < TN; j++)
#pragma unroll
                    for (int pl = 0; pl < MATH::PB; pl++)
                        fb[j][pl] = lds_frag(cur + MATH::PA * PLA + pl * PLB, rowB + 32 * j, ss, lane);
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++) MATH::mma(acc[i][j], fa[i], fb[j]);

                if constexpr (GW) {
                    const int kpos = k0 + (ss + 1) * MATH::KEL;   // K consumed so far
                    if (kpos <= kend && (kpos % args.kt) == 0)
                        gw_epilogue<TM, TN, BM, BN, WTN, ROWSCALE, B_I4, DUMP>(
                            args, acc, accf, reinterpret_cast<const float *>(cur + OFFSC),
                            (kpos - 1) / args.group, k0 / args.group, rowA, wn, lane, m0, n0, M, N, p);
                }
            }
            {
                char *nxt = smem + ((s + 1) & 1) * STAGE;
                const int v = (u + 1) % D;
                la[v].store(nxt, PLA, tid);
                lb[v].store(nxt + MATH::PA * PLA, PLB, tid);
                if constexpr (GW) ls[v].store(reinterpret_cast<float *>(nxt + OFFSC), tid);
            }
            lds_barrier();
        }
    }

    // ---- epilogue: lane holds rows m0 + 32 i, four runs of four columns per block ----
#pragma unroll
    for (int i = 0; i < TM; i++) {
        const int m = m0 + 32 * i;
        if (m >= M) continue;
        const float rs = (GW && ROWSCALE) ? P.a_scale[m] : 1.f;
#pragma unroll
        for (int j = 0; j < TN; j++) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int n = n0 + 32 * j + 8 * q;
                if (n >= N) continue;
                const long off = (long)m * N + n;
                if constexpr (EPI == Epi::I32) {
                    i32x4 v = {acc[i][j][0][4 * q], acc[i][j][0][4 * q + 1], acc[i][j][0][4 * q + 2],
                               acc[i][j][0][4 * q + 3]};
                    if (B_I4) v = v >> 4;
                    i32x4 *c = reinterpret_cast<i32x4 *>(static_cast<int32_t *>(P.C) + off);
                    if (args.accum) v += *c;
                    *c = v;
                } else if constexpr (EPI == Epi::I64) {
                    i64 *c = static_cast<i64 *>(P.C) + off;
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        i64 v = (i64)acc[i][j][0][4 * q + r] * 65536 + (i64)acc[i][j][1][4 * q + r] * 256 +
                                (i64)acc[i][j][2][4 * q + r];
                        if (args.accum) v += c[r];
                        c[r] = v;
                    }
                } else if constexpr (EPI == Epi::F16) {
                    f16x4 h = {(_Float16)acc[i][j][0][4 * q], (_Float16)acc[i][j][0][4 * q + 1],
                               (_Float16)acc[i][j][0][4 * q + 2], (_Float16)acc[i][j][0][4 * q + 3]};
                    *reinterpret_cast<f16x4 *>(static_cast<_Float16 *>(P.C) + off) = h;
                } else if constexpr (EPI == Epi::F32) {
                    *reinterpret_cast<f32x4 *>(static_cast<float *>(P.C) + off) =
                        f32x4{acc[i][j][0][4 * q], acc[i][j][0][4 * q + 1], acc[i][j][0][4 * q + 2],
                              acc[i][j][0][4 * q + 3]};
                } else {   // GW
                    const f32x16 &v = accf[i < TMG ? i : 0][j < TNG ? j : 0];
                    *reinterpret_cast<f32x4 *>(static_cast<float *>(P.C) + off) =
                        f32x4{v[4 * q] * rs, v[4 * q + 1] * rs, v[4 * q + 2] * rs, v[4 * q + 3] * rs};
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------------
// int4 packing: one thread per packed dword (8 values of K).
// ------------------------------------------------------------------------------------
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

// ------------------------------------------------------------------------------------
// Dispatch.
// ------------------------------------------------------------------------------------
template <int BM, int BN, Fmt FA, Fmt FB, class MATH, Epi EPI, bool RS, bool DUMP = false>
hipError_t launch_one(const KArgs &ka, int tiles, hipStream_t s)
{
    constexpr int lds = KCfg<BM, BN, FA, FB, MATH, EPI, RS>::LDS;
    static_assert(lds <= 160 * 1024, "LDS budget");
    auto kern = k_gemm<BM, BN, FA, FB, MATH, EPI, RS, DUMP>;
    static bool opted = false;          // dynamic LDS above 64 KiB needs an opt-in, once
    if (!opted) {
        if (hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                lds) != hipSuccess)
            return hipGetLastError();
        opted = true;
    }
    hipLaunchKernelGGL(kern, dim3(tiles), dim3(256), lds, s, ka);
    return hipGetLastError();
}

}  // namespace

void gemm_tile(Fmt fmt_a, Epi epi, int M, int N, int *bm, int *bn)
{
    // The largest tile that still yields about one workgroup per CU; a CU needs roughly
    // 64 operand bytes of MFMA work per L2 byte, which 256 x 128 gives and 64 x 64 does not.
    const long cus = 256;
    auto tiles = [&](int tm, int tn) { return (long)((M + tm - 1) / tm) * ((N + tn - 1) / tn); };
    // group-wise keeps an int32 and an fp32 accumulator set: at most 128 x 128 per workgroup
    const bool two_plane = (fmt_a == Fmt::I16 || fmt_a == Fmt::F32TF32);
    if (!two_plane && epi != Epi::GW && tiles(256, 128) >= cus * 15 / 16) { *bm = 256; *bn = 128; return; }
    if (fmt_a != Fmt::I16 && tiles(128, 128) >= cus * 15 / 16) { *bm = 128; *bn = 128; return; }
    if (tiles(128, 64) >= cus / 2) { *bm = 128; *bn = 64; return; }
    *bm = 64; *bn = 64;
}

template <int BM, int BN>
static hipError_t dispatch_tile(const Launch &L, const KArgs &ka, int tiles)
{
    hipStream_t s = L.stream;
    const bool rs = L.rowscale;
    if (L.fmt_a == Fmt::I8 && L.fmt_b == Fmt::I8) {
        if (L.epi == Epi::I32) return launch_one<BM, BN, Fmt::I8, Fmt::I8, MathI8, Epi::I32, false>(ka, tiles, s);
        if constexpr (BM <= 128)
            if (L.epi == Epi::GW) {
                if (L.dump) return launch_one<BM, BN, Fmt::I8, Fmt::I8, MathI8, Epi::GW, false, true>(ka, tiles, s);
                return rs ? launch_one<BM, BN, Fmt::I8, Fmt::I8, MathI8, Epi::GW, true>(ka, tiles, s)
                          : launch_one<BM, BN, Fmt::I8, Fmt::I8, MathI8, Epi::GW, false>(ka, tiles, s);
            }
    }
    if (L.fmt_a == Fmt::I8 && L.fmt_b == Fmt::I4P) {
        if (L.epi == Epi::I32) return launch_one<BM, BN, Fmt::I8, Fmt::I4P, MathI8, Epi::I32, false>(ka, tiles, s);
        if constexpr (BM <= 128)
            if (L.epi == Epi::GW) {
                if (L.dump) return launch_one<BM, BN, Fmt::I8, Fmt::I4P, MathI8, Epi::GW, false, true>(ka, tiles, s);
                return rs ? launch_one<BM, BN, Fmt::I8, Fmt::I4P, MathI8, Epi::GW, true>(ka, tiles, s)
                          : launch_one<BM, BN, Fmt::I8, Fmt::I4P, MathI8, Epi::GW, false>(ka, tiles, s);
            }
    }
    if (L.fmt_a == Fmt::F16 && L.fmt_b == Fmt::F16) {
        if (L.epi == Epi::F16) return launch_one<BM, BN, Fmt::F16, Fmt::F16, MathF16, Epi::F16, false>(ka, tiles, s);
        if (L.epi == Epi::F32) return launch_one<BM, BN, Fmt::F16, Fmt::F16, MathF16, Epi::F32, false>(ka, tiles, s);
    }
    if (L.fmt_a == Fmt::F32BF16 && L.fmt_b == Fmt::F32BF16 && L.epi == Epi::F32)
        return launch_one<BM, BN, Fmt::F32BF16, Fmt::F32BF16, MathBF16, Epi::F32, false>(ka, tiles, s);
    if constexpr (BM <= 128) {   // two-plane operands: 2 x 2 planes per stage
        if (L.fmt_a == Fmt::I16 && L.fmt_b == Fmt::I16 && L.epi == Epi::I64)
            return launch_one<BM, BN, Fmt::I16, Fmt::I16, MathI16, Epi::I64, false>(ka, tiles, s);
        if (L.fmt_a == Fmt::F32TF32 && L.fmt_b == Fmt::F32TF32 && L.epi == Epi::F32)
            return launch_one<BM, BN, Fmt::F32TF32, Fmt::F32TF32, MathTF32, Epi::F32, false>(ka, tiles, s);
    }
    return hipErrorInvalidValue;
}

// Workgroups are renumbered over this many XCDs (MI355X has 8); ROCKET_HIP_XCD overrides,
// 1 keeps the hardware order.
static int xcd_count()
{
    static int n = -1;
    if (n < 0) {
        const char *e = getenv("ROCKET_HIP_XCD");
        n = e ? atoi(e) : 8;
        if (n < 1 || n > 64) n = 8;
    }
    return n;
}

static long row_bytes(Fmt f, int K)
{
    switch (f) {
    case Fmt::I8: return K;
    case Fmt::I4P: return K / 2;
    case Fmt::I16: case Fmt::F16: return 2L * K;
    case Fmt::F32BF16: case Fmt::F32TF32: return 4L * K;
    }
    return 0;
}

static bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

hipError_t gemm_launch(const Launch &L, uint64_t *blocks_out)
{
    if (blocks_out) *blocks_out = 0;
    // what the kernels assume: K in whole 32-element chunks, N in whole 16-column blocks,
    // 16-byte aligned operand rows, a valid K range and problem count
    if (L.nprob < 1 || L.nprob > kMaxProblems || L.N <= 0 || L.K <= 0) return hipErrorInvalidValue;
    if (L.K % 32 != 0 && !(L.K % 16 == 0 && L.fmt_a == Fmt::F32TF32)) return hipErrorInvalidValue;
    if (L.N % 16 != 0) return hipErrorInvalidValue;
    if (L.kbeg < 0 || L.kend > L.K || L.kbeg >= L.kend || L.kbeg % 128 != 0) return hipErrorInvalidValue;
    if (L.fmt_b == Fmt::I4P && (L.K % 32 != 0)) return hipErrorInvalidValue;
    if (L.epi == Epi::GW) {
        if (L.group < 32 || L.group % 32 || L.K % L.group || L.kt < 32 || L.kt % 32 || L.group % L.kt)
            return hipErrorInvalidValue;
        if (L.kbeg != 0 || L.kend != L.K || L.accum) return hipErrorInvalidValue;
        if (L.dump && L.rowscale) return hipErrorInvalidValue;
    } else if (L.rowscale || L.dump) {
        return hipErrorInvalidValue;
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
        maxM = std::max(maxM, P.M);
    }
    if (maxM == 0) return hipSuccess;

    int bm, bn;
    gemm_tile(L.fmt_a, L.epi, maxM, L.N, &bm, &bn);

    KArgs ka;
    ka.N = L.N; ka.K = L.K; ka.kbeg = L.kbeg; ka.kend = L.kend; ka.accum = L.accum;
    ka.group = L.group; ka.kt = L.kt; ka.nG = L.group ? L.K / L.group : 0;
    ka.lda = lda; ka.ldb = ldb;
    ka.nprob = L.nprob;
    ka.dump = L.dump; ka.dump_row0 = L.dump_row0; ka.dump_rows = L.dump_rows;
    ka.xcds = xcd_count();
    const int nbn = (L.N + bn - 1) / bn;
    long tiles = 0;
    for (int i = 0; i < L.nprob; i++) {
        ka.prob[i] = L.prob[i];
        ka.tile_start[i] = (int)tiles;
        tiles += (long)((L.prob[i].M + bm - 1) / bm) * nbn;
    }
    ka.tile_start[L.nprob] = (int)tiles;
    if (tiles > 0x7FFFFFFFL) return hipErrorInvalidValue;
    if (blocks_out) *blocks_out = (uint64_t)tiles;

    if (bm == 256) return dispatch_tile<256, 128>(L, ka, (int)tiles);
    if (bm == 128 && bn == 128) return dispatch_tile<128, 128>(L, ka, (int)tiles);
    if (bm == 128) return dispatch_tile<128, 64>(L, ka, (int)tiles);
    return dispatch_tile<64, 64>(L, ka, (int)tiles);
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

}  // namespace rk
