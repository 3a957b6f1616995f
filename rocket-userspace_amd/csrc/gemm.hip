// gemm.hip — gfx950 MFMA GEMM kernels for every matmul entry of the library.
//
// C[M,N] = A[M,K] * B[N,K]^T with both operands K-contiguous. One workgroup owns a
// BM x BN output tile; its 4 waves (2 x 2) own (BM/2) x (BN/2) sub-tiles built from
// 16x16 MFMA blocks. K advances in stages of 128 LDS bytes per tile row; each stage is
// staged global -> registers -> LDS (double-buffered, one barrier per stage) while the
// previous stage feeds the MFMAs.
//
// LDS tile row layout: 128 bytes = eight 16-byte chunks, chunk c of row r stored at slot
// c ^ (r & 7), so the eight lanes a ds_read_b128 serves together (eight consecutive rows,
// one chunk) hit eight different bank groups.
//
// MFMA operand convention: the B fragment is the instruction's first (row) operand and
// the A fragment its second, so the 16x16 result lands with lane l holding row
// m = l % 16 and the four consecutive columns n = 4*(l/16) .. +3, i.e. one 16-byte
// vector store per lane per block. Lane l supplies row l % 16 of each fragment and the
// K bytes [16*(l/16), +16) of the 64-byte substep, identically for both operands.
#include "gemm.h"

#include <algorithm>
#include <type_traits>

namespace rk {
namespace {

typedef int      i32x4  __attribute__((ext_vector_type(4)));
typedef int      i32x2  __attribute__((ext_vector_type(2)));
typedef float    f32x4  __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8  __attribute__((ext_vector_type(8)));
typedef __bf16   bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4  __attribute__((ext_vector_type(4)));
typedef long long i64;

constexpr int ROWB = 128;   // LDS bytes per tile row per plane per stage

__device__ __forceinline__ int swz(int row, int chunk) { return row * ROWB + ((chunk ^ (row & 7)) << 4); }

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
};

// Workgroup w is dispatched to XCD w % 8. Renumber so the workgroups of one XCD get
// consecutive logical ids, then walk M fastest: an XCD's tiles share B column blocks,
// which its own L2 then serves.
__device__ __forceinline__ int xcd_remap(int w, int G)
{
    const int xcd = w & 7, idx = w >> 3, per = G >> 3, rem = G & 7;
    return xcd * per + (xcd < rem ? xcd : rem) + idx;
}

// ------------------------------------------------------------------------------------
// Operand loaders: global -> registers (load) and registers -> LDS planes (store).
// R rows of the tile, NT threads; a stage covers KPS elements of K.
// ------------------------------------------------------------------------------------
template <Fmt F, int R, int NT> struct Loader;

template <int R, int NT> struct Loader<Fmt::I8, R, NT> {
    static constexpr int PLANES = 1, KPS = 128, NCH = R * 8, CH = (NCH + NT - 1) / NT;
    i32x4 r[CH];
    __device__ __forceinline__ void load(const char *base, long ld, int row0, int rows,
                                         int k0, int kend, int tid)
    {
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT, row = q >> 3, c = q & 7;
            const int gr = row0 + row, kk = k0 + c * 16;
            r[i] = i32x4{0, 0, 0, 0};
            if ((NCH % NT == 0 || q < NCH) && gr < rows && kk < kend)
                r[i] = *reinterpret_cast<const i32x4 *>(base + (long)gr * ld + kk);
        }
    }
    __device__ __forceinline__ void store(char *lds, int pstride, int tid) const
    {
        (void)pstride;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT;
            if (NCH % NT == 0 || q < NCH)
                *reinterpret_cast<i32x4 *>(lds + swz(q >> 3, q & 7)) = r[i];
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
    static constexpr int PLANES = 1, KPS = 128, NCH = R * 4, CH = (NCH + NT - 1) / NT;
    i32x4 r[CH];
    __device__ __forceinline__ void load(const char *base, long ld, int row0, int rows,
                                         int k0, int kend, int tid)
    {
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT, row = q >> 2, pc = q & 3;
            const int gr = row0 + row, kk = k0 + pc * 32;
            r[i] = i32x4{0, 0, 0, 0};
            if ((NCH % NT == 0 || q < NCH) && gr < rows && kk < kend)
                r[i] = *reinterpret_cast<const i32x4 *>(base + (long)gr * ld + (kk >> 1));
        }
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
__device__ __forceinline__ unsigned hi_byte16(int x)
{
    x = x > 32639 ? 32639 : x;
    return (unsigned)((x + 128) >> 8) & 0xFFu;
}
// two int16 in w -> (lo bytes, hi bytes) as 16-bit halves
__device__ __forceinline__ void split2(int w, unsigned &lo2, unsigned &hi2)
{
    const int x0 = (int)(short)(w & 0xFFFF), x1 = w >> 16;
    lo2 = ((unsigned)w & 0xFFu) | (((unsigned)w >> 8) & 0xFF00u);
    hi2 = hi_byte16(x0) | (hi_byte16(x1) << 8);
}

template <int R, int NT> struct Loader<Fmt::I16, R, NT> {
    static constexpr int PLANES = 2, KPS = 128, NCH = R * 8, CH = (NCH + NT - 1) / NT;
    i32x4 r[CH][2];
    __device__ __forceinline__ void load(const char *base, long ld, int row0, int rows,
                                         int k0, int kend, int tid)
    {
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT, row = q >> 3, c = q & 7;
            const int gr = row0 + row, kk = k0 + c * 16;
            r[i][0] = r[i][1] = i32x4{0, 0, 0, 0};
            if ((NCH % NT == 0 || q < NCH) && gr < rows && kk < kend) {
                const i32x4 *p = reinterpret_cast<const i32x4 *>(base + (long)gr * ld + 2L * kk);
                r[i][0] = p[0];
                r[i][1] = p[1];
            }
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
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int e = 0; e < 4; e++) split2(r[i][h][e], lo[h * 4 + e], hi[h * 4 + e]);
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
    static constexpr int PLANES = 1, KPS = 64, NCH = R * 8, CH = (NCH + NT - 1) / NT;
    i32x4 r[CH];
    __device__ __forceinline__ void load(const char *base, long ld, int row0, int rows,
                                         int k0, int kend, int tid)
    {
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT, row = q >> 3, c = q & 7;
            const int gr = row0 + row, kk = k0 + c * 8;
            r[i] = i32x4{0, 0, 0, 0};
            if ((NCH % NT == 0 || q < NCH) && gr < rows && kk < kend)
                r[i] = *reinterpret_cast<const i32x4 *>(base + (long)gr * ld + 2L * kk);
        }
    }
    __device__ __forceinline__ void store(char *lds, int pstride, int tid) const
    {
        (void)pstride;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT;
            if (NCH % NT == 0 || q < NCH)
                *reinterpret_cast<i32x4 *>(lds + swz(q >> 3, q & 7)) = r[i];
        }
    }
};

// fp32 -> bf16 by truncation: the high halves of two fp32 words packed into one word.
__device__ __forceinline__ int bf16pack(int f0, int f1)
{
    return (int)(((unsigned)f0 >> 16) | ((unsigned)f1 & 0xFFFF0000u));
}

template <int R, int NT> struct Loader<Fmt::F32BF16, R, NT> {
    static constexpr int PLANES = 1, KPS = 64, NCH = R * 8, CH = (NCH + NT - 1) / NT;
    i32x4 r[CH][2];
    __device__ __forceinline__ void load(const char *base, long ld, int row0, int rows,
                                         int k0, int kend, int tid)
    {
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT, row = q >> 3, c = q & 7;
            const int gr = row0 + row, kk = k0 + c * 8;
            r[i][0] = r[i][1] = i32x4{0, 0, 0, 0};
            if ((NCH % NT == 0 || q < NCH) && gr < rows && kk < kend) {
                const i32x4 *p = reinterpret_cast<const i32x4 *>(base + (long)gr * ld + 4L * kk);
                r[i][0] = p[0];
                r[i][1] = p[1];
            }
        }
    }
    __device__ __forceinline__ void store(char *lds, int pstride, int tid) const
    {
        (void)pstride;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT;
            if (NCH % NT == 0 || q < NCH) {
                const i32x4 a = r[i][0], b = r[i][1];
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
    static constexpr int PLANES = 2, KPS = 64, NCH = R * 8, CH = (NCH + NT - 1) / NT;
    i32x4 r[CH][2];
    __device__ __forceinline__ void load(const char *base, long ld, int row0, int rows,
                                         int k0, int kend, int tid)
    {
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int q = tid + i * NT, row = q >> 3, c = q & 7;
            const int gr = row0 + row, kk = k0 + c * 8;
            r[i][0] = r[i][1] = i32x4{0, 0, 0, 0};
            if ((NCH % NT == 0 || q < NCH) && gr < rows && kk < kend) {
                const i32x4 *p = reinterpret_cast<const i32x4 *>(base + (long)gr * ld + 4L * kk);
                r[i][0] = p[0];
                r[i][1] = p[1];
            }
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
                    tf32split(r[i][0][e], h[e], l[e]);
                    tf32split(r[i][1][e], h[4 + e], l[4 + e]);
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
// MFMA math. KSB = LDS bytes per row one substep consumes, KEL = K elements per substep.
// ------------------------------------------------------------------------------------
__device__ __forceinline__ i32x4 lds_frag16(const char *plane, int row, int sub, int lane)
{
    return *reinterpret_cast<const i32x4 *>(plane + swz(row, sub * 4 + (lane >> 4)));
}
__device__ __forceinline__ i32x2 lds_frag8(const char *plane, int row, int sub, int lane)
{
    const int g = lane >> 4;   // bytes [32*sub + 8*g, +8)
    return *reinterpret_cast<const i32x2 *>(plane + swz(row, sub * 2 + (g >> 1)) + ((g & 1) << 3));
}

struct MathI8 {            // int8 x int8, v_mfma_i32_16x16x64_i8
    using Acc = i32x4;
    static constexpr int NACC = 1, PA = 1, PB = 1, KSB = 64, KEL = 64;
    using Frag = i32x4;
    __device__ static Frag read(const char *pl, int row, int sub, int lane) { return lds_frag16(pl, row, sub, lane); }
    __device__ static void mma(Acc *acc, const Frag *a, const Frag *b)
    {
        acc[0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(b[0], a[0], acc[0], 0, 0, 0);
    }
};

struct MathI8x32 {         // int8 x int8, v_mfma_i32_16x16x32_i8 (groups that are odd multiples of 32)
    using Acc = i32x4;
    static constexpr int NACC = 1, PA = 1, PB = 1, KSB = 32, KEL = 32;
    using Frag = i32x2;
    __device__ static Frag read(const char *pl, int row, int sub, int lane) { return lds_frag8(pl, row, sub, lane); }
    __device__ static void mma(Acc *acc, const Frag *a, const Frag *b)
    {
        acc[0] = __builtin_amdgcn_mfma_i32_16x16x32_i8(__builtin_bit_cast(long, b[0]),
                                                       __builtin_bit_cast(long, a[0]), acc[0], 0, 0, 0);
    }
};

struct MathI16 {           // byte planes: acc0 = hi*hi, acc1 = hi*lo + lo*hi, acc2 = lo*lo
    using Acc = i32x4;
    static constexpr int NACC = 3, PA = 2, PB = 2, KSB = 64, KEL = 64;
    using Frag = i32x4;
    __device__ static Frag read(const char *pl, int row, int sub, int lane) { return lds_frag16(pl, row, sub, lane); }
    __device__ static void mma(Acc *acc, const Frag *a, const Frag *b)
    {
        acc[0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(b[0], a[0], acc[0], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(b[0], a[1], acc[1], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(b[1], a[0], acc[1], 0, 0, 0);
        acc[2] = __builtin_amdgcn_mfma_i32_16x16x64_i8(b[1], a[1], acc[2], 0, 0, 0);
    }
};

struct MathF16 {
    using Acc = f32x4;
    static constexpr int NACC = 1, PA = 1, PB = 1, KSB = 64, KEL = 32;
    using Frag = i32x4;
    __device__ static Frag read(const char *pl, int row, int sub, int lane) { return lds_frag16(pl, row, sub, lane); }
    __device__ static void mma(Acc *acc, const Frag *a, const Frag *b)
    {
        acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, b[0]),
                                                        __builtin_bit_cast(f16x8, a[0]), acc[0], 0, 0, 0);
    }
};

struct MathBF16 {
    using Acc = f32x4;
    static constexpr int NACC = 1, PA = 1, PB = 1, KSB = 64, KEL = 32;
    using Frag = i32x4;
    __device__ static Frag read(const char *pl, int row, int sub, int lane) { return lds_frag16(pl, row, sub, lane); }
    __device__ static void mma(Acc *acc, const Frag *a, const Frag *b)
    {
        acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, b[0]),
                                                         __builtin_bit_cast(bf16x8, a[0]), acc[0], 0, 0, 0);
    }
};

struct MathTF32 {          // bf16 hi/lo planes: hi*hi + lo*hi + hi*lo (lo*lo dropped)
    using Acc = f32x4;
    static constexpr int NACC = 1, PA = 2, PB = 2, KSB = 64, KEL = 32;
    using Frag = i32x4;
    __device__ static Frag read(const char *pl, int row, int sub, int lane) { return lds_frag16(pl, row, sub, lane); }
    __device__ static void mma(Acc *acc, const Frag *a, const Frag *b)
    {
        const bf16x8 ah = __builtin_bit_cast(bf16x8, a[0]), al = __builtin_bit_cast(bf16x8, a[1]);
        const bf16x8 bh = __builtin_bit_cast(bf16x8, b[0]), bl = __builtin_bit_cast(bf16x8, b[1]);
        acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bh, ah, acc[0], 0, 0, 0);
        acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bl, ah, acc[0], 0, 0, 0);
        acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bh, al, acc[0], 0, 0, 0);
    }
};

// ------------------------------------------------------------------------------------
// The kernel.
// ------------------------------------------------------------------------------------
template <int BM, int BN, Fmt FA, Fmt FB, class MATH, Epi EPI>
__global__ __launch_bounds__(256) void k_gemm(const KArgs args)
{
    constexpr int NT = 256, WGM = 2, WGN = 2;
    constexpr int TM = BM / WGM / 16, TN = BN / WGN / 16;
    using LA = Loader<FA, BM, NT>;
    using LB = Loader<FB, BN, NT>;
    static_assert(LA::KPS == LB::KPS, "operand stage K mismatch");
    static_assert(LA::KPS == MATH::KEL * (ROWB / MATH::KSB), "stage K vs MFMA substeps");
    static_assert(LA::PLANES == MATH::PA && LB::PLANES == MATH::PB, "plane count");
    constexpr int KPS = LA::KPS, NSUB = ROWB / MATH::KSB;
    constexpr int PLA = BM * ROWB, PLB = BN * ROWB;
    constexpr int STAGE = MATH::PA * PLA + MATH::PB * PLB;
    constexpr bool INT_ACC = std::is_same<typename MATH::Acc, i32x4>::value;
    constexpr bool B_I4 = (FB == Fmt::I4P);

    __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];

    // ---- which problem / tile ----
    int tile = xcd_remap((int)blockIdx.x, (int)gridDim.x);
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
    const int rowA = wm * (BM / WGM) + (lane & 15);   // A-tile row of block i: rowA + 16 i
    const int rowB = wn * (BN / WGN) + (lane & 15);   // B-tile row of block j: rowB + 16 j

    typename MATH::Acc acc[TM][TN][MATH::NACC];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int a = 0; a < MATH::NACC; a++) acc[i][j][a] = typename MATH::Acc{};

    // group-wise fp32 accumulators
    constexpr int TMG = (EPI == Epi::GW) ? TM : 1, TNG = (EPI == Epi::GW) ? TN : 1;
    f32x4 accf[TMG][TNG];
#pragma unroll
    for (int i = 0; i < TMG; i++)
#pragma unroll
        for (int j = 0; j < TNG; j++) accf[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // output coordinates of this lane
    const int m0 = bm * BM + wm * (BM / WGM) + (lane & 15);          // + 16 i
    const int n0 = bn * BN + wn * (BN / WGN) + 4 * (lane >> 4);      // + 16 j, 4 consecutive

    const char *Ab = static_cast<const char *>(P.A);
    const char *Bb = static_cast<const char *>(P.B);
    const int kbeg = args.kbeg, kend = args.kend;

    LA la;
    LB lb;
    la.load(Ab, args.lda, bm * BM, M, kbeg, kend, tid);
    lb.load(Bb, args.ldb, bn * BN, N, kbeg, kend, tid);
    la.store(smem, PLA, tid);
    lb.store(smem + MATH::PA * PLA, PLB, tid);
    __syncthreads();

    const int nst = (kend - kbeg + KPS - 1) / KPS;
#pragma unroll 1
    for (int s = 0; s < nst; s++) {
        const char *cur = smem + (s & 1) * STAGE;
        const bool more = (s + 1 < nst);
        if (more) {
            la.load(Ab, args.lda, bm * BM, M, kbeg + (s + 1) * KPS, kend, tid);
            lb.load(Bb, args.ldb, bn * BN, N, kbeg + (s + 1) * KPS, kend, tid);
        }
#pragma unroll
        for (int ss = 0; ss < NSUB; ss++) {
            typename MATH::Frag fa[TM][MATH::PA], fb[TN][MATH::PB];
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int pl = 0; pl < MATH::PA; pl++)
                    fa[i][pl] = MATH::read(cur + pl * PLA, rowA + 16 * i, ss, lane);
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int pl = 0; pl < MATH::PB; pl++)
                    fb[j][pl] = MATH::read(cur + MATH::PA * PLA + pl * PLB, rowB + 16 * j, ss, lane);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) MATH::mma(acc[i][j], fa[i], fb[j]);

            if constexpr (EPI == Epi::GW) {
                const int kpos = kbeg + s * KPS + (ss + 1) * MATH::KEL;   // K consumed so far
                if (kpos <= kend && (kpos % args.kt) == 0) {
                    const int g = (kpos - 1) / args.group, nG = args.nG;
                    float sa[TM], sb[TN][4];
#pragma unroll
                    for (int i = 0; i < TM; i++) {
                        const int m = m0 + 16 * i;
                        sa[i] = (m < M) ? P.a_scale[(long)m * nG + g] : 0.f;
                    }
#pragma unroll
                    for (int j = 0; j < TN; j++)
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            const int n = n0 + 16 * j + r;
                            const float b = (n < N) ? P.b_scale[(long)n * nG + g] : 0.f;
                            sb[j][r] = B_I4 ? b * 0.0625f : b;   // exact: removes the x16
                        }
                    const bool dump = args.dump && p == 0 && args.kt == args.group;
#pragma unroll
                    for (int i = 0; i < TM; i++)
#pragma unroll
                        for (int j = 0; j < TN; j++) {
                            const i32x4 v = acc[i][j][0];
#pragma unroll
                            for (int r = 0; r < 4; r++)
                                accf[i][j][r] = __builtin_fmaf(sa[i] * sb[j][r], (float)v[r], accf[i][j][r]);
                            if (dump) {
                                const int m = m0 + 16 * i, n = n0 + 16 * j;
                                if (m >= args.dump_row0 && m < args.dump_row0 + args.dump_rows && m < M && n < N) {
                                    const i32x4 q = B_I4 ? (v >> 4) : v;
                                    *reinterpret_cast<i32x4 *>(args.dump +
                                        ((long)(m - args.dump_row0) * nG + g) * N + n) = q;
                                }
                            }
                            acc[i][j][0] = i32x4{0, 0, 0, 0};
                        }
                }
            }
        }
        if (more) {
            char *nxt = smem + ((s + 1) & 1) * STAGE;
            la.store(nxt, PLA, tid);
            lb.store(nxt + MATH::PA * PLA, PLB, tid);
        }
        __syncthreads();
    }

    // ---- epilogue ----
#pragma unroll
    for (int i = 0; i < TM; i++) {
        const int m = m0 + 16 * i;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = n0 + 16 * j;
            if (n >= N) continue;
            const long off = (long)m * N + n;
            if constexpr (EPI == Epi::I32) {
                i32x4 v = acc[i][j][0];
                if (B_I4) v = v >> 4;
                i32x4 *c = reinterpret_cast<i32x4 *>(static_cast<int32_t *>(P.C) + off);
                if (args.accum) v += *c;
                *c = v;
            } else if constexpr (EPI == Epi::I64) {
                i64 *c = static_cast<i64 *>(P.C) + off;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    i64 v = (i64)acc[i][j][0][r] * 65536 + (i64)acc[i][j][1][r] * 256 + (i64)acc[i][j][2][r];
                    if (args.accum) v += c[r];
                    c[r] = v;
                }
            } else if constexpr (EPI == Epi::F16) {
                const f32x4 v = acc[i][j][0];
                f16x4 h = {(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
                *reinterpret_cast<f16x4 *>(static_cast<_Float16 *>(P.C) + off) = h;
            } else if constexpr (EPI == Epi::F32) {
                *reinterpret_cast<f32x4 *>(static_cast<float *>(P.C) + off) = acc[i][j][0];
            } else {   // GW
                *reinterpret_cast<f32x4 *>(static_cast<float *>(P.C) + off) = accf[i < TMG ? i : 0][j < TNG ? j : 0];
            }
            (void)INT_ACC;
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
template <int BM, int BN, Fmt FA, Fmt FB, class MATH, Epi EPI>
hipError_t launch_one(const KArgs &ka, int tiles, hipStream_t s)
{
    hipLaunchKernelGGL((k_gemm<BM, BN, FA, FB, MATH, EPI>), dim3(tiles), dim3(256), 0, s, ka);
    return hipGetLastError();
}

bool is_two_plane(Fmt f) { return f == Fmt::I16 || f == Fmt::F32TF32; }

}  // namespace

void gemm_tile(Fmt fmt_a, Epi epi, int M, int N, int *bm, int *bn)
{
    (void)epi;
    if (is_two_plane(fmt_a)) { *bm = 64; *bn = 64; return; }
    // 128 x 128 while it yields at least one workgroup per CU, else 64 x 64
    const long big = (long)((M + 127) / 128) * ((N + 127) / 128);
    if (big >= 256) { *bm = 128; *bn = 128; }
    else            { *bm = 64;  *bn = 64;  }
}

template <int BM, int BN>
static hipError_t dispatch_tile(const Launch &L, const KArgs &ka, int tiles)
{
    hipStream_t s = L.stream;
    const bool x32 = (L.epi == Epi::GW) && (L.kt % 64) != 0;
    if (L.fmt_a == Fmt::I8 && L.fmt_b == Fmt::I8) {
        if (L.epi == Epi::I32) return launch_one<BM, BN, Fmt::I8, Fmt::I8, MathI8, Epi::I32>(ka, tiles, s);
        if (L.epi == Epi::GW)
            return x32 ? launch_one<BM, BN, Fmt::I8, Fmt::I8, MathI8x32, Epi::GW>(ka, tiles, s)
                       : launch_one<BM, BN, Fmt::I8, Fmt::I8, MathI8, Epi::GW>(ka, tiles, s);
    }
    if (L.fmt_a == Fmt::I8 && L.fmt_b == Fmt::I4P) {
        if (L.epi == Epi::I32) return launch_one<BM, BN, Fmt::I8, Fmt::I4P, MathI8, Epi::I32>(ka, tiles, s);
        if (L.epi == Epi::GW)
            return x32 ? launch_one<BM, BN, Fmt::I8, Fmt::I4P, MathI8x32, Epi::GW>(ka, tiles, s)
                       : launch_one<BM, BN, Fmt::I8, Fmt::I4P, MathI8, Epi::GW>(ka, tiles, s);
    }
    if (L.fmt_a == Fmt::F16 && L.fmt_b == Fmt::F16) {
        if (L.epi == Epi::F16) return launch_one<BM, BN, Fmt::F16, Fmt::F16, MathF16, Epi::F16>(ka, tiles, s);
        if (L.epi == Epi::F32) return launch_one<BM, BN, Fmt::F16, Fmt::F16, MathF16, Epi::F32>(ka, tiles, s);
    }
    if (L.fmt_a == Fmt::F32BF16 && L.fmt_b == Fmt::F32BF16 && L.epi == Epi::F32)
        return launch_one<BM, BN, Fmt::F32BF16, Fmt::F32BF16, MathBF16, Epi::F32>(ka, tiles, s);
    if constexpr (BM == 64 && BN == 64) {   // two-plane formats fit 64 KiB of LDS only at 64 x 64
        if (L.fmt_a == Fmt::I16 && L.fmt_b == Fmt::I16 && L.epi == Epi::I64)
            return launch_one<64, 64, Fmt::I16, Fmt::I16, MathI16, Epi::I64>(ka, tiles, s);
        if (L.fmt_a == Fmt::F32TF32 && L.fmt_b == Fmt::F32TF32 && L.epi == Epi::F32)
            return launch_one<64, 64, Fmt::F32TF32, Fmt::F32TF32, MathTF32, Epi::F32>(ka, tiles, s);
    }
    return hipErrorInvalidValue;
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

    if (bm == 128) return dispatch_tile<128, 128>(L, ka, (int)tiles);
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
