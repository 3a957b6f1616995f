// attn.hip — fused attention for gfx950 (FlashAttention-2 style online softmax).
//
// One workgroup = 4 waves = 128 queries of one head; each wave owns 32 queries. The key
// axis is walked in tiles of 64 keys; the K tiles [64][dk], the V^T tiles [dv][64] and (for
// aligned masks) the mask tiles [128][64] go global -> LDS by buffer-load DMA ahead of use.
// The loop is software-pipelined: one iteration runs the previous tile's PV products with
// this tile's score arithmetic issued between them, then the next tile's QK products with
// this tile's exponentials between them, so the matrix pipe and the VALU work side by side
// (K runs a tile ahead of V^T).
//
// Scores are computed transposed, S^T = K Q^T (v_mfma_f32_32x32x16_f16, the K fragment
// first), so a lane holds ONE query (column l % 32) and 16 keys per 32-key block: the
// row max and row sum of the softmax are in-lane, plus one exchange between the two
// half-waves. The query's Q row stays in registers for the whole key loop. The output is
// accumulated transposed too, O^T += V^T P^T: P never leaves registers — the score
// registers of a 32-key block, rounded to fp16, become the second MFMA's B operand after
// one lane-half swap of two registers per 16 keys (v_permlane32_swap) puts them in natural
// key order, so each V^T fragment is one 16-byte LDS read. O is rescaled only when some
// running max grows by more than 8.
#include "attn.h"

#include <atomic>
#include <type_traits>

namespace rk {
namespace {

typedef int      i32x2  __attribute__((ext_vector_type(2)));
typedef int      i32x4  __attribute__((ext_vector_type(4)));
typedef float    f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x4  __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8  __attribute__((ext_vector_type(8)));
typedef __amdgpu_buffer_rsrc_t Rsrc;

constexpr uint32_t kOOB = 0x80000000u;   // an offset past every range: loads return 0
constexpr int BQ = 128, BK = 64, NW = 4;

__device__ __forceinline__ Rsrc rsrc(const void *base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

template <int N> __device__ __forceinline__ void wait_vm()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
#endif
}

__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

struct FaArgs {
    const _Float16 *Q, *K, *Vt, *mask;
    _Float16 *O;
    long q_hs, q_rs, k_hs, k_rs, v_hs, v_rs, o_hs, o_rs, m_rs;
    int T, n_kv, dk, dv, gqa, n_head;
    float scale, softcap;
    // key-axis split: workgroup z walks key tiles [z * tps, min((z + 1) * tps, tiles)) and,
    // when nsplit > 1, stores its output divided by its own sum (fp16: a convex combination
    // of V rows) and (max, sum) per query in part
    int nsplit, tps;
    void *part;     // [split][head][T][dv] fp16 outputs, then [split][head][T] (max, sum) fp32 pairs
    int nqb;        // query blocks of BQ
};

// LDS per stage: the K tile (64 rows of DHP halves) then the V^T tile (DVP rows of 64 keys,
// 128 bytes). 16-byte chunk c of row r sits at slot c ^ x(r), chosen so that the sixteen
// lanes one LDS cycle serves (sixteen consecutive rows, one chunk) hit all 64 banks once:
// x(r) = r & 15 when a row is a multiple of 256 bytes (every row starts on bank 0), else
// (r >> 1) & 7 (rows of 128 or 384 bytes start alternately on banks 0 and 32).
template <int DHP, int DVP> struct FaCfg {
    static constexpr int KC = DHP / 16;          // score MFMA k-steps
    static constexpr int KCPR = DHP / 8;         // 16-byte chunks per K row
    static constexpr int KINS = DHP / 32;        // K-tile DMA instructions per wave (64 * KCPR / 256)
    static constexpr int VINS = DVP / 32;        // V^T-tile DMA instructions per wave (DVP * 8 / 256)
    static constexpr int KBYTES = BK * DHP * 2, VBYTES = DVP * BK * 2, STAGE = KBYTES + VBYTES;
    static constexpr int DB = DVP / 32;          // 32-row blocks of the output dims
    static constexpr int LDS = 2 * STAGE;
    static constexpr int MBYTES = BQ * BK * 2;   // a mask tile (128 queries x 64 keys), DMA path only
    template <bool MDMA> static constexpr int lds() { return LDS + (MDMA ? 2 * MBYTES : 0); }
    __device__ static int kx(int row) { return (DHP * 2) % 256 == 0 ? (row & 15) : ((row >> 1) & 7); }
};
__device__ __forceinline__ int vx(int row) { return (row >> 1) & 7; }   // V^T rows: 128 bytes

template <int DHP, int DVP, bool MVEC, bool CAP>
__global__ __launch_bounds__(256) void k_flash_attn(const FaArgs a)
{
    using CF = FaCfg<DHP, DVP>;
    constexpr int KC = CF::KC, KCPR = CF::KCPR, KINS = CF::KINS, DB = CF::DB;
    [[maybe_unused]] constexpr int VINS = CF::VINS;
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int tid = threadIdx.x, lane = tid & 63, hh = lane >> 5, l32 = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Workgroup w runs on XCD w % 8. Logical ids are renumbered so each XCD gets a contiguous
    // range, and consecutive logical ids are the query blocks, then the query heads, that read
    // the same K / V key range: those workgroups share one XCD's L2.
    int qb, h, zs;
    {
        const int total = (int)gridDim.x, w = (int)blockIdx.x;
        const int xcd = w % 8, idx = w / 8, per = total / 8, rem = total % 8;
        int lid = xcd * per + (xcd < rem ? xcd : rem) + idx;
        qb = lid % a.nqb;
        lid /= a.nqb;
        const int hg = lid % a.gqa;
        lid /= a.gqa;
        const int hkk = lid % (a.n_head / a.gqa);
        zs = lid / (a.n_head / a.gqa);
        h = hkk * a.gqa + hg;
    }
    const int hk = h / a.gqa;
    const int q = qb * BQ + wave * 32 + l32;
    const bool qok = q < a.T;

    // this lane's query row as the B operand of the score MFMAs: step c takes dims
    // 16c + 8hh .. +8
    i32x4 qf[KC];
    {
        const _Float16 *qrow = a.Q + (size_t)h * a.q_hs + (size_t)(qok ? q : 0) * a.q_rs;
#pragma unroll
        for (int c = 0; c < KC; c++)
            qf[c] = (qok && 16 * c + 8 * hh < a.dk) ? *reinterpret_cast<const i32x4 *>(qrow + 16 * c + 8 * hh)
                                                    : i32x4{0, 0, 0, 0};
    }

    // DMA: lane slot g of a tile -> (row, chunk); the global chunk is the swizzled one. When
    // 256 slots (one instruction of every wave) cover whole rows, the lane's chunk is the same
    // in every instruction and instruction i only moves down 256 / KCPR rows: one offset
    // register plus a uniform step per instruction.
    // (x(r) repeats every 16 rows, so the step must be a multiple of 16 rows)
    constexpr bool KSEP = 256 % KCPR == 0 && (256 / KCPR) % 16 == 0;
    constexpr int KN = KSEP ? 1 : KINS;
    uint32_t kvo[KN];
#pragma unroll
    for (int i = 0; i < KN; i++) {
        const int g = (i * NW + wave) * 64 + lane, row = g / KCPR, lc = (g % KCPR) ^ CF::kx(row);
        kvo[i] = (lc * 8 < a.dk) ? (uint32_t)((long)row * a.k_rs + lc * 8) * 2u : kOOB;
    }
    // V^T: 8 chunks a row, so always separable (rows past dv are past the descriptor range)
    uint32_t vvo;
    {
        const int g = wave * 64 + lane, row = g >> 3, lc = (g & 7) ^ vx(row);
        vvo = (uint32_t)((long)row * a.v_rs + lc * 8) * 2u;
    }
    const uint32_t kstep = (uint32_t)((256 / KCPR) * a.k_rs * 2), vstep = (uint32_t)(32 * a.v_rs * 2);
    const _Float16 *Kh = a.K + (size_t)hk * a.k_hs;
    const _Float16 *Vh = a.Vt + (size_t)hk * a.v_hs;
    (void)Kh;   // used by the device pass only
    (void)Vh;
    // K tile kb into K slot `slot` (smem + slot * STAGE) and the V^T tile into V^T slot `slot`
    // (right after it): separate calls, so the K tiles can run a tile ahead of the V^T tiles.
    auto issue_k = [&](int kb, int slot) __attribute__((always_inline)) {
#if defined(__HIP_DEVICE_COMPILE__)
        const long k0 = (long)kb * BK;
        const long krows = a.n_kv - k0;
        const Rsrc rk = rsrc(Kh + k0 * a.k_rs, (uint32_t)((krows > 0 ? krows : 0) * a.k_rs * 2));
        char *ks = smem + slot * CF::STAGE;
        // (the per-instruction step goes into the vector offset: the descriptor's range check
        // covers the vector offset, not the scalar one)
#pragma unroll
        for (int i = 0; i < KINS; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void *)(ks + (i * NW + wave) * 1024),
                                                     16, KSEP ? kvo[0] + i * kstep : kvo[i < KN ? i : 0], 0, 0, 0);
#else
        (void)kb; (void)slot; (void)kvo; (void)kstep;
#endif
    };
    auto issue_v = [&](int kb, int slot) __attribute__((always_inline)) {
#if defined(__HIP_DEVICE_COMPILE__)
        const long k0 = (long)kb * BK;
        const Rsrc rv = rsrc(Vh + k0, (uint32_t)((long)a.dv * a.v_rs * 2 - k0 * 2));
        char *vs = smem + slot * CF::STAGE + CF::KBYTES;
#pragma unroll
        for (int i = 0; i < VINS; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (__attribute__((address_space(3))) void *)(vs + (i * NW + wave) * 1024),
                                                     16, vvo + i * vstep, 0, 0, 0);
#else
        (void)kb; (void)slot; (void)vvo; (void)vstep;
#endif
    };

    float m_run = -INFINITY, l_run = 0.f;
    f32x16 O[DB];
#pragma unroll
    for (int d = 0; d < DB; d++) O[d] = f32x16{};
    const bool use_mask = a.mask != nullptr && qok;
    const int tiles = (a.n_kv + BK - 1) / BK;
    const int kb0 = zs * a.tps, kb1 = min(tiles, kb0 + a.tps);

    // This lane's mask values of a tile (keys key0 + 32 sb + 8 b + 4 hh + c). MVEC (rows of
    // a multiple of 8 halves, a 16-byte aligned mask): the workgroup's 128 x 64 tile goes
    // global -> LDS by DMA a tile ahead, 128 contiguous bytes a row (16-byte chunk c of row r
    // at slot c ^ vx(r)), and each lane reads its keys from LDS after the barrier (the
    // lane-per-query loads it replaces touched 32 rows per instruction: 60.9 -> 59.3 us a
    // call at 512 x 4096, d 256). Otherwise buffer loads a tile ahead, 8 bytes where rows are
    // a multiple of 4 halves and the mask 8-byte aligned, else 2 (rows past T read zeros;
    // keys past n_kv may read the next row, which does not matter as those keys weigh 0).
    // No mask: no loads, zeros.
    const Rsrc rm = rsrc(a.mask, a.mask ? (uint32_t)((long)a.T * a.m_rs * 2) : 0u);
    const uint32_t mbase = use_mask ? (uint32_t)((long)q * a.m_rs * 2) : kOOB;
    [[maybe_unused]] uint32_t mvo = 0;
    if constexpr (MVEC) {
        const int g = wave * 64 + lane, row = g >> 3;
        mvo = (uint32_t)((long)(qb * BQ + row) * a.m_rs + ((g & 7) ^ vx(row)) * 8) * 2u;
    }
    const bool m8 = a.m_rs % 4 == 0 && ((uintptr_t)a.mask & 7u) == 0;
    auto load_mask = [&](int kb, f16x4 (&m)[2][4]) __attribute__((always_inline)) {
        if (a.mask == nullptr) return;
        const int key0 = kb * BK;
#pragma unroll
        for (int sb = 0; sb < 2; sb++)
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const uint32_t off = mbase + (uint32_t)(key0 + 32 * sb + 8 * b + 4 * hh) * 2u;
                if (m8) {
                    m[sb][b] = __builtin_bit_cast(f16x4, __builtin_amdgcn_raw_buffer_load_b64(rm, off, 0, 0));
                } else {
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        m[sb][b][c] = __builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(rm, off + 2 * c, 0, 0));
                }
            }
    };
    // MVEC: mask tile kb into mask slot `slot` (four instructions a wave, 8 rows each; rows
    // past T lie past the descriptor's range and read zeros)
    auto issue_m = [&](int kb, int slot) __attribute__((always_inline)) {
#if defined(__HIP_DEVICE_COMPILE__)
        if constexpr (MVEC) {
            const long k0 = (long)kb * BK;
            const Rsrc rt = rsrc(a.mask + k0, (uint32_t)((long)a.T * a.m_rs * 2 - k0 * 2));
            char *ms = smem + CF::LDS + slot * CF::MBYTES;
#pragma unroll
            for (int i = 0; i < 4; i++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rt, (__attribute__((address_space(3))) void *)(ms + (i * NW + wave) * 1024),
                                                         16, mvo + (uint32_t)i * (uint32_t)(32 * a.m_rs * 2), 0, 0, 0);
        }
#else
        (void)kb; (void)slot;
#endif
    };
    auto read_mask = [&](int slot, f16x4 (&m)[2][4]) __attribute__((always_inline)) {
        const int row = wave * 32 + l32;
        const char *mr = smem + CF::LDS + slot * CF::MBYTES + row * 128 + 8 * hh;
#pragma unroll
        for (int sb = 0; sb < 2; sb++)
#pragma unroll
            for (int b = 0; b < 4; b++) m[sb][b] = *reinterpret_cast<const f16x4 *>(mr + (((4 * sb + b) ^ vx(row)) << 4));
    };
    f16x4 mnext[2][4] = {};
    if constexpr (!MVEC) load_mask(kb0, mnext);

    // S^T for the 64 keys of the K tile in slot `slot`: two 32-key blocks; the K fragments of
    // step c + 2 are read while step c's MFMAs run (three steps of fragments in registers)
    auto qk = [&](int slot, f32x16 (&Sx)[2], auto &&beside) __attribute__((always_inline)) {
        const char *ks = smem + slot * CF::STAGE;
        Sx[0] = f32x16{};
        Sx[1] = f32x16{};
        auto kfrag = [&](int c, int sb) __attribute__((always_inline)) {
            const int row = 32 * sb + l32, lc = 2 * c + hh;
            return *reinterpret_cast<const i32x4 *>(ks + row * (DHP * 2) + ((lc ^ CF::kx(row)) << 4));
        };
        i32x4 kf[3][2];
        kf[0][0] = kfrag(0, 0);
        kf[0][1] = kfrag(0, 1);
        if constexpr (KC > 1) {
            kf[1][0] = kfrag(1, 0);
            kf[1][1] = kfrag(1, 1);
        }
#pragma unroll
        for (int c = 0; c < KC; c++) {
            if (c + 2 < KC) {
                kf[(c + 2) % 3][0] = kfrag(c + 2, 0);
                kf[(c + 2) % 3][1] = kfrag(c + 2, 1);
            }
#pragma unroll
            for (int sb = 0; sb < 2; sb++) {
                Sx[sb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, kf[c % 3][sb]),
                                                                __builtin_bit_cast(f16x8, qf[c]), Sx[sb], 0, 0, 0);
                beside(2 * c + sb);   // independent VALU work issued under this MFMA
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    // The scores of tile kb (the reference's fp32 steps; the soft-cap variant is its own
    // kernel, so the common one carries no tanh code and its registers), in log2 units
    // (x log2 e) so that p = 2^(v - m) is one v_exp_f32; returns their max over the tile.
    // score element e (block e / 16, register e % 16) of a tile
    auto transform1 = [&](f32x16 (&Sx)[2], int e) __attribute__((always_inline)) {
        constexpr float L2E = 1.4426950408889634f;
        const int sb = e >> 4, r = e & 15;
        float v;
        if constexpr (CAP) {
            v = a.softcap * tanhf(Sx[sb][r] * a.scale / a.softcap);
            v = fmaxf(v + (float)mnext[sb][r >> 2][r & 3], -30000.f) * L2E;
        } else {
            v = fmaf((float)mnext[sb][r >> 2][r & 3], L2E, Sx[sb][r] * (a.scale * L2E));
            v = fmaxf(v, -30000.f * L2E);
        }
        Sx[sb][r] = v;
    };
    auto transform = [&](f32x16 (&Sx)[2]) __attribute__((always_inline)) {
#pragma unroll
        for (int e = 0; e < 32; e++) transform1(Sx, e);
    };
    auto finish = [&](int kb, f32x16 (&Sx)[2]) __attribute__((always_inline)) {
        const int key0 = kb * BK;
        if (__builtin_expect(key0 + BK > a.n_kv, 0)) {   // keys past n_kv weigh 0 (last tile only)
#pragma unroll
            for (int sb = 0; sb < 2; sb++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int key = key0 + 32 * sb + 8 * (r >> 2) + 4 * hh + (r & 3);
                    if (key >= a.n_kv) Sx[sb][r] = -INFINITY;
                }
        }
        float mloc = -INFINITY;
#pragma unroll
        for (int sb = 0; sb < 2; sb++)
#pragma unroll
            for (int r = 0; r < 16; r++) mloc = fmaxf(mloc, Sx[sb][r]);
        if constexpr (!MVEC) {
            if (kb + 1 < kb1) load_mask(kb + 1, mnext);   // lands during the next tile's products
        }
        return fmaxf(mloc, __shfl_xor(mloc, 32, 64));
    };
    // The running max moves only when some query's scores pass it by more than 8 (natural
    // units; 11.5 in log2 units, so p = 2^(v - m) <= 2^11.5 stays well inside fp16): O and
    // the sum are then rescaled by 2^(m_old - m_new). The final division by the sum makes
    // the result independent of which max was used. Returns the factor for the sum.
    auto grow = [&](float mloc) __attribute__((always_inline)) {
        float alpha = 1.f;
        if (__builtin_expect(__any(mloc > m_run + 11.5f), 0)) {
            const float m_new = fmaxf(m_run, mloc);
            alpha = exp2f(m_run - m_new);
            m_run = m_new;
#pragma unroll
            for (int d = 0; d < DB; d++) O[d] *= alpha;
        }
        return alpha;
    };
    // p = 2^(v - m_run) in fp16, their sum, and P reordered to natural key order per
    // half-wave: of each 16 keys, half 0 supplies keys 0..7 and half 1 keys 8..15, so one
    // 16-byte LDS read is a V^T fragment. Half 0 holds keys 0-3 and 8-11, half 1 keys 4-7 and
    // 12-15 (the score layout): swap half 0's keys 8-11 with half 1's keys 4-7 (two packed
    // registers, lanes 0-31 <-> 32-63).
    auto prob1 = [&](const f32x16 (&Sx)[2], f16x8 (&pb)[2][2], float &psum, int e) __attribute__((always_inline)) {
        const int sb = e >> 4, r = e & 15;
        const float p = __builtin_amdgcn_exp2f(Sx[sb][r] - m_run);
        psum += p;
        pb[sb][r >> 3][r & 7] = (_Float16)p;
    };
    auto reorder = [&](f16x8 (&pb)[2][2]) __attribute__((always_inline)) {
#pragma unroll
        for (int sb = 0; sb < 2; sb++)
#pragma unroll
            for (int t = 0; t < 2; t++) {
                i32x4 w = __builtin_bit_cast(i32x4, pb[sb][t]);
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const auto r = __builtin_amdgcn_permlane32_swap((unsigned)w[e], (unsigned)w[2 + e], false, false);
                    w[e] = (int)r[0];
                    w[2 + e] = (int)r[1];
                }
                pb[sb][t] = __builtin_bit_cast(f16x8, w);
            }
    };
    // O^T += V^T P^T for the V^T tile in slot `slot`: four 16-key steps, each an MFMA into
    // every 32-dim block (independent accumulators back to back); the V^T fragments of the
    // next step are read meanwhile
    auto pv = [&](int slot, const f16x8 (&pb)[2][2], auto &&beside) __attribute__((always_inline)) {
        const char *vs = smem + slot * CF::STAGE + CF::KBYTES;
        auto vfrag = [&](int j, int db) __attribute__((always_inline)) {   // keys 16 j + 8 hh .. +8
            const int d = 32 * db + l32;
            return *reinterpret_cast<const i32x4 *>(vs + d * 128 + (((2 * j + hh) ^ vx(d)) << 4));
        };
        i32x4 vf[2][DB];
#pragma unroll
        for (int db = 0; db < DB; db++) vf[0][db] = vfrag(0, db);
#pragma unroll
        for (int j = 0; j < 4; j++) {
#pragma unroll
            for (int db = 0; db < DB; db++) {
                if (j + 1 < 4) vf[(j + 1) & 1][db] = vfrag(j + 1, db);
                O[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, vf[j & 1][db]),
                                                               pb[j >> 1][j & 1], O[db], 0, 0, 0);
                beside(j * DB + db);   // independent VALU work issued under this MFMA
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    // Software pipeline over the key tiles: iteration kb runs tile kb - 1's PV products beside
    // tile kb's score arithmetic, then tile kb + 1's QK products beside tile kb's
    // exponentials, so each phase's MFMAs have independent VALU work to overlap. K runs a
    // tile ahead of V^T: at the top of iteration kb (after the barrier) K tile kb + 2 goes
    // into the K slot tile kb left (its QK ran in iteration kb - 1) and V^T tile kb into the
    // V^T slot tile kb - 2 left (its PV ran in iteration kb - 1); iteration kb reads K tile
    // kb + 1 and V^T tile kb - 1, which the previous iteration issued.
    issue_k(kb0, 0);
    issue_m(kb0, 0);
    wait_vm<0>();
    lds_barrier();
    if (kb0 + 1 < kb1) issue_k(kb0 + 1, 1);
    // the elements of a tile's softmax work spread over a phase's 32 MFMAs (KC = 16 score
    // steps of two MFMAs for head size 256; fewer steps take several elements each)
    constexpr int QKM = 2 * KC, PVM = 4 * DB;
    auto none = [](int) {};
    f32x16 S[2];
    qk(0, S, none);
    f16x8 P[2][2];
    float psum;
    auto exps = [&](int m) __attribute__((always_inline)) {
#pragma unroll
        for (int e = m * 32 / QKM; e < (m + 1) * 32 / QKM; e++) prob1(S, P, psum, e);
    };
    // One iteration; the first has no PV products yet, the last no next tile to score.
    auto body = [&](auto FIRST, auto LAST, int kb) __attribute__((always_inline)) {
        const int cur = (kb - kb0) & 1;
        wait_vm<0>();
        lds_barrier();
        if (kb + 2 < kb1) issue_k(kb + 2, cur);
        issue_v(kb, cur);
        if constexpr (MVEC) {
            if (kb + 1 < kb1) issue_m(kb + 1, cur ^ 1);
            read_mask(cur, mnext);
        }
        if constexpr (decltype(FIRST)::value) {
            transform(S);
        } else {
            pv(cur ^ 1, P, [&](int m) __attribute__((always_inline)) {
#pragma unroll
                for (int e = m * 32 / PVM; e < (m + 1) * 32 / PVM; e++) transform1(S, e);
            });
        }
        const float alpha = grow(finish(kb, S));
        psum = 0.f;
        if constexpr (decltype(LAST)::value) {
#pragma unroll
            for (int e = 0; e < 32; e++) prob1(S, P, psum, e);
        } else {
            f32x16 Sn[2];
            qk(cur ^ 1, Sn, exps);
            S[0] = Sn[0];
            S[1] = Sn[1];
        }
        reorder(P);
        l_run = l_run * alpha + psum;
    };
    using T_ = std::true_type;
    using F_ = std::false_type;
    if (kb1 - kb0 == 1) {
        body(T_{}, T_{}, kb0);
    } else {
        body(T_{}, F_{}, kb0);
#pragma unroll 1
        for (int kb = kb0 + 1; kb < kb1 - 1; kb++) body(F_{}, F_{}, kb);
        body(F_{}, T_{}, kb1 - 1);
    }
    wait_vm<0>();
    lds_barrier();
    pv((kb1 - 1 - kb0) & 1, P, none);

    // normalise; lane holds dims 32 db + 8 b + 4 hh + c of its query
    const float l = l_run + __shfl_xor(l_run, 32, 64);
    if (a.nsplit > 1) {   // this split's share: its output over its sum (fp16), running max and sum
        if (qok) {
            const size_t row = ((size_t)zs * a.n_head + h) * a.T + q;
            _Float16 *po = static_cast<_Float16 *>(a.part) + row * a.dv;
            const float linv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
            for (int db = 0; db < DB; db++)
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const int d0 = 32 * db + 8 * b + 4 * hh;
                    if (d0 < a.dv) {
                        f16x4 v;
#pragma unroll
                        for (int c = 0; c < 4; c++) v[c] = (_Float16)(O[db][4 * b + c] * linv);
                        *reinterpret_cast<f16x4 *>(po + d0) = v;
                    }
                }
            if (hh == 0) {
                float *pml = reinterpret_cast<float *>(static_cast<_Float16 *>(a.part) +
                                                       (size_t)a.nsplit * a.n_head * a.T * a.dv) + 2 * row;
                pml[0] = m_run;
                pml[1] = l;
            }
        }
        return;
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    if (qok) {
        _Float16 *orow = a.O + (size_t)h * a.o_hs + (size_t)q * a.o_rs;
#pragma unroll
        for (int db = 0; db < DB; db++)
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const int d0 = 32 * db + 8 * b + 4 * hh;
                if (d0 < a.dv) {
                    f16x4 v;
#pragma unroll
                    for (int c = 0; c < 4; c++) v[c] = (_Float16)(O[db][4 * b + c] * inv);
                    *reinterpret_cast<f16x4 *>(orow + d0) = v;
                }
            }
    }
}

// Merges the key-axis splits: out = sum_s w_s On_s / sum_s w_s with w_s = 2^(m_s - m) l_s,
// m = max_s m_s (the splits' running maxima, in log2 units) and On_s = O_s / l_s the split's
// stored output, for 8 output dims of one (head, query) per thread. (The same quotient as
// sum_s 2^(m_s - m) O_s / sum_s 2^(m_s - m) l_s; the stored On_s are convex combinations of
// V rows, so fp16 holds them at half the bytes of unnormalised fp32 sums.)
template <int MAXS>
__global__ __launch_bounds__(256) void k_fa_combine(const void *__restrict__ part, _Float16 *__restrict__ O,
                                                     long o_hs, long o_rs, int n_head, int T, int dv, int nsplit)
{
    // 8 output dims a thread; every split's (m, l) pair and 16-byte output slice are loaded
    // up front (nsplit <= MAXS), then folded in split order
    const int dq = dv / 8;
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long)n_head * T * dq) return;
    const int d0 = (int)(i % dq) * 8;
    const long hq = i / dq;   // h * T + q
    const int h = (int)(hq / T), q = (int)(hq % T);
    const size_t rows = (size_t)n_head * T;
    const _Float16 *po = static_cast<const _Float16 *>(part);
    const float *ml = reinterpret_cast<const float *>(po + (size_t)nsplit * rows * dv);
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    f32x2 mls[MAXS];
    f16x8 os[MAXS];
#pragma unroll
    for (int sp = 0; sp < MAXS; sp++)
        if (sp < nsplit) {
            const size_t row = sp * rows + hq;
            mls[sp] = *reinterpret_cast<const f32x2 *>(ml + 2 * row);
            os[sp] = *reinterpret_cast<const f16x8 *>(po + row * dv + d0);
        }
    float m = -INFINITY;
#pragma unroll
    for (int sp = 0; sp < MAXS; sp++)
        if (sp < nsplit) m = fmaxf(m, mls[sp][0]);
    float l = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sp = 0; sp < MAXS; sp++)
        if (sp < nsplit) {
            const float w = exp2f(mls[sp][0] - m) * mls[sp][1];   // the maxima are in log2 units
            l += w;
#pragma unroll
            for (int c = 0; c < 8; c++) acc[c] += w * (float)os[sp][c];
        }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    _Float16 *dst = O + (size_t)h * o_hs + (size_t)q * o_rs + d0;
#pragma unroll
    for (int hv = 0; hv < 2; hv++) {
        f16x4 v;
#pragma unroll
        for (int c = 0; c < 4; c++) v[c] = (_Float16)(acc[4 * hv + c] * inv);
        *reinterpret_cast<f16x4 *>(dst + 4 * hv) = v;
    }
}

__global__ void k_pad_cols(const _Float16 *__restrict__ src, long src_rs, _Float16 *__restrict__ dst, long rows,
                           int cols, int cols_pad)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * cols_pad) return;
    const long r = i / cols_pad;
    const int c = (int)(i % cols_pad);
    dst[i] = c < cols ? src[r * src_rs + c] : (_Float16)0.f;
}

__global__ void k_heads_transpose(const _Float16 *__restrict__ src, _Float16 *__restrict__ dst, int T, int n_head,
                                  int dh, int t_pad)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long total = (long)n_head * dh * t_pad;
    if (i >= total) return;
    const int t = (int)(i % t_pad);
    const long hc = i / t_pad;                 // h * dh + c
    dst[i] = t < T ? src[(long)t * n_head * dh + hc] : (_Float16)0.f;
}

template <int DHP, int DVP, bool MVEC, bool CAP>
hipError_t launch_fa(const FaArgs &a, dim3 grid, hipStream_t s)
{
    using CF = FaCfg<DHP, DVP>;
    constexpr int lds = CF::template lds<MVEC>();
    static_assert(lds <= 160 * 1024, "LDS budget");
    auto kern = k_flash_attn<DHP, DVP, MVEC, CAP>;
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
    hipLaunchKernelGGL(kern, grid, dim3(256), lds, s, a);
    return hipGetLastError();
}

template <int DHP, int DVP>
hipError_t launch_fa2(const FaArgs &a, bool mvec, dim3 grid, hipStream_t s)
{
    if (a.softcap != 0.f)
        return mvec ? launch_fa<DHP, DVP, true, true>(a, grid, s) : launch_fa<DHP, DVP, false, true>(a, grid, s);
    return mvec ? launch_fa<DHP, DVP, true, false>(a, grid, s) : launch_fa<DHP, DVP, false, false>(a, grid, s);
}

int round_dim(int d) { return d <= 64 ? 64 : (d <= 128 ? 128 : (d <= 192 ? 192 : 256)); }

hipError_t launch_fa_dims(const FaArgs &a, bool mvec, int dhp, int dvp, dim3 grid, hipStream_t s);

bool al(const void *p, unsigned n) { return ((uintptr_t)p & (n - 1)) == 0; }

}  // namespace

static int fa_splits(const FaLaunch &L)
{
    // enough workgroups for every CU (256), each split keeping at least 4 key tiles
    const long wgs = (long)((L.T + BQ - 1) / BQ) * L.n_head;
    const int tiles = (L.n_kv + BK - 1) / BK;
    long want = (256 + wgs - 1) / wgs;
    if (want > tiles / 4) want = tiles / 4;
    if (want > 16) want = 16;
    return want < 1 ? 1 : (int)want;
}

size_t flash_attn_ws_bytes(const FaLaunch &L)
{
    const int ns = fa_splits(L);
    return ns > 1 ? (size_t)ns * L.n_head * L.T * (L.dv * sizeof(_Float16) + 2 * sizeof(float)) : 0;
}

hipError_t flash_attn(const FaLaunch &L, hipStream_t s, uint64_t *blocks_out)
{
    if (blocks_out) *blocks_out = 0;
    if (L.T < 1 || L.n_kv < 1 || L.n_head < 1 || L.gqa < 1 || L.n_head % L.gqa) return hipErrorInvalidValue;
    if (L.dk < 16 || L.dk % 16 || L.dk > kAttnMaxHeadDim || L.dv < 16 || L.dv % 16 || L.dv > kAttnMaxHeadDim)
        return hipErrorInvalidValue;
    if (!L.Q || !L.K || !L.Vt || !L.O) return hipErrorInvalidValue;
    // 16-byte Q / K chunks, 16-byte V^T DMA chunks, 8-byte output stores
    if (!al(L.Q, 16) || !al(L.K, 16) || !al(L.Vt, 16) || !al(L.O, 8) || L.q_rs % 8 || L.q_hs % 8 || L.k_rs % 8 ||
        L.k_hs % 8 || L.v_rs % 64 || L.v_hs % 8 || L.v_rs < L.n_kv || L.o_rs % 4 || L.o_hs % 4)
        return hipErrorInvalidValue;
    // buffer ranges and DMA offsets are 32-bit
    if ((long)L.n_kv * L.k_rs * 2 >= (1L << 31) || (long)L.dv * L.v_rs * 2 >= (1L << 31) ||
        (L.mask && ((long)L.T * L.m_rs * 2 >= (1L << 31) || L.m_rs < L.n_kv)))
        return hipErrorInvalidValue;
    const bool mvec = L.mask && L.m_rs % 8 == 0 && al(L.mask, 16);
    FaArgs a;
    a.Q = L.Q; a.K = L.K; a.Vt = L.Vt; a.mask = L.mask; a.O = L.O;
    a.q_hs = L.q_hs; a.q_rs = L.q_rs; a.k_hs = L.k_hs; a.k_rs = L.k_rs; a.v_hs = L.v_hs; a.v_rs = L.v_rs;
    a.o_hs = L.o_hs; a.o_rs = L.o_rs; a.m_rs = L.m_rs;
    a.T = L.T; a.n_kv = L.n_kv; a.dk = L.dk; a.dv = L.dv; a.gqa = L.gqa; a.n_head = L.n_head;
    a.scale = L.scale; a.softcap = L.softcap;
    const int tiles = (L.n_kv + BK - 1) / BK;
    a.nsplit = L.ws ? fa_splits(L) : 1;
    if (a.nsplit > 1 && L.ws_bytes < flash_attn_ws_bytes(L)) a.nsplit = 1;
    a.tps = (tiles + a.nsplit - 1) / a.nsplit;
    a.nsplit = (tiles + a.tps - 1) / a.tps;   // no empty split
    a.part = a.nsplit > 1 ? L.ws : nullptr;
    int dvp = round_dim(L.dv), dhp = round_dim(L.dk);
    if (dhp < dvp) dhp = dvp;
    a.nqb = (L.T + BQ - 1) / BQ;
    const long wgs = (long)a.nqb * L.n_head * a.nsplit;
    if (wgs > 0x7FFFFFFFL) return hipErrorInvalidValue;
    const dim3 grid((unsigned)wgs);
    if (blocks_out) *blocks_out = (uint64_t)wgs;
    const hipError_t e = launch_fa_dims(a, mvec, dhp, dvp, grid, s);
    if (e != hipSuccess || a.nsplit == 1) return e;
    const long n = (long)L.n_head * L.T * (L.dv / 8), blocks = (n + 255) / 256;
    if (a.nsplit <= 4)
        hipLaunchKernelGGL(k_fa_combine<4>, dim3((unsigned)blocks), dim3(256), 0, s, a.part, L.O, L.o_hs, L.o_rs,
                           L.n_head, L.T, L.dv, a.nsplit);
    else if (a.nsplit <= 8)
        hipLaunchKernelGGL(k_fa_combine<8>, dim3((unsigned)blocks), dim3(256), 0, s, a.part, L.O, L.o_hs, L.o_rs,
                           L.n_head, L.T, L.dv, a.nsplit);
    else
        hipLaunchKernelGGL(k_fa_combine<16>, dim3((unsigned)blocks), dim3(256), 0, s, a.part, L.O, L.o_hs, L.o_rs,
                           L.n_head, L.T, L.dv, a.nsplit);
    if (blocks_out) *blocks_out += (uint64_t)blocks;
    return hipGetLastError();
}

namespace {

hipError_t launch_fa_dims(const FaArgs &a, bool mvec, int dhp, int dvp, dim3 grid, hipStream_t s)
{
    switch (dhp * 1000 + dvp) {
    case 64064: return launch_fa2<64, 64>(a, mvec, grid, s);
    case 128064: return launch_fa2<128, 64>(a, mvec, grid, s);
    case 128128: return launch_fa2<128, 128>(a, mvec, grid, s);
    case 192064: return launch_fa2<192, 64>(a, mvec, grid, s);
    case 192128: return launch_fa2<192, 128>(a, mvec, grid, s);
    case 192192: return launch_fa2<192, 192>(a, mvec, grid, s);
    case 256064: return launch_fa2<256, 64>(a, mvec, grid, s);
    case 256128: return launch_fa2<256, 128>(a, mvec, grid, s);
    case 256192: return launch_fa2<256, 192>(a, mvec, grid, s);
    case 256256: return launch_fa2<256, 256>(a, mvec, grid, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace

hipError_t pad_cols_f16(const _Float16 *src, long src_rs, _Float16 *dst, long rows, int cols, int cols_pad,
                        hipStream_t s)
{
    if (rows < 1 || cols < 1 || cols_pad < cols || src_rs < cols) return hipErrorInvalidValue;
    const long n = rows * cols_pad, blocks = (n + 255) / 256;
    if (blocks > 0x7FFFFFFFL) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_pad_cols, dim3((unsigned)blocks), dim3(256), 0, s, src, src_rs, dst, rows, cols, cols_pad);
    return hipGetLastError();
}

hipError_t heads_transpose_f16(const _Float16 *src, _Float16 *dst, int T, int n_head, int dh, int t_pad,
                               hipStream_t s)
{
    if (T < 1 || n_head < 1 || dh < 1 || t_pad < T) return hipErrorInvalidValue;
    const long n = (long)n_head * dh * t_pad, blocks = (n + 255) / 256;
    if (blocks > 0x7FFFFFFFL) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_heads_transpose, dim3((unsigned)blocks), dim3(256), 0, s, src, dst, T, n_head, dh, t_pad);
    return hipGetLastError();
}

}  // namespace rk
