// matmul.cpp — the one-shot matmul entries of rocket_matmul.h and their planners.
//
// Each entry keeps the reference's validation and return codes (reference
// src/rocket_matmul.c; lines cited per entry) and runs one gfx950 kernel launch
// (gemm.hip) on the handle's stream through rk::run.
#include "ops.h"
#include "rocket_hip.h"
#include "rocket_hw_profile.h"
#include "rocket_matmul.h"

#include <stdlib.h>
#include <string.h>

#include <algorithm>

namespace rk {

size_t fmt_row_bytes(Fmt f, int K)
{
    switch (f) {
    case Fmt::I8: return (size_t)K;
    case Fmt::I4P: return (size_t)K / 2;
    case Fmt::I16: case Fmt::F16: case Fmt::BF16: return 2 * (size_t)K;
    case Fmt::F32BF16: case Fmt::F32TF32: case Fmt::BF16X2: return 4 * (size_t)K;
    }
    return 0;
}

size_t epi_elem_bytes(Epi e)
{
    switch (e) {
    case Epi::I32: return 4;
    case Epi::I64: return 8;
    case Epi::F16: case Epi::GLU: case Epi::ACT: return 2;
    case Epi::F32: case Epi::GW: return 4;
    }
    return 0;
}

// n fp32 values at device address src (and n2 at src2, when src2 is given) converted into
// arena scratch in one launch; false on failure (the Call then carries the error).
static bool convert(Call &c, const void *src, size_t n, Fmt to, const void **out, const void *src2 = nullptr,
                    size_t n2 = 0, const void **out2 = nullptr)
{
    const size_t el = to == Fmt::BF16X2 ? 4 : 2;
    void *dst = c.scratch(n * el);
    void *dst2 = src2 ? c.scratch(n2 * el) : nullptr;
    if (!dst || (src2 && !dst2)) return false;
    if (convert_f32(static_cast<const float *>(src), dst, (long)n, to, c.stream(), static_cast<const float *>(src2),
                    dst2, src2 ? (long)n2 : 0) != hipSuccess) {
        (void)hipGetLastError();
        ROCKET_LOGE("%s: fp32 conversion launch failed\n", c.who());
        return false;
    }
    count_launch((uint64_t)((n / 8 + (src2 ? n2 / 8 : 0) + 255) / 256));
    *out = dst;
    if (src2) *out2 = dst2;
    return true;
}

int gw_period(int group)
{
    if (group <= 65536) return group;
    for (int d = 65536 / 32 * 32; d >= 32; d -= 32)
        if (group % d == 0) return d;
    return 32;
}

// fp32 operands (bf16 / tf32 entries) are either converted as the GEMM loads them, or
// converted first in one streaming pass into the handle's arena (bf16: half the bytes;
// tf32: hi/lo pairs), so the GEMM moves half the bytes through L2 (bf16) and spends no VALU
// on the conversion. The pass costs one extra read + write of the operand, so it pays for
// an operand whose rows many tiles re-read: A (read once per 128-column tile) from N >= 256,
// B (read once per 256-row tile) from M >= 2048 (measured on MI355X: A alone is 5-25%
// faster than neither from M = 64 up; both are 1.4-2.3x faster from M = 2048 up, A alone
// up to M = 1024). Returns 0 (no pass), 1 (both operands) or 2 (A only).
// ROCKET_HIP_F32_PREPASS = 0 / 1 / 2 forces a choice (read per call). All give identical bits.
int f32_prepass(const Req &r)
{
    if (r.fa != Fmt::F32BF16 && r.fa != Fmt::F32TF32) return 0;
    if (const char *e = getenv("ROCKET_HIP_F32_PREPASS")) {
        if (e[0] >= '0' && e[0] <= '2' && e[1] == 0) return e[0] - '0';
    }
    int maxM = 0;
    for (int p = 0; p < r.nprob; p++) maxM = std::max(maxM, r.M[p]);
    if (r.N < 256) return 0;
    return (maxM >= 2048 && r.N >= 2048) ? 1 : 2;
}

int run(int fd, const Req &r)
{
    Locked L(fd);
    if (!L.ok()) {
        ROCKET_LOGE("%s: fd %d is not an open rocket handle\n", r.who, fd);
        return ROCKET_E_DEVICE;
    }
    if (r.nprob < 1) return ROCKET_E_SHAPE;
    const int nG = r.group ? r.K / r.group : 0;
    const bool gw = (r.epi == Epi::GW);
    // B as it arrives from the caller: int8 per value when we pack it ourselves
    const size_t brow_in = r.pack_b_int4 ? (size_t)r.K : fmt_row_bytes(r.fb, r.K);
    const int prepass = f32_prepass(r);
    const Fmt cvt = r.fa == Fmt::F32TF32 ? Fmt::BF16X2 : Fmt::BF16;
    const Fmt fa_dev = prepass ? cvt : r.fa;
    const Fmt fb_dev = r.pack_b_int4 ? Fmt::I4P : (prepass == 1 ? cvt : r.fb);

    // quantised-on-device activations: bytes per source element, and the pre-pass plan
    const size_t qa_bytes = r.quant_a == 1 ? 4 : (r.quant_a == 2 ? 2 : 0);
    if (qa_bytes && (!gw || !r.rowscale || r.fa != Fmt::I8 || r.K % 8)) return ROCKET_E_SHAPE;
    const bool glu_in = r.act != 0;
    if (glu_in && (!qa_bytes || !r.A2)) return ROCKET_E_SHAPE;
    if (r.f16out && !gw) return ROCKET_E_SHAPE;
    const size_t c_elem = r.f16out ? 2 : epi_elem_bytes(r.epi);
    const size_t a_row_in = qa_bytes ? qa_bytes * r.K : fmt_row_bytes(r.fa, r.K);

    Call c(L.h, r.who);
    for (int p = 0; p < r.nprob; p++) {
        const size_t M = (size_t)r.M[p];
        if (M == 0) continue;
        c.want(r.A[p], M * a_row_in);
        if (glu_in) c.want(r.A2[p], M * a_row_in);
        if (qa_bytes) {
            c.want_scratch(M * r.K);
            c.want_scratch(M * sizeof(float));
        }
        c.want(r.B[p], (size_t)r.N * brow_in);
        c.want(r.C[p], M * r.N * c_elem);
        if (gw) {
            if (!qa_bytes) c.want(r.a_scale[p], M * (r.rowscale ? 1 : nG) * sizeof(float));
            c.want(r.b_scale[p], (size_t)r.N * nG * sizeof(float));
        }
        if (r.pack_b_int4) c.want_scratch((size_t)r.N * r.K / 2);
        if (prepass) c.want_scratch(M * fmt_row_bytes(fa_dev, r.K));
        if (prepass == 1) c.want_scratch((size_t)r.N * fmt_row_bytes(fb_dev, r.K));
    }
    auto dump_of = [&](int p) -> int32_t * { return (r.dump && r.dump_rows[p] > 0) ? r.dump[p] : nullptr; };
    auto dump_bytes = [&](int p) { return (size_t)r.dump_rows[p] * nG * r.N * sizeof(int32_t); };
    for (int p = 0; p < r.nprob; p++)
        if (dump_of(p) && r.M[p]) c.want(dump_of(p), dump_bytes(p));
    // split-K workspace (plain int32, fp16 and fp32 results): the largest any launch of the
    // call needs; successive launches reuse it in stream order
    size_t ws = 0;
    if (r.epi == Epi::I32 || r.epi == Epi::F16 || r.epi == Epi::F32) {
        for (int p0 = 0; p0 < r.nprob; p0 += kMaxProblems) {
            Launch Lp;
            Lp.fmt_a = fa_dev; Lp.fmt_b = fb_dev; Lp.epi = r.epi; Lp.N = r.N; Lp.K = r.K;
            Lp.nprob = std::min(kMaxProblems, r.nprob - p0);
            for (int q = 0; q < Lp.nprob; q++) Lp.prob[q].M = r.M[p0 + q];
            Lp.kbeg = 0;
            Lp.kend = (r.kchunk > 0 && r.K > r.kchunk) ? r.kchunk : r.K;
            ws = std::max(ws, gemm_ws_bytes(Lp));
        }
        c.want_scratch(ws);
    }
    if (int rc = c.begin()) return rc;
    int32_t *wsp = ws ? static_cast<int32_t *>(c.scratch(ws)) : nullptr;

    // launches hold up to kMaxProblems problems each
    for (int p0 = 0; p0 < r.nprob; p0 += kMaxProblems) {
        // the launch's activations quantised per row first (one pre-pass launch)
        QuantRows qr;
        if (qa_bytes) {
            qr.n = std::min(kMaxProblems, r.nprob - p0);
            qr.K = r.K;
            qr.f16 = r.quant_a == 2;
            qr.act = r.act;
            for (int i = 0; i < qr.n; i++) {
                const int p = p0 + i;
                qr.M[i] = r.M[p];
                if (!qr.M[i]) continue;
                qr.A[i] = c.in(r.A[p], (size_t)qr.M[i] * a_row_in);
                if (glu_in) {
                    qr.A2[i] = c.in(r.A2[p], (size_t)qr.M[i] * a_row_in);
                    if (!qr.A2[i]) return c.finish();
                }
                qr.Aq[i] = static_cast<int8_t *>(c.scratch((size_t)qr.M[i] * r.K));
                qr.row_scale[i] = static_cast<float *>(c.scratch((size_t)qr.M[i] * sizeof(float)));
                if (!qr.A[i] || !qr.Aq[i] || !qr.row_scale[i]) return c.finish();
            }
            uint64_t qb = 0;
            if (quant_rows(qr, c.stream(), &qb) != hipSuccess) {
                (void)hipGetLastError();
                ROCKET_LOGE("%s: activation quantisation launch rejected\n", r.who);
                (void)c.finish();
                return ROCKET_E_DEVICE;
            }
            count_launch(qb);
        }
        Launch Lc;
        Lc.fmt_a = fa_dev;
        Lc.fmt_b = fb_dev;
        Lc.epi = r.epi;
        Lc.N = r.N;
        Lc.K = r.K;
        Lc.group = r.group;
        Lc.rowscale = r.rowscale;
        Lc.f16out = r.f16out ? 1 : 0;
        Lc.kt = gw ? gw_period(r.group) : 0;
        Lc.ws = wsp;
        Lc.ws_bytes = wsp ? ws : 0;
        Lc.nprob = std::min(kMaxProblems, r.nprob - p0);
        for (int q = 0; q < Lc.nprob; q++) {
            const int p = p0 + q;
            Problem &P = Lc.prob[q];
            P.M = r.M[p];
            P.B2 = nullptr;
            if (P.M == 0) { P.A = P.B = nullptr; P.C = nullptr; P.a_scale = P.b_scale = nullptr; continue; }
            P.A = qa_bytes ? qr.Aq[q] : c.in(r.A[p], (size_t)P.M * fmt_row_bytes(r.fa, r.K));
            const void *b = c.in(r.B[p], (size_t)r.N * brow_in);
            if (r.pack_b_int4 && b) {
                void *packed = c.scratch((size_t)r.N * r.K / 2);
                if (packed) {
                    if (pack_int4(static_cast<const int8_t *>(b), static_cast<uint8_t *>(packed), r.N, r.K,
                                  c.stream()) != hipSuccess) {
                        (void)hipGetLastError();
                        ROCKET_LOGE("%s: int4 pack launch failed\n", r.who);
                        return ROCKET_E_DEVICE;
                    }
                    count_launch((uint64_t)(((size_t)r.N * r.K / 8 + 255) / 256));
                }
                b = packed;
            }
            P.B = b;
            if (prepass && P.A && P.B) {
                const bool ok = prepass == 1
                                    ? convert(c, P.A, (size_t)P.M * r.K, fa_dev, &P.A, P.B, (size_t)r.N * r.K, &P.B)
                                    : convert(c, P.A, (size_t)P.M * r.K, fa_dev, &P.A);
                if (!ok) {
                    const int e = c.finish();
                    return e ? e : ROCKET_E_DEVICE;
                }
            }
            P.C = c.out(r.C[p], (size_t)P.M * r.N * c_elem);
            P.a_scale = !gw ? nullptr
                        : qa_bytes ? qr.row_scale[q]
                                   : static_cast<const float *>(
                                         c.in(r.a_scale[p], (size_t)P.M * (r.rowscale ? 1 : nG) * sizeof(float)));
            P.b_scale = gw ? static_cast<const float *>(c.in(r.b_scale[p], (size_t)r.N * nG * sizeof(float))) : nullptr;
            if (!P.A || !P.B || !P.C || (gw && (!P.a_scale || !P.b_scale))) return c.finish();
            if (dump_of(p)) {
                P.dump = static_cast<int32_t *>(c.out(dump_of(p), dump_bytes(p)));
                P.dump_row0 = r.dump_row0[p];
                P.dump_rows = r.dump_rows[p];
                if (!P.dump) return c.finish();
            }
        }
        if (r.kchunk > 0 && r.K > r.kchunk) {
            for (int k0 = 0; k0 < r.K; k0 += r.kchunk) {
                Lc.kbeg = k0;
                Lc.kend = std::min(r.K, k0 + r.kchunk);
                Lc.accum = k0 > 0;
                if (c.launch(Lc)) return c.finish();
            }
        } else {
            Lc.kbeg = 0;
            Lc.kend = r.K;
            if (c.launch(Lc)) return c.finish();
        }
    }
    return c.finish();
}

}  // namespace rk

using namespace rk;

namespace {

bool dims_ok(int M, int K, int N)
{
    return M > 0 && K > 0 && N > 0 && M <= kDimMax && K <= kDimMax && N <= kDimMax;
}

// Shared planner body: the reference's alignment test, then the MI355X workgroup tiling.
int plan(int M, int K, int N, int kal, int nal, Fmt fa, Epi epi, int kt, int *pMt, int *pKt, int *pNt)
{
    if (!dims_ok(M, K, N) || K % kal || N % nal || M % 4) return ROCKET_E_SHAPE;
    int bm, bn;
    gemm_tile(fa, epi, M, N, &bm, &bn);
    const long count = (long)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    if (count > 0x7FFFFFFFL) return ROCKET_E_SHAPE;
    if (pMt) *pMt = std::min(M, bm);
    if (pNt) *pNt = std::min(N, bn);
    if (pKt) *pKt = kt ? kt : K;
    return (int)count;
}

// M==1 is accepted by the one-shot entries (the reference pads it to a 4-row tile,
// rocket_matmul.c:258-267; the kernels here take any M, so the single row is computed
// directly and equals row 0 of the padded product). Other M go through the planner.
int oneshot_shape(int M, int K, int N, int kal, int nal)
{
    if (M == 1) return (dims_ok(1, K, N) && K % kal == 0 && N % nal == 0) ? 0 : ROCKET_E_SHAPE;
    return plan(M, K, N, kal, nal, Fmt::I8, Epi::I32, 0, nullptr, nullptr, nullptr) < 0 ? ROCKET_E_SHAPE : 0;
}

bool dtype_ok(int precision)
{
    return rocket_hw_dtype_supported(rocket_hw_current(), precision);
}

int single(int fd, const char *who, Fmt fa, Fmt fb, Epi epi, int M, int K, int N,
           const void *A, const void *B, void *C)
{
    if (!A || !B || !C) {
        ROCKET_LOGE("%s: NULL operand\n", who);
        return ROCKET_E_SHAPE;
    }
    Req r;
    r.who = who; r.fa = fa; r.fb = fb; r.epi = epi; r.K = K; r.N = N;
    r.M = &M; r.A = &A; r.B = &B; r.C = &C;
    return run(fd, r);
}

}  // namespace

extern "C" {

// ---- planners ----------------------------------------------------------------------
int rocket_matmul_plan(int M, int K, int N, int *Mt, int *Kt, int *Nt)
{   // reference rocket_matmul.c:498-568: K%32, N%16, M%4, 0 < dims <= 2^24
    return plan(M, K, N, 32, 16, Fmt::F16, Epi::F16, 0, Mt, Kt, Nt);
}

int rocket_matmul_plan_int8(int M, int K, int N, int *Mt, int *Kt, int *Nt)
{   // reference rocket_matmul.c:2383-2437: K%32, N%32, M%4
    return plan(M, K, N, 32, 32, Fmt::I8, Epi::I32, 0, Mt, Kt, Nt);
}

int rocket_matmul_plan_int8_gw(int M, int K, int N, int group, int *Mt, int *Kt, int *Nt)
{   // reference rocket_matmul.c:2671-2714: + group >= 32, group%32, K%group; Kt | group
    if (!dims_ok(M, K, N) || K % 32 || N % 32 || M % 4) return ROCKET_E_SHAPE;
    if (group < 32 || group % 32 || K % group) return ROCKET_E_SHAPE;
    return plan(M, K, N, 32, 32, Fmt::I8, Epi::GW, gw_period(group), Mt, Kt, Nt);
}

int rocket_matmul_plan_int4(int M, int K, int N, int *Mt, int *Kt, int *Nt)
{   // reference rocket_matmul.c:2917-2956: K%32, N%64, M%4
    return plan(M, K, N, 32, 64, Fmt::I8, Epi::I32, 0, Mt, Kt, Nt);
}

int rocket_matmul_plan_int16(int M, int K, int N, int *Mt, int *Kt, int *Nt)
{   // reference rocket_matmul.c:3320-3359: K%32, N%16, M%4
    return plan(M, K, N, 32, 16, Fmt::I16, Epi::I64, 0, Mt, Kt, Nt);
}

int rocket_matmul_plan_bf16(int M, int K, int N, int *Mt, int *Kt, int *Nt)
{   // reference rocket_matmul.c:3448-3452: the int16 geometry and alignment
    return plan(M, K, N, 32, 16, Fmt::F32BF16, Epi::F32, 0, Mt, Kt, Nt);
}

int rocket_matmul_plan_tf32(int M, int K, int N, int *Mt, int *Kt, int *Nt)
{   // reference rocket_matmul.c:3797-3838: K%16, N%16, M%4
    return plan(M, K, N, 16, 16, Fmt::F32TF32, Epi::F32, 0, Mt, Kt, Nt);
}

// ---- fp16 ----------------------------------------------------------------------------
int rocket_matmul_fp16(int fd, int M, int K, int N, const _Float16 *A, const _Float16 *B, _Float16 *C)
{   // reference rocket_matmul.c:1945-1998
    if (!dtype_ok(precision_float16)) return ROCKET_E_UNSUPPORTED;
    if (oneshot_shape(M, K, N, 32, 16)) {
        ROCKET_LOGE("rocket_matmul_fp16: unsupported shape M=%d K=%d N=%d (need K%%32, N%%16, M%%4||1)\n", M, K, N);
        return ROCKET_E_SHAPE;
    }
    return single(fd, "rocket_matmul_fp16", Fmt::F16, Fmt::F16, Epi::F16, M, K, N, A, B, C);
}

int rocket_matmul_fp16_f32out(int fd, int M, int K, int N, const _Float16 *A, const _Float16 *B, float *C)
{   // reference rocket_matmul.c:3620-3758
    if (!dtype_ok(precision_float16)) return ROCKET_E_UNSUPPORTED;
    if (oneshot_shape(M, K, N, 32, 16)) {
        ROCKET_LOGE("rocket_matmul_fp16_f32out: unsupported shape M=%d K=%d N=%d (need K%%32, N%%16, M%%4||1)\n", M, K, N);
        return ROCKET_E_SHAPE;
    }
    return single(fd, "rocket_matmul_fp16_f32out", Fmt::F16, Fmt::F16, Epi::F32, M, K, N, A, B, C);
}

int rocket_matmul_fp16_batch(int fd, int M, int K, int N, int nbatch,
                             const _Float16 *const *A, const _Float16 *const *B, _Float16 *const *C)
{   // reference rocket_matmul.c:2042-2310: M%4, K%32, N%16; nbatch==1 -> rocket_matmul_fp16
    if (nbatch < 1 || !A || !B || !C) return ROCKET_E_SHAPE;
    if (nbatch == 1) return rocket_matmul_fp16(fd, M, K, N, A[0], B[0], C[0]);
    if (plan(M, K, N, 32, 16, Fmt::F16, Epi::F16, 0, nullptr, nullptr, nullptr) < 0) {
        ROCKET_LOGE("rocket_matmul_fp16_batch: unsupported shape M=%d K=%d N=%d (need M%%4, K%%32, N%%16)\n", M, K, N);
        return ROCKET_E_SHAPE;
    }
    for (int i = 0; i < nbatch; i++)
        if (!A[i] || !B[i] || !C[i]) return ROCKET_E_SHAPE;
    std::vector<int> Ms(nbatch, M);
    Req r;
    r.who = "rocket_matmul_fp16_batch"; r.fa = r.fb = Fmt::F16; r.epi = Epi::F16;
    r.K = K; r.N = N; r.nprob = nbatch; r.M = Ms.data();
    r.A = reinterpret_cast<const void *const *>(A);
    r.B = reinterpret_cast<const void *const *>(B);
    r.C = reinterpret_cast<void *const *>(C);
    return run(fd, r);
}

// ---- int8 ----------------------------------------------------------------------------
int rocket_matmul_int8(int fd, int M, int K, int N, const int8_t *A, const int8_t *B, int32_t *C)
{   // reference rocket_matmul.c:2439-2627
    if (!dtype_ok(precision_int8)) return ROCKET_E_UNSUPPORTED;
    if (oneshot_shape(M, K, N, 32, 32)) {
        ROCKET_LOGE("rocket_matmul_int8: unsupported shape M=%d K=%d N=%d (need K%%32, N%%32, M%%4||1)\n", M, K, N);
        return ROCKET_E_SHAPE;
    }
    return single(fd, "rocket_matmul_int8", Fmt::I8, Fmt::I8, Epi::I32, M, K, N, A, B, C);
}

static int gw_common(int fd, const char *who, bool b_int4, int M, int K, int N,
                     const int8_t *A, const int8_t *B, const float *as, const float *bs,
                     float *Cf, int group, int32_t *dump, int row0, int nrows, bool rowscale = false)
{
    if (!A || !B || !as || !bs || !Cf) { ROCKET_LOGE("%s: NULL operand\n", who); return ROCKET_E_SHAPE; }
    Req r;
    const void *a = A, *b = B;
    void *c = Cf;
    r.who = who; r.fa = Fmt::I8; r.fb = b_int4 ? Fmt::I4P : Fmt::I8; r.pack_b_int4 = b_int4;
    r.epi = Epi::GW; r.K = K; r.N = N; r.M = &M; r.A = &a; r.B = &b; r.C = &c;
    r.a_scale = &as; r.b_scale = &bs; r.group = group;
    r.dump = &dump; r.dump_row0 = &row0; r.dump_rows = &nrows;
    r.rowscale = rowscale;
    return run(fd, r);
}

int rocket_matmul_int8_groupwise(int fd, int M, int K, int N, const int8_t *A, const int8_t *B,
                                 const float *a_scale, const float *b_scale, float *Cf, int group)
{   // reference rocket_matmul.c:2716-2871 (no M==1 pad: M%4)
    if (!dtype_ok(precision_int8)) return ROCKET_E_UNSUPPORTED;
    if (rocket_matmul_plan_int8_gw(M, K, N, group, nullptr, nullptr, nullptr) < 0) {
        ROCKET_LOGE("rocket_matmul_int8_groupwise: unsupported shape M=%d K=%d N=%d group=%d "
                    "(need K%%32, N%%32, M%%4, group%%32, group|K)\n", M, K, N, group);
        return ROCKET_E_SHAPE;
    }
    return gw_common(fd, "rocket_matmul_int8_groupwise", false, M, K, N, A, B, a_scale, b_scale, Cf,
                     group, nullptr, 0, 0);
}

// ---- int4 ----------------------------------------------------------------------------
int rocket_matmul_int4_ex(int fd, int M, int K, int N, const int8_t *A, const int8_t *B, int32_t *C, int kt_cap)
{   // reference rocket_matmul.c:2958-3114. kt_cap bounded the NPU's int16 K-tile readback;
    // the int32 accumulation here is exact for every kt_cap, so it does not change C.
    (void)kt_cap;
    if (!dtype_ok(precision_int4)) return ROCKET_E_UNSUPPORTED;
    if (oneshot_shape(M, K, N, 32, 64)) {
        ROCKET_LOGE("rocket_matmul_int4: unsupported shape M=%d K=%d N=%d (need K%%32, N%%64, M%%4||1)\n", M, K, N);
        return ROCKET_E_SHAPE;
    }
    if (!A || !B || !C) return ROCKET_E_SHAPE;
    Req r;
    const void *a = A, *b = B;
    void *c = C;
    r.who = "rocket_matmul_int4"; r.fa = Fmt::I8; r.fb = Fmt::I4P; r.pack_b_int4 = true;
    r.epi = Epi::I32; r.K = K; r.N = N; r.M = &M; r.A = &a; r.B = &b; r.C = &c;
    r.kchunk = 65536;   // the x16 int4 accumulators stay exact below 2^17 products of int8 x int4
    return run(fd, r);
}

int rocket_matmul_int4(int fd, int M, int K, int N, const int8_t *A, const int8_t *B, int32_t *C)
{
    return rocket_matmul_int4_ex(fd, M, K, N, A, B, C, 0);
}

int rocket_matmul_int4_groupwise(int fd, int M, int K, int N, const int8_t *A, const int8_t *B,
                                 const float *a_scale, const float *b_scale, float *Cf, int group)
{   // reference rocket_matmul.c:3132-3282
    if (!dtype_ok(precision_int4)) return ROCKET_E_UNSUPPORTED;
    if (group < 32 || group % 32 || K % group || M % 4 || 49 * group >= 32767) {
        ROCKET_LOGE("rocket_matmul_int4_groupwise: bad group=%d (need %%32, |K, 49*group<32767, M%%4) K=%d M=%d\n",
                    group, K, M);
        return ROCKET_E_SHAPE;
    }
    if (rocket_matmul_plan_int4(M, K, N, nullptr, nullptr, nullptr) < 0) {
        ROCKET_LOGE("rocket_matmul_int4_groupwise: unsupported shape M=%d K=%d N=%d\n", M, K, N);
        return ROCKET_E_SHAPE;
    }
    return gw_common(fd, "rocket_matmul_int4_groupwise", true, M, K, N, A, B, a_scale, b_scale, Cf,
                     group, nullptr, 0, 0);
}

// ---- per-row activation scales (rocket_hip.h) ------------------------------------------
int rocket_matmul_int8_groupwise_rowscale(int fd, int M, int K, int N, const int8_t *A, const int8_t *B,
                                          const float *a_row_scale, const float *b_scale, float *Cf, int group)
{   // validation of rocket_matmul_int8_groupwise
    if (!dtype_ok(precision_int8)) return ROCKET_E_UNSUPPORTED;
    if (rocket_matmul_plan_int8_gw(M, K, N, group, nullptr, nullptr, nullptr) < 0) {
        ROCKET_LOGE("rocket_matmul_int8_groupwise_rowscale: unsupported shape M=%d K=%d N=%d group=%d\n", M, K, N,
                    group);
        return ROCKET_E_SHAPE;
    }
    return gw_common(fd, "rocket_matmul_int8_groupwise_rowscale", false, M, K, N, A, B, a_row_scale, b_scale, Cf,
                     group, nullptr, 0, 0, true);
}

int rocket_matmul_int4_groupwise_rowscale(int fd, int M, int K, int N, const int8_t *A, const int8_t *B,
                                          const float *a_row_scale, const float *b_scale, float *Cf, int group)
{   // validation of rocket_matmul_int4_groupwise
    if (!dtype_ok(precision_int4)) return ROCKET_E_UNSUPPORTED;
    if (group < 32 || group % 32 || K % group || M % 4 || 49 * group >= 32767 ||
        rocket_matmul_plan_int4(M, K, N, nullptr, nullptr, nullptr) < 0) {
        ROCKET_LOGE("rocket_matmul_int4_groupwise_rowscale: unsupported shape M=%d K=%d N=%d group=%d\n", M, K, N,
                    group);
        return ROCKET_E_SHAPE;
    }
    return gw_common(fd, "rocket_matmul_int4_groupwise_rowscale", true, M, K, N, A, B, a_row_scale, b_scale, Cf,
                     group, nullptr, 0, 0, true);
}

// ---- int16 exact ---------------------------------------------------------------------
int rocket_matmul_int16_exact(int fd, int M, int K, int N, const int16_t *A, const int16_t *B, int64_t *C)
{   // reference rocket_matmul.c:3377-3421 (int8 alignment: K%32, N%32, M%4||1)
    if (!dtype_ok(precision_int8)) return ROCKET_E_UNSUPPORTED;
    if (oneshot_shape(M, K, N, 32, 32)) {
        ROCKET_LOGE("rocket_matmul_int16_exact: unsupported shape M=%d K=%d N=%d (need K%%32, N%%32, M%%4||1)\n", M, K, N);
        return ROCKET_E_SHAPE;
    }
    if (!A || !B || !C) return ROCKET_E_SHAPE;
    Req r;
    const void *a = A, *b = B;
    void *c = C;
    r.who = "rocket_matmul_int16_exact"; r.fa = r.fb = Fmt::I16; r.epi = Epi::I64;
    r.K = K; r.N = N; r.M = &M; r.A = &a; r.B = &b; r.C = &c;
    r.kchunk = 32768;   // every int32 byte-plane accumulator stays below 2^31
    return run(fd, r);
}

// ---- bf16 / tf32 ---------------------------------------------------------------------
int rocket_matmul_bf16(int fd, int M, int K, int N, const float *A, const float *B, float *C)
{   // reference rocket_matmul.c:3454-3596
    if (!dtype_ok(precision_bfloat16)) return ROCKET_E_UNSUPPORTED;
    if (oneshot_shape(M, K, N, 32, 16)) {
        ROCKET_LOGE("rocket_matmul_bf16: unsupported shape M=%d K=%d N=%d (need K%%32, N%%16, M%%4||1)\n", M, K, N);
        return ROCKET_E_SHAPE;
    }
    return single(fd, "rocket_matmul_bf16", Fmt::F32BF16, Fmt::F32BF16, Epi::F32, M, K, N, A, B, C);
}

int rocket_matmul_tf32(int fd, int M, int K, int N, const float *A, const float *B, float *C)
{   // reference rocket_matmul.c:3840-3982
    if (!dtype_ok(precision_tf32)) return ROCKET_E_UNSUPPORTED;
    if (oneshot_shape(M, K, N, 16, 16)) {
        ROCKET_LOGE("rocket_matmul_tf32: unsupported shape M=%d K=%d N=%d (need K%%16, N%%16, M%%4||1)\n", M, K, N);
        return ROCKET_E_SHAPE;
    }
    return single(fd, "rocket_matmul_tf32", Fmt::F32TF32, Fmt::F32TF32, Epi::F32, M, K, N, A, B, C);
}

// ---- RK3576 entries: a different chip's requantising contract -------------------------
int rocket_matmul_plan_int8_rk3576(int M, int K, int N, int *Mt, int *Kt, int *Nt)
{
    (void)M; (void)K; (void)N; (void)Mt; (void)Kt; (void)Nt;
    return ROCKET_E_UNSUPPORTED;
}
int rocket_matmul_int8_rk3576(int fd, int M, int K, int N, const int8_t *A, const int8_t *B,
                              const int32_t *bias, float scale, int8_t *C)
{
    (void)fd; (void)M; (void)K; (void)N; (void)A; (void)B; (void)bias; (void)scale; (void)C;
    return ROCKET_E_UNSUPPORTED;
}
int rocket_matmul_int8_rk3576_perc(int fd, int M, int K, int N, const int8_t *A, const int8_t *B,
                                   const int32_t *bias, const float *scale_n, int8_t *C, double *worst_rel_err)
{
    (void)fd; (void)M; (void)K; (void)N; (void)A; (void)B; (void)bias; (void)scale_n; (void)C; (void)worst_rel_err;
    return ROCKET_E_UNSUPPORTED;
}
int rocket_matmul_int8_rk3576_perc_sa(int fd, int M, int K, int N, const int8_t *A, const int8_t *B,
                                      const int32_t *bias, const float *scale_n, const int64_t *sum_abs_w,
                                      int8_t *C, double *worst_rel_err)
{
    (void)fd; (void)M; (void)K; (void)N; (void)A; (void)B; (void)bias; (void)scale_n; (void)sum_abs_w;
    (void)C; (void)worst_rel_err;
    return ROCKET_E_UNSUPPORTED;
}
int rocket_rk3576_wbo_create(int fd, int K, int N, const int8_t *B, struct rocket_rk3576_wbo **out)
{
    (void)fd; (void)K; (void)N; (void)B;
    if (out) *out = nullptr;
    return ROCKET_E_UNSUPPORTED;
}
void rocket_rk3576_wbo_free(int fd, struct rocket_rk3576_wbo *w) { (void)fd; (void)w; }
int rocket_matmul_int8_rk3576_perc_wbo(int fd, int M, int K, int N, const int8_t *A,
                                       const struct rocket_rk3576_wbo *wbo, const int32_t *bias,
                                       const float *scale_n, const int64_t *sum_abs_w, int8_t *C,
                                       double *worst_rel_err)
{
    (void)fd; (void)M; (void)K; (void)N; (void)A; (void)wbo; (void)bias; (void)scale_n; (void)sum_abs_w;
    (void)C; (void)worst_rel_err;
    return ROCKET_E_UNSUPPORTED;
}
void rocket_rk3576_bo_pool_drain(int fd) { (void)fd; }
int rocket_matmul_int8_rk3576_i32(int fd, int M, int K, int N, const int8_t *A, const int8_t *B,
                                  const int32_t *bias, int32_t *C)
{
    (void)fd; (void)M; (void)K; (void)N; (void)A; (void)B; (void)bias; (void)C;
    return ROCKET_E_UNSUPPORTED;
}
void rocket_rk3576_i32_last_stats(rocket_rk3576_i32_stats *out)
{
    if (out) memset(out, 0, sizeof(*out));
}

}  // extern "C"
