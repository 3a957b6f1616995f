/*
 * oracle.c — CPU restatement of the reference host arithmetic for the matmul path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): used by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg as the checker and as the timed CPU baseline; never by
 * the library. Built by oracle/Makefile with gcc -O3 -fopenmp into oracle/liboracle.so.
 *
 * Parity pins for every function here live in tests/test_oracle.py (closed forms,
 * exhaustive sweeps, numpy's independent routines, brute force on tiny shapes and the
 * committed fixtures under tests/golden/).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------
 * Generators. splitmix64 as used by tests/matmul_correctness_matrix_rocket.c:50-61
 * (Steele, Lea & Flood 2014: state += 0x9E3779B97F4A7C15, then the variant-13 mixer).
 * ---------------------------------------------------------------------------------- */
static inline uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

uint64_t rko_splitmix64_next(uint64_t *state)
{
    *state += 0x9E3779B97F4A7C15ULL;
    return mix64(*state);
}

uint64_t rko_splitmix64_at(uint64_t seed, uint64_t i)
{
    return mix64(seed + (i + 1) * 0x9E3779B97F4A7C15ULL);
}

/* integer in [lo, hi] from the high 32 bits by multiply-shift (bias < 2^-24 here) */
static inline int64_t draw_int(uint64_t r, int lo, int hi)
{
    uint64_t span = (uint64_t)((int64_t)hi - lo + 1);
    return (int64_t)lo + (int64_t)(((r >> 32) * span) >> 32);
}

/* uniform in [0,1) with 24 random bits (exactly representable in fp32) */
static inline double draw_u01(uint64_t r) { return (double)(r >> 40) * (1.0 / 16777216.0); }

void rko_gen_i8(int8_t *out, size_t n, uint64_t seed, int lo, int hi)
{
    #pragma omp parallel for schedule(static) if (n > 65536)
    for (size_t i = 0; i < n; i++) out[i] = (int8_t)draw_int(rko_splitmix64_at(seed, i), lo, hi);
}

void rko_gen_i16(int16_t *out, size_t n, uint64_t seed, int lo, int hi)
{
    #pragma omp parallel for schedule(static) if (n > 65536)
    for (size_t i = 0; i < n; i++) out[i] = (int16_t)draw_int(rko_splitmix64_at(seed, i), lo, hi);
}

void rko_gen_f32_uniform(float *out, size_t n, uint64_t seed, float lo, float hi)
{
    #pragma omp parallel for schedule(static) if (n > 65536)
    for (size_t i = 0; i < n; i++)
        out[i] = (float)((double)lo + ((double)hi - (double)lo) * draw_u01(rko_splitmix64_at(seed, i)));
}

/* Box–Muller on outputs 2i and 2i+1; u1 is shifted into (0,1] so log() is finite. */
void rko_gen_f32_normal(float *out, size_t n, uint64_t seed, float mean, float std)
{
    #pragma omp parallel for schedule(static) if (n > 65536)
    for (size_t i = 0; i < n; i++) {
        double u1 = ((double)(rko_splitmix64_at(seed, 2 * i) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        double u2 = (double)(rko_splitmix64_at(seed, 2 * i + 1) >> 11) * (1.0 / 9007199254740992.0);
        double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925 * u2);
        out[i] = (float)((double)mean + (double)std * z);
    }
}

/* ------------------------------------------------------------------------------------
 * Conversions.
 * ---------------------------------------------------------------------------------- */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE 754 binary32 -> binary16, round to nearest, ties to even. */
uint16_t rko_f32_to_f16(float f)
{
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u)                       /* inf / nan (nan stays quiet nan) */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? (0x200u | ((ax >> 13) & 0x3FFu)) : 0u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);   /* >= 65520 rounds to inf */
    if (ax >= 0x38800000u) {                                  /* normal in binary16 */
        uint32_t m = ax - (112u << 23);                        /* rebias 127 -> 15 */
        uint32_t q = m >> 13, rem = m & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    if (ax <= 0x33000000u) return sign;                        /* <= 2^-25 rounds to 0 */
    {                                                         /* binary16 subnormal */
        int e = (int)(ax >> 23);
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        int shift = 126 - e;                                   /* 14..24 */
        uint32_t q = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
}

float rko_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0x1Fu) return u2f(sign | 0x7F800000u | (m << 13));
    if (e == 0) {
        if (m == 0) return u2f(sign);
        float v = (float)m * (1.0f / 16777216.0f);             /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

void rko_f32_to_f16_n(const float *in, uint16_t *out, size_t n)
{
    #pragma omp parallel for schedule(static) if (n > 65536)
    for (size_t i = 0; i < n; i++) out[i] = rko_f32_to_f16(in[i]);
}

void rko_f16_to_f32_n(const uint16_t *in, float *out, size_t n)
{
    #pragma omp parallel for schedule(static) if (n > 65536)
    for (size_t i = 0; i < n; i++) out[i] = rko_f16_to_f32(in[i]);
}

uint16_t rko_f32_to_bf16_trunc(float f) { return (uint16_t)(f2u(f) >> 16); }
float    rko_bf16_to_f32(uint16_t b)    { return u2f((uint32_t)b << 16); }
float    rko_tf32_trunc(float f)        { return u2f(f2u(f) & 0xFFFFE000u); }

void rko_int16_split(int16_t x, int8_t *hi, int8_t *lo)
{
    int v = x;
    if (v > 32639) v = 32639;
    if (v < -32768) v = -32768;
    int l = ((v + 128) & 0xFF) - 128;
    *lo = (int8_t)l;
    *hi = (int8_t)((v - l) >> 8);
}

/* ------------------------------------------------------------------------------------
 * References. Rows are independent, so every routine is parallel over m.
 * ---------------------------------------------------------------------------------- */

void rko_matmul_fp16(int M, int K, int N, const uint16_t *A, const uint16_t *B, uint16_t *C)
{
    float *Bf = malloc((size_t)N * K * sizeof(float));
    if (!Bf) return;
    rko_f16_to_f32_n(B, Bf, (size_t)N * K);
    #pragma omp parallel
    {
        float *a = malloc((size_t)K * sizeof(float));
        #pragma omp for schedule(static)
        for (int m = 0; m < M; m++) {
            for (int k = 0; k < K; k++) a[k] = rko_f16_to_f32(A[(size_t)m * K + k]);
            for (int n = 0; n < N; n++) {
                const float *b = Bf + (size_t)n * K;
                float s = 0.0f;
                for (int k = 0; k < K; k++) s += a[k] * b[k];   /* sequential fp32 sum */
                C[(size_t)m * N + n] = rko_f32_to_f16(s);
            }
        }
        free(a);
    }
    free(Bf);
}

/* The reference tests' own host loop (tests/matmul_fp16_rocket.c:43-50): one thread, each
 * operand converted from fp16 where it is read, an fp32 sum over k, fp16 out. Same results as
 * rko_matmul_fp16; it is timed as the comparability row of the CPU baseline. */
void rko_matmul_fp16_naive(int M, int K, int N, const uint16_t *A, const uint16_t *B, uint16_t *C)
{
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++) {
            float s = 0.0f;
            for (int l = 0; l < K; l++)
                s += rko_f16_to_f32(A[(size_t)i * K + l]) * rko_f16_to_f32(B[(size_t)j * K + l]);
            C[(size_t)i * N + j] = rko_f32_to_f16(s);
        }
}

void rko_matmul_fp16_f32out(int M, int K, int N, const uint16_t *A, const uint16_t *B, float *C)
{
    float *Bf = malloc((size_t)N * K * sizeof(float));
    if (!Bf) return;
    rko_f16_to_f32_n(B, Bf, (size_t)N * K);
    #pragma omp parallel
    {
        float *a = malloc((size_t)K * sizeof(float));
        #pragma omp for schedule(static)
        for (int m = 0; m < M; m++) {
            for (int k = 0; k < K; k++) a[k] = rko_f16_to_f32(A[(size_t)m * K + k]);
            for (int n = 0; n < N; n++) {
                const float *b = Bf + (size_t)n * K;
                double s = 0.0;
                for (int k = 0; k < K; k++) s += (double)a[k] * (double)b[k];
                C[(size_t)m * N + n] = (float)s;
            }
        }
        free(a);
    }
    free(Bf);
}

/* exact int8 dot product: int32 partial sums over chunks of 2^16 terms cannot overflow
 * (|a*b| <= 2^14), then widened into int64 */
static inline int64_t dot_i8(const int8_t *a, const int8_t *b, int K)
{
    int64_t s = 0;
    for (int k0 = 0; k0 < K; k0 += 65536) {
        int k1 = K - k0 < 65536 ? K : k0 + 65536;
        int32_t p = 0;
        for (int k = k0; k < k1; k++) p += (int32_t)a[k] * (int32_t)b[k];
        s += p;
    }
    return s;
}

void rko_matmul_int8(int M, int K, int N, const int8_t *A, const int8_t *B, int32_t *C)
{
    #pragma omp parallel for schedule(static)
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++)
            C[(size_t)m * N + n] = (int32_t)(uint32_t)(uint64_t)
                dot_i8(A + (size_t)m * K, B + (size_t)n * K, K);
}

void rko_matmul_int16_exact(int M, int K, int N, const int16_t *A, const int16_t *B, int64_t *C)
{
    #pragma omp parallel
    {
        int32_t *a = malloc((size_t)K * sizeof(int32_t));
        #pragma omp for schedule(static)
        for (int m = 0; m < M; m++) {
            for (int k = 0; k < K; k++) {
                int v = A[(size_t)m * K + k];
                a[k] = v > 32639 ? 32639 : v;                 /* -32768 is already the floor */
            }
            for (int n = 0; n < N; n++) {
                const int16_t *b = B + (size_t)n * K;
                int64_t s = 0;
                for (int k = 0; k < K; k++) {
                    int v = b[k] > 32639 ? 32639 : b[k];
                    s += (int64_t)a[k] * (int64_t)v;
                }
                C[(size_t)m * N + n] = s;
            }
        }
        free(a);
    }
}

void rko_gw_partials(int M, int K, int N, int group, const int8_t *A, const int8_t *B, int32_t *P)
{
    const int nG = K / group;
    #pragma omp parallel for schedule(static)
    for (int m = 0; m < M; m++)
        for (int g = 0; g < nG; g++)
            for (int n = 0; n < N; n++)
                P[((size_t)m * nG + g) * N + n] = (int32_t)(uint32_t)(uint64_t)
                    dot_i8(A + (size_t)m * K + (size_t)g * group,
                           B + (size_t)n * K + (size_t)g * group, group);
}

void rko_matmul_gw_f32(int M, int K, int N, int group, const int8_t *A, const int8_t *B,
                       const float *a_scale, const float *b_scale, float *Cf)
{
    const int nG = K / group;
    #pragma omp parallel for schedule(static)
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float acc = 0.0f;
            for (int g = 0; g < nG; g++) {
                int32_t p = (int32_t)dot_i8(A + (size_t)m * K + (size_t)g * group,
                                            B + (size_t)n * K + (size_t)g * group, group);
                float s = a_scale[(size_t)m * nG + g] * b_scale[(size_t)n * nG + g];
                acc = fmaf(s, (float)p, acc);
            }
            Cf[(size_t)m * N + n] = acc;
        }
}

void rko_matmul_gw_rowscale_f32(int M, int K, int N, int group, const int8_t *A, const int8_t *B,
                                const float *a_row, const float *b_scale, float *Cf)
{
    const int nG = K / group;
    #pragma omp parallel for schedule(static)
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float acc = 0.0f;
            for (int g = 0; g < nG; g++) {
                int32_t p = (int32_t)dot_i8(A + (size_t)m * K + (size_t)g * group,
                                            B + (size_t)n * K + (size_t)g * group, group);
                acc = fmaf(b_scale[(size_t)n * nG + g], (float)p, acc);
            }
            Cf[(size_t)m * N + n] = a_row[m] * acc;
        }
}

void rko_matmul_gw_f64(int M, int K, int N, int group, const int8_t *A, const int8_t *B,
                       const float *a_scale, const float *b_scale, double *Cd)
{
    const int nG = K / group;
    #pragma omp parallel for schedule(static)
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            double acc = 0.0;
            for (int g = 0; g < nG; g++) {
                int64_t p = dot_i8(A + (size_t)m * K + (size_t)g * group,
                                   B + (size_t)n * K + (size_t)g * group, group);
                acc += (double)a_scale[(size_t)m * nG + g] *
                       (double)b_scale[(size_t)n * nG + g] * (double)p;
            }
            Cd[(size_t)m * N + n] = acc;
        }
}

/* double-accumulated product of two fp32 matrices after an elementwise transform */
typedef float (*xform_fn)(float);
static float id_f(float f)   { return f; }
static float bf16_f(float f) { return rko_bf16_to_f32(rko_f32_to_bf16_trunc(f)); }

static void matmul_f64acc(int M, int K, int N, const float *A, const float *B, float *C, xform_fn t)
{
    double *Bd = malloc((size_t)N * K * sizeof(double));
    if (!Bd) return;
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < (size_t)N * K; i++) Bd[i] = (double)t(B[i]);
    #pragma omp parallel
    {
        double *a = malloc((size_t)K * sizeof(double));
        #pragma omp for schedule(static)
        for (int m = 0; m < M; m++) {
            for (int k = 0; k < K; k++) a[k] = (double)t(A[(size_t)m * K + k]);
            for (int n = 0; n < N; n++) {
                const double *b = Bd + (size_t)n * K;
                double s = 0.0;
                for (int k = 0; k < K; k++) s += a[k] * b[k];
                C[(size_t)m * N + n] = (float)s;
            }
        }
        free(a);
    }
    free(Bd);
}

void rko_matmul_bf16(int M, int K, int N, const float *A, const float *B, float *C)
{ matmul_f64acc(M, K, N, A, B, C, bf16_f); }
void rko_matmul_tf32(int M, int K, int N, const float *A, const float *B, float *C)
{ matmul_f64acc(M, K, N, A, B, C, rko_tf32_trunc); }
void rko_matmul_f32(int M, int K, int N, const float *A, const float *B, float *C)
{ matmul_f64acc(M, K, N, A, B, C, id_f); }

int rko_set_threads(int n)
{
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
    return omp_get_max_threads();
#else
    (void)n;
    return 1;
#endif
}

/* ------------------------------------------------------------------------------------
 * Feed-forward blocks (reference src/rocket_ffn.c).
 * ---------------------------------------------------------------------------------- */
static inline uint64_t d2u(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }

/* IEEE 754 binary64 -> binary16, round to nearest, ties to even, from the double's bits
 * directly (no intermediate binary32 rounding). */
uint16_t rko_f64_to_f16(double d)
{
    uint64_t x = d2u(d);
    uint16_t sign = (uint16_t)((x >> 48) & 0x8000u);
    uint64_t ax = x & 0x7FFFFFFFFFFFFFFFull;
    int e = (int)(ax >> 52);
    if (e == 0x7FF) return (uint16_t)(sign | 0x7C00u | ((ax & 0xFFFFFFFFFFFFFull) ? 0x200u : 0u));
    if (ax >= 0x40EFFE0000000000ull) return (uint16_t)(sign | 0x7C00u);   /* >= 65520 -> inf */
    uint64_t m = (ax & 0xFFFFFFFFFFFFFull) | (e ? (1ull << 52) : 0);       /* 53-bit significand */
    int ue = e - 1023;                                                     /* unbiased exponent */
    if (ue >= -14) {                                                       /* binary16 normal */
        uint64_t q = m >> 42, rem = m & ((1ull << 42) - 1), half = 1ull << 41;   /* 11 bits kept */
        if (rem > half || (rem == half && (q & 1ull))) q++;
        /* q in [1024, 2048]: a carry to 2048 bumps the exponent through the field add */
        return (uint16_t)(sign | (uint16_t)(((uint64_t)(ue + 15) << 10) + (q - 1024)));
    }
    /* binary16 subnormal: value = m * 2^(ue - 52) in units of 2^-24 */
    int shift = 52 - 24 - ue;                                              /* 29 + (-ue - 1) */
    if (shift > 63) return sign;
    {
        uint64_t q = m >> shift, rem = m & ((1ull << shift) - 1), half = 1ull << (shift - 1);
        if (rem > half || (rem == half && (q & 1ull))) q++;
        return (uint16_t)(sign | (uint16_t)q);                             /* q = 1024 -> min normal */
    }
}

double rko_act_exact(int kind, double g)
{
    if (kind == 5) return 0.5 * g * (1.0 + erf(g * 0.70710678118654752440));
    return g / (1.0 + exp(-g));
}

void rko_geglu_f16(const uint16_t *gate, const uint16_t *up, int kind, uint16_t *prod, size_t n)
{
    #pragma omp parallel for schedule(static) if (n > 65536)
    for (size_t i = 0; i < n; i++)
        prod[i] = rko_f64_to_f16(rko_act_exact(kind, (double)rko_f16_to_f32(gate[i])) *
                                 (double)rko_f16_to_f32(up[i]));
}

void rko_ffn_f16(int M, int H, int I, const uint16_t *x, const uint16_t *Wg, const uint16_t *Wu,
                 const uint16_t *Wd, int kind, uint16_t *out)
{
    #pragma omp parallel for schedule(dynamic, 1)
    for (int m = 0; m < M; m++) {
        double *prod = (double *)malloc((size_t)I * sizeof(double));
        const uint16_t *xr = x + (size_t)m * H;
        for (int i = 0; i < I; i++) {
            const uint16_t *wg = Wg + (size_t)i * H, *wu = Wu + (size_t)i * H;
            double g = 0, u = 0;
            for (int h = 0; h < H; h++) {
                const double xv = rko_f16_to_f32(xr[h]);
                g += xv * (double)rko_f16_to_f32(wg[h]);
                u += xv * (double)rko_f16_to_f32(wu[h]);
            }
            prod[i] = rko_act_exact(kind, g) * u;
        }
        for (int h = 0; h < H; h++) {
            const uint16_t *wd = Wd + (size_t)h * I;
            double acc = 0;
            for (int i = 0; i < I; i++) acc += prod[i] * (double)rko_f16_to_f32(wd[i]);
            out[(size_t)m * H + h] = rko_f64_to_f16(acc);
        }
        free(prod);
    }
}

void rko_mlp_f16(int M, int Din, int Dff, int Dout, const uint16_t *x, const uint16_t *W1, const uint16_t *b1,
                 const uint16_t *W2, int kind, uint16_t *out)
{
    #pragma omp parallel for schedule(dynamic, 1)
    for (int m = 0; m < M; m++) {
        uint16_t *act = (uint16_t *)malloc((size_t)Dff * sizeof(uint16_t));
        const uint16_t *xr = x + (size_t)m * Din;
        for (int o = 0; o < Dff; o++) {
            const uint16_t *w = W1 + (size_t)o * Din;
            double a = b1 ? (double)rko_f16_to_f32(b1[o]) : 0.0;
            for (int i = 0; i < Din; i++) a += (double)rko_f16_to_f32(xr[i]) * (double)rko_f16_to_f32(w[i]);
            act[o] = rko_f64_to_f16(rko_act_exact(kind, a));
        }
        for (int o = 0; o < Dout; o++) {
            const uint16_t *w = W2 + (size_t)o * Dff;
            double a = 0;
            for (int i = 0; i < Dff; i++) a += (double)rko_f16_to_f32(act[i]) * (double)rko_f16_to_f32(w[i]);
            out[(size_t)m * Dout + o] = rko_f64_to_f16(a);
        }
        free(act);
    }
}

/* ------------------------------------------------------------------------------------
 * Per-row activation quantisation: the host loop of the reference's W8A8 tool
 * (tools/rk3576-w8a8-hostterm.c:51-68), in fp32 with the default rounding mode.
 * ---------------------------------------------------------------------------------- */
void rko_quant_rows_f32(int M, int K, const float *A, int8_t *Aq, float *row_scale)
{
    #pragma omp parallel for schedule(static) if ((long)M * K > 65536)
    for (int m = 0; m < M; m++) {
        const float *a = A + (size_t)m * K;
        float mx = 0.0f;
        for (int k = 0; k < K; k++) { float v = fabsf(a[k]); if (v > mx) mx = v; }
        const float s = (mx > 0.0f) ? 127.0f / mx : 0.0f;
        int8_t *o = Aq + (size_t)m * K;
        for (int k = 0; k < K; k++) {
            const int q = (int)nearbyintf(a[k] * s);
            o[k] = (int8_t)(q > 127 ? 127 : (q < -128 ? -128 : q));
        }
        row_scale[m] = (mx > 0.0f) ? mx / 127.0f : 0.0f;
    }
}

/* ------------------------------------------------------------------------------------
 * Attention (reference src/rocket_attn.c).
 * ---------------------------------------------------------------------------------- */
static inline double h2d(uint16_t h) { return (double)rko_f16_to_f32(h); }

/* rocket_attn.c:181-187: the score in fp32 from the fp64 dot product cast to float */
static float fa_score_f32(float qk, float scale, float softcap, float m)
{
    float s = qk * scale;
    if (softcap != 0.0f) s = softcap * tanhf(s / softcap);
    s += m;
    return s < -30000.0f ? -30000.0f : s;
}

void rko_flash_attn_f16(int T, int n_kv, int dk, int dv, int n_head, int n_kv_heads, float scale, float softcap,
                        const uint16_t *Q, const uint16_t *K, const uint16_t *V, const uint16_t *mask, uint16_t *out)
{
    const int gqa = n_head / n_kv_heads;
    #pragma omp parallel for collapse(2) schedule(dynamic, 4)
    for (int h = 0; h < n_head; h++) {
        for (int t = 0; t < T; t++) {
            const int hk = h / gqa;
            const uint16_t *qr = Q + ((size_t)h * T + t) * dk;
            const uint16_t *Kh = K + (size_t)hk * n_kv * dk;
            const uint16_t *Vh = V + (size_t)hk * dv * n_kv;
            const uint16_t *mr = mask ? mask + (size_t)t * n_kv : NULL;
            double *sc = (double *)malloc((size_t)n_kv * sizeof(double));
            double mx = -INFINITY;
            for (int j = 0; j < n_kv; j++) {
                const uint16_t *kr = Kh + (size_t)j * dk;
                double qk = 0;
                for (int c = 0; c < dk; c++) qk += h2d(qr[c]) * h2d(kr[c]);
                const double sj = fa_score_f32((float)qk, scale, softcap, mr ? rko_f16_to_f32(mr[j]) : 0.0f);
                sc[j] = sj;
                if (sj > mx) mx = sj;
            }
            double sum = 0;
            for (int j = 0; j < n_kv; j++) { sc[j] = exp(sc[j] - mx); sum += sc[j]; }
            const double inv = sum > 0 ? 1.0 / sum : 0.0;
            uint16_t *o = out + ((size_t)h * T + t) * dv;
            for (int c = 0; c < dv; c++) {
                double a = 0;
                for (int j = 0; j < n_kv; j++) a += sc[j] * h2d(Vh[(size_t)c * n_kv + j]);
                o[c] = rko_f64_to_f16(a * inv);
            }
            free(sc);
        }
    }
}

void rko_mha_self_f16(int T, int d, int n_head, const uint16_t *x, const uint16_t *Wq, const uint16_t *bq,
                      const uint16_t *Wk, const uint16_t *bk, const uint16_t *Wv, const uint16_t *bv,
                      const uint16_t *Wo, const uint16_t *bo, uint16_t *out)
{
    const int dh = d / n_head;
    const double scale = 1.0 / sqrt((double)dh);
    double *q = (double *)malloc((size_t)T * d * sizeof(double));
    double *k = (double *)malloc((size_t)T * d * sizeof(double));
    double *v = (double *)malloc((size_t)T * d * sizeof(double));
    double *ctx = (double *)malloc((size_t)T * d * sizeof(double));
    #pragma omp parallel for schedule(static)
    for (int t = 0; t < T; t++)
        for (int o = 0; o < d; o++) {
            double aq = 0, ak = 0, av = 0;
            for (int i = 0; i < d; i++) {
                const double xi = h2d(x[(size_t)t * d + i]);
                aq += xi * h2d(Wq[(size_t)o * d + i]);
                ak += xi * h2d(Wk[(size_t)o * d + i]);
                av += xi * h2d(Wv[(size_t)o * d + i]);
            }
            q[(size_t)t * d + o] = aq + (bq ? h2d(bq[o]) : 0);
            k[(size_t)t * d + o] = ak + (bk ? h2d(bk[o]) : 0);
            v[(size_t)t * d + o] = av + (bv ? h2d(bv[o]) : 0);
        }
    #pragma omp parallel for collapse(2) schedule(static)
    for (int h = 0; h < n_head; h++)
        for (int i = 0; i < T; i++) {
            const int off = h * dh;
            double *sc = (double *)malloc((size_t)T * sizeof(double));
            double mx = -INFINITY;
            for (int j = 0; j < T; j++) {
                double s = 0;
                for (int c = 0; c < dh; c++) s += q[(size_t)i * d + off + c] * k[(size_t)j * d + off + c];
                s *= scale;
                sc[j] = s;
                if (s > mx) mx = s;
            }
            double sum = 0;
            for (int j = 0; j < T; j++) { sc[j] = exp(sc[j] - mx); sum += sc[j]; }
            for (int c = 0; c < dh; c++) {
                double a = 0;
                for (int j = 0; j < T; j++) a += sc[j] * v[(size_t)j * d + off + c];
                ctx[(size_t)i * d + off + c] = a / sum;
            }
            free(sc);
        }
    #pragma omp parallel for schedule(static)
    for (int t = 0; t < T; t++)
        for (int o = 0; o < d; o++) {
            double a = 0;
            for (int i = 0; i < d; i++) a += ctx[(size_t)t * d + i] * h2d(Wo[(size_t)o * d + i]);
            out[(size_t)t * d + o] = rko_f64_to_f16(a + (bo ? h2d(bo[o]) : 0));
        }
    free(q); free(k); free(v); free(ctx);
}
