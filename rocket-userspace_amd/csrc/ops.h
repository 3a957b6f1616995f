// ops.h — the one request type every matmul entry point reduces to.
#pragma once

#include "internal.h"

namespace rk {

constexpr int kDimMax = 1 << 24;   // reference rocket_matmul.c:492 (ROCKET_MM_DIM_MAX)

struct Req {
    const char *who = "";
    Fmt fa = Fmt::I8, fb = Fmt::I8;
    Epi epi = Epi::I32;
    int K = 0, N = 0;
    int nprob = 1;
    // per problem (nprob entries)
    const int *M = nullptr;
    const void *const *A = nullptr;
    const void *const *B = nullptr;      // host or device; int8 per byte when pack_b_int4
    void *const *C = nullptr;
    const float *const *a_scale = nullptr;
    const float *const *b_scale = nullptr;
    int group = 0;
    bool rowscale = false;               // GW: a_scale holds one fp32 per row, not per (row, group)
    bool pack_b_int4 = false;            // B arrives one int4 value per byte: pack on device
    bool b_packed = false;               // B already in the device I4P layout (resident)
    int kchunk = 0;                      // >0: launch K in chunks, accumulating into C
    // GW: per-group partials per problem (nprob entries each; a null pointer or 0 rows: none)
    int32_t *const *dump = nullptr;
    const int *dump_row0 = nullptr, *dump_rows = nullptr;
    // GW rowscale: A holds fp32 (1) or fp16 (2) activations that a pre-pass quantises per
    // row into the arena (int8 codes + one scale per row, which the GEMM then uses)
    int quant_a = 0;
    // quant_a 1 (fp32) or 2 (fp16) with act (kActSilu / kActGelu): the rows quantised are
    // act(A) * A2
    const void *const *A2 = nullptr;
    int act = 0;
    // GW: C holds fp16, each fp32 result rounded once
    bool f16out = false;
};

// Runs a request on handle fd: stages host operands, launches, copies back, waits.
int run(int fd, const Req &r);

// Bytes of one operand row in HBM for a format.
size_t fmt_row_bytes(Fmt f, int K);
// Bytes of one C element for an epilogue.
size_t epi_elem_bytes(Epi e);
// int32 partial period for a quant group: the group itself up to 65536, else its largest
// multiple-of-32 divisor not above 65536 (keeps every int32 partial exact).
int gw_period(int group);

}  // namespace rk
