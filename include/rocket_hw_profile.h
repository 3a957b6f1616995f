/*
 * rocket_hw_profile.h — machine-parameter profile (interface of reference
 * include/rocket_hw_profile.h:60-124, same struct layout and prototypes).
 *
 * The reference keys its tiling on an NPU CBUF. On MI355X the struct is kept for ABI
 * compatibility and filled with the GPU's figures, re-read in the fields' own terms:
 *   cbuf_banks / cbuf_bank_size  LDS per CU expressed as 5 banks of 32 KiB (160 KiB)
 *   max_tile                     the largest M/N workgroup tile the kernels use (256)
 *   kgroup_2b / kgroup_4b        K bytes one MFMA consumes per lane group (64 / 64)
 *   ngroup                       MFMA N granularity (16)
 *   dtype_supported              every precision_* value below
 *   default_workers              1 (one GPU grid replaces the per-fd worker fan-out)
 * rocket_hw_current() returns the "mi355x" profile; ROCKET_CHIP may name it. The
 * reference's "rk3588" and "rk3576" names resolve to the same GPU profile with a
 * warning, since no NPU exists behind this library.
 */
#ifndef ROCKET_HW_PROFILE_H
#define ROCKET_HW_PROFILE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Precision encodings (values of reference include/npu_hw.h:302-309). */
#ifndef NPU_HW_H
enum { precision_int8 = 0,
       precision_int16 = 1,
       precision_float16 = 2,
       precision_bfloat16 = 3,
       precision_int32 = 4,
       precision_float32 = 5,
       precision_int4 = 6,
       precision_tf32 = 7 };
#endif

#define ROCKET_DT_BIT(prec)   (1u << (prec))

struct rocket_hw_profile {
    const char *name;
    int cbuf_banks;
    int cbuf_bank_size;
    int max_tile;
    int kgroup_2b;
    int kgroup_4b;
    int ngroup;
    uint32_t dtype_supported;
    const char *select_warning;
    int default_workers;
};

const struct rocket_hw_profile *rocket_hw_current(void);
const struct rocket_hw_profile *rocket_hw_by_name(const char *name);

/* The MI355X profile; the reference's two NPU profile objects are exported as
 * aliases of the same GPU figures (names "rk3588" / "rk3576"). */
extern const struct rocket_hw_profile rocket_hw_mi355x;
extern const struct rocket_hw_profile rocket_hw_rk3588;
extern const struct rocket_hw_profile rocket_hw_rk3576;

static inline int rocket_hw_dtype_supported(const struct rocket_hw_profile *p, int precision)
{
    return (p->dtype_supported & ROCKET_DT_BIT(precision)) != 0;
}

#ifdef __cplusplus
}
#endif
#endif /* ROCKET_HW_PROFILE_H */
