// hw_profile.cpp — the machine profile (interface of reference include/rocket_hw_profile.h,
// selection logic of reference src/rocket_hw_profile.c:197-256), filled with MI355X
// figures: 160 KiB of LDS per CU as 5 x 32 KiB "banks", the kernels' largest output tile,
// the K alignment of the 1-2-byte and the 4-byte entries, and every precision.
#include "rocket_hw_profile.h"
#include "rocket_log.h"

#include <stdlib.h>
#include <string.h>

#include <mutex>

extern "C" {

#define RK_ALL_DTYPES 0xFFu

const struct rocket_hw_profile rocket_hw_mi355x = {
    "mi355x", 5, 32768, 128, 32, 16, 16, RK_ALL_DTYPES, nullptr, 1,
};

// The reference's NPU profile names, kept so code that references them links; they
// describe the same GPU and say so when selected.
const struct rocket_hw_profile rocket_hw_rk3588 = {
    "rk3588", 5, 32768, 128, 32, 16, 16, RK_ALL_DTYPES,
    "ROCKET_CHIP=rk3588: this librocketnpu drives an MI355X GPU; GPU parameters apply", 1,
};
const struct rocket_hw_profile rocket_hw_rk3576 = {
    "rk3576", 5, 32768, 128, 32, 16, 16, RK_ALL_DTYPES,
    "ROCKET_CHIP=rk3576: this librocketnpu drives an MI355X GPU; GPU parameters apply", 1,
};

const struct rocket_hw_profile *rocket_hw_by_name(const char *name)
{
    if (!name) return nullptr;
    if (!strcmp(name, "mi355x") || !strcmp(name, "gfx950")) return &rocket_hw_mi355x;
    if (!strcmp(name, "rk3588")) return &rocket_hw_rk3588;
    if (!strcmp(name, "rk3576")) return &rocket_hw_rk3576;
    return nullptr;
}

const struct rocket_hw_profile *rocket_hw_current(void)
{
    static const struct rocket_hw_profile *cur = nullptr;
    static std::once_flag once;
    std::call_once(once, [] {
        cur = &rocket_hw_mi355x;
        if (const char *e = getenv("ROCKET_CHIP")) {
            const struct rocket_hw_profile *p = rocket_hw_by_name(e);
            if (p) cur = p;
            else ROCKET_LOGW("rocket_hw_current: unknown ROCKET_CHIP=%s, using mi355x\n", e);
        }
        if (cur->select_warning) ROCKET_LOGW("%s\n", cur->select_warning);
    });
    return cur;
}

}  // extern "C"
