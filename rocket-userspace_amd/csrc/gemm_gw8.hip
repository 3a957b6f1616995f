// gemm_gw8.hip — instantiations of the GEMM kernel for group-wise products with int8 weights.
#include "gemm_impl.h"

namespace rk {
namespace gk {

hipError_t dispatch_gw_i8(int bm, int bn, const Launch &L, const KArgs &ka, int blocks)
{
    hipStream_t s = L.stream;
    return by_tile(bm, bn, [&](auto BM_, auto BN_) -> hipError_t {
        constexpr int BM = decltype(BM_)::value, BN = decltype(BN_)::value;
        (void)s;
        if (L.fmt_a == Fmt::I8 && L.fmt_b == Fmt::I8 && L.epi == Epi::GW)
            return launch_gw<BM, BN, Fmt::I8, Fmt::I8>(L, ka, blocks);
        return hipErrorInvalidValue;
    });
}

}  // namespace gk
}  // namespace rk
