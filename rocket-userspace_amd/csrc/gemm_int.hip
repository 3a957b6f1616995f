// gemm_int.hip — instantiations of the GEMM kernel for int8 / int4 products to int32 and the int16-exact product.
#include "gemm_impl.h"

namespace rk {
namespace gk {

hipError_t dispatch_int(int bm, int bn, const Launch &L, const KArgs &ka, int blocks)
{
    hipStream_t s = L.stream;
    return by_tile(bm, bn, [&](auto BM_, auto BN_) -> hipError_t {
        constexpr int BM = decltype(BM_)::value, BN = decltype(BN_)::value;
        (void)s;
        if (L.fmt_a == Fmt::I8 && L.fmt_b == Fmt::I8 && L.epi == Epi::I32)
            return launch_one<BM, BN, Fmt::I8, Fmt::I8, MathI8, Epi::I32, false>(ka, blocks, s);
        if (L.fmt_a == Fmt::I8 && L.fmt_b == Fmt::I4P && L.epi == Epi::I32)
            return launch_one<BM, BN, Fmt::I8, Fmt::I4P, MathI8, Epi::I32, false>(ka, blocks, s);
        if constexpr (BM <= 128)   // two byte planes per operand: 2 x 2 planes per stage
            if (L.fmt_a == Fmt::I16 && L.fmt_b == Fmt::I16 && L.epi == Epi::I64)
                return launch_one<BM, BN, Fmt::I16, Fmt::I16, MathI16, Epi::I64, false>(ka, blocks, s);
        return hipErrorInvalidValue;
    });
}

}  // namespace gk
}  // namespace rk
