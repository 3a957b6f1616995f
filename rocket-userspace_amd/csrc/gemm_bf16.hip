// gemm_bf16.hip — instantiations of the GEMM kernel for products of fp32 operands in bf16 and tf32 (bf16 hi/lo) arithmetic.
#include "gemm_impl.h"

namespace rk {
namespace gk {

hipError_t dispatch_bf16(int bm, int bn, const Launch &L, const KArgs &ka, int blocks)
{
    hipStream_t s = L.stream;
    if (bm == 256 && bn == 256) {   // 256 x 256 tiles: bf16 operands converted ahead
        if (L.epi == Epi::F32 && L.fmt_a == Fmt::BF16 && L.fmt_b == Fmt::BF16)
            return launch_one<256, 256, Fmt::BF16, Fmt::BF16, MathBF16x16, Epi::F32, false>(ka, blocks, s);
        return hipErrorInvalidValue;
    }
    return by_tile(bm, bn, [&](auto BM_, auto BN_) -> hipError_t {
        constexpr int BM = decltype(BM_)::value, BN = decltype(BN_)::value;
        if (L.epi != Epi::F32) return hipErrorInvalidValue;
        if (L.fmt_a == Fmt::F32BF16 && L.fmt_b == Fmt::F32BF16)
            return launch_one<BM, BN, Fmt::F32BF16, Fmt::F32BF16, MathBF16, Epi::F32, false>(ka, blocks, s);
        // 16 x 16 x 32 MFMAs on the 256-row tiles (config 4 343 -> 334 us a call)
        using MT = std::conditional_t<BM == 256, MathBF16x16, MathBF16>;
        if (L.fmt_a == Fmt::BF16 && L.fmt_b == Fmt::BF16)
            return launch_one<BM, BN, Fmt::BF16, Fmt::BF16, MT, Epi::F32, false>(ka, blocks, s);
        if (L.fmt_a == Fmt::BF16 && L.fmt_b == Fmt::F32BF16)
            return launch_one<BM, BN, Fmt::BF16, Fmt::F32BF16, MathBF16, Epi::F32, false>(ka, blocks, s);
        if constexpr (BM <= 128) {   // two-plane operands: 2 x 2 planes per stage
            if (L.fmt_a == Fmt::F32TF32 && L.fmt_b == Fmt::F32TF32)
                return launch_one<BM, BN, Fmt::F32TF32, Fmt::F32TF32, MathTF32, Epi::F32, false>(ka, blocks, s);
            if (L.fmt_a == Fmt::BF16X2 && L.fmt_b == Fmt::BF16X2)
                return launch_one<BM, BN, Fmt::BF16X2, Fmt::BF16X2, MathTF32, Epi::F32, false>(ka, blocks, s);
            if (L.fmt_a == Fmt::BF16X2 && L.fmt_b == Fmt::F32TF32)
                return launch_one<BM, BN, Fmt::BF16X2, Fmt::F32TF32, MathTF32, Epi::F32, false>(ka, blocks, s);
        }
        return hipErrorInvalidValue;
    });
}

}  // namespace gk
}  // namespace rk
