// gemm_f16.hip — instantiations of the GEMM kernel for fp16 products (fp16 / fp32 results, bias + activation and gated epilogues).
#include "gemm_impl.h"

namespace rk {
namespace gk {

hipError_t dispatch_f16(int bm, int bn, const Launch &L, const KArgs &ka, int blocks)
{
    hipStream_t s = L.stream;
    if (bm == 256 && bn == 256) {   // 256 x 256 tiles: fp16 / fp32 / activation / gated epilogues
        if (L.fmt_a == Fmt::F16 && L.fmt_b == Fmt::F16) {
            if (L.epi == Epi::F16) return launch_one<256, 256, Fmt::F16, Fmt::F16, MathF16, Epi::F16, false>(ka, blocks, s);
            if (L.epi == Epi::F32) return launch_one<256, 256, Fmt::F16, Fmt::F16, MathF16, Epi::F32, false>(ka, blocks, s);
            if (L.epi == Epi::ACT) return launch_one<256, 256, Fmt::F16, Fmt::F16, MathF16, Epi::ACT, false>(ka, blocks, s);
            if (L.epi == Epi::GLU) return launch_one<256, 256, Fmt::F16, Fmt::F16, MathF16, Epi::GLU, false>(ka, blocks, s);
        }
        return hipErrorInvalidValue;
    }
    return by_tile(bm, bn, [&](auto BM_, auto BN_) -> hipError_t {
        constexpr int BM = decltype(BM_)::value, BN = decltype(BN_)::value;
        if (L.fmt_a == Fmt::F16 && L.fmt_b == Fmt::F16) {
            if (L.epi == Epi::F16) return launch_one<BM, BN, Fmt::F16, Fmt::F16, MathF16, Epi::F16, false>(ka, blocks, s);
            if (L.epi == Epi::F32) return launch_one<BM, BN, Fmt::F16, Fmt::F16, MathF16, Epi::F32, false>(ka, blocks, s);
            if (L.epi == Epi::ACT) return launch_one<BM, BN, Fmt::F16, Fmt::F16, MathF16, Epi::ACT, false>(ka, blocks, s);
            if constexpr (BN == 128 && BM <= 256)
                if (L.epi == Epi::GLU) return launch_one<BM, BN, Fmt::F16, Fmt::F16, MathF16, Epi::GLU, false>(ka, blocks, s);
        }
        return hipErrorInvalidValue;
    });
}

}  // namespace gk
}  // namespace rk
