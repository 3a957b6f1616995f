// gemm_f16.hip — instantiations of the GEMM kernel for fp16 products (fp16 / fp32 results, bias + activation and gated epilogues).
#include "gemm_impl.h"

namespace rk {
namespace gk {

hipError_t dispatch_f16(int bm, int bn, const Launch &L, const KArgs &ka, int blocks)
{
    hipStream_t s = L.stream;
    if (bm == 256 && bn == 256) {   // 256 x 256 tiles: fp16 / fp32 / activation / gated epilogues
        if (L.fmt_a == Fmt::F16 && L.fmt_b == Fmt::F16) {
            // 16 x 16 x 32 MFMAs on the 256-row tiles (a wave holds 32 blocks of 16 x 16): fp16
            // 512 x 3840 x 30720 145 -> 135 us, 2048 x 3840 x 15360 280 -> 261 us against
            // 32 x 32 x 16 (same operand bytes per flop; shorter MFMA latency, more independent
            // accumulator chains)
            using MW = MathF16x16;
            if (L.epi == Epi::F16) return launch_one<256, 256, Fmt::F16, Fmt::F16, MW, Epi::F16, false>(ka, blocks, s);
            if (L.epi == Epi::F32) return launch_one<256, 256, Fmt::F16, Fmt::F16, MW, Epi::F32, false>(ka, blocks, s);
            if (L.epi == Epi::ACT) return launch_one<256, 256, Fmt::F16, Fmt::F16, MW, Epi::ACT, false>(ka, blocks, s);
            if (L.epi == Epi::GLU) return launch_one<256, 256, Fmt::F16, Fmt::F16, MW, Epi::GLU, false>(ka, blocks, s);
        }
        return hipErrorInvalidValue;
    }
    return by_tile(bm, bn, [&](auto BM_, auto BN_) -> hipError_t {
        constexpr int BM = decltype(BM_)::value, BN = decltype(BN_)::value;
        using MT = std::conditional_t<BM == 256, MathF16x16, MathF16>;
        if (L.fmt_a == Fmt::F16 && L.fmt_b == Fmt::F16) {
            if (L.epi == Epi::F16) return launch_one<BM, BN, Fmt::F16, Fmt::F16, MT, Epi::F16, false>(ka, blocks, s);
            if (L.epi == Epi::F32) return launch_one<BM, BN, Fmt::F16, Fmt::F16, MT, Epi::F32, false>(ka, blocks, s);
            if (L.epi == Epi::ACT) return launch_one<BM, BN, Fmt::F16, Fmt::F16, MT, Epi::ACT, false>(ka, blocks, s);
            if constexpr (BN == 128 && BM <= 256)
                if (L.epi == Epi::GLU) return launch_one<BM, BN, Fmt::F16, Fmt::F16, MT, Epi::GLU, false>(ka, blocks, s);
        }
        return hipErrorInvalidValue;
    });
}

}  // namespace gk
}  // namespace rk
