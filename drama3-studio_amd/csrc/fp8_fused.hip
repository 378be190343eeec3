// Single-launch decode: the call-size check and the dispatch by weight
// format.  The kernel itself is fp8_fused_kernel.hpp; the E4M3 instances are
// built here, the integer-format instances in fp8_fused_w4.hip / _w6.hip.
#include "fp8_fused_kernel.hpp"

namespace dmoe {

bool fused_decode_fits(int pairs, int rows, int H, int I, int experts, int top_k, int x_esize, int routed_tokens) {
    const int KBd = I / 128;
    return pairs >= 1 && pairs <= kFusedMaxPairs && rows >= 1 && (int64_t)rows * H <= kFusedXBytes &&
           (int64_t)rows * H * x_esize <= kFusedRawBytes && (int64_t)pairs * I <= kFusedHBytes &&
           H <= kFusedMaxH && I <= kFusedMaxI && H % kTileRows == 0 && experts <= kMaxExperts && top_k >= 1 &&
           top_k <= 64 && KBd >= 1 && KBd <= 8;
}

bool launch_fp8_fused_decode(const FusedDecodeArgs& a, hipStream_t stream) {
    switch (a.w13.wfmt) {
        case kWfFp8: return launch_fused_format<kWfFp8>(a, stream);
        case kWfInt4: return launch_fused_int4(a, stream);
        case kWfInt6: return launch_fused_int6(a, stream);
        default: return false;
    }
}

}  // namespace dmoe
