// Single-launch decode instances for 4-bit integer weights with group-128
// scales (wfmt.hpp), built apart from the E4M3 instances to compile in parallel.
#include "fp8_fused_kernel.hpp"

namespace dmoe {

bool launch_fused_int4(const FusedDecodeArgs& a, hipStream_t stream) {
    return launch_fused_format<kWfInt4>(a, stream);
}

}  // namespace dmoe
