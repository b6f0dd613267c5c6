// bf16 fast-path backward instantiations for head dims 33..128 (compiled with
// MFMA accumulators in VGPRs: every live value fits the 256 VGPRs).
#include "attn_bwd_fast.h"

namespace mft {
namespace bwd {
hipError_t launch_bwd_fast_64(const AttnShape& s, const BwdArgs& a, int stages, hipStream_t st) {
    return launch_bwd_fast<64>(s, a, stages, st);
}
hipError_t launch_bwd_fast_128(const AttnShape& s, const BwdArgs& a, int stages, hipStream_t st) {
    return launch_bwd_fast<128>(s, a, stages, st);
}
}  // namespace bwd
}  // namespace mft
