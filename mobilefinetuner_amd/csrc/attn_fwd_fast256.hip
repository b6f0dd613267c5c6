// D = 256 instantiation of the bf16 fast forward (attn_fwd_fast.h), in a
// translation unit of its own so that it compiles in parallel with the
// rest; built, like attn_fwd.hip, with MFMA accumulators in VGPRs.
#include "attn_fwd_fast.h"

namespace mft {
namespace fwd {
hipError_t launch_fwd_fast256(const AttnShape& s, FwdArgs a, hipStream_t st) {
    return launch_fwd_fast_t<256>(s, a, st);
}
}  // namespace fwd
}  // namespace mft
