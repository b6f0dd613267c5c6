// bf16 fast-path backward instantiation for head dims 129..256.  Its roles
// hold more than 256 registers of state (K, V, dK, dV fragments), so the
// long-lived accumulators live in AGPRs: this file is compiled with the
// compiler's default MFMA register form.
#include "attn_bwd_fast.h"

namespace mft {
namespace bwd {
hipError_t launch_bwd_fast_256(const AttnShape& s, const BwdArgs& a, int stages, hipStream_t st) {
    return launch_bwd_fast<256>(s, a, stages, st);
}
}  // namespace bwd
}  // namespace mft
