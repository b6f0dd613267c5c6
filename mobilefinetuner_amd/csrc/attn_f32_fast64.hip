// fp32 fast-path instantiations for padded head dim 64, and the
// dispatch of fp32 shapes by head dim.
#include "attn_f32_fast.h"

namespace mft {
namespace f32 {
template hipError_t launch_fwd_dpf<64>(const AttnShape&, const FwdArgs&, hipStream_t);
template hipError_t launch_bwd_units<64, true, true>(const AttnShape&, const BwdArgs&, int, hipStream_t);
template hipError_t launch_bwd_units<64, false, true>(const AttnShape&, const BwdArgs&, int, hipStream_t);
template hipError_t launch_bwd_units<64, true, false>(const AttnShape&, const BwdArgs&, int, hipStream_t);
template hipError_t launch_bwd_units<64, false, false>(const AttnShape&, const BwdArgs&, int, hipStream_t);

bool fast_path(const AttnShape& s) { return !s.bf16 && s.D % 4 == 0 && s.D > 32 && s.D <= 256; }

hipError_t launch_fwd_fast(const AttnShape& s, const FwdArgs& a, hipStream_t st) {
    if (s.D <= 64) return launch_fwd_dpf<64>(s, a, st);
    if (s.D <= 128) return launch_fwd_dpf<128>(s, a, st);
    return launch_fwd_dpf<256>(s, a, st);
}

hipError_t launch_bwd_fast(const AttnShape& s, const BwdArgs& a, int stages, hipStream_t st) {
    if (s.D <= 64) return launch_bwd_dpf<64>(s, a, stages, st);
    if (s.D <= 128) return launch_bwd_dpf<128>(s, a, stages, st);
    return launch_bwd_dpf<256>(s, a, stages, st);
}
}  // namespace f32
}  // namespace mft
