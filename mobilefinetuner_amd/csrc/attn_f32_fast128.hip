// fp32 fast-path instantiations for padded head dim 128.
#include "attn_f32_fast.h"

namespace mft {
namespace f32 {
template hipError_t launch_fwd_dpf<128>(const AttnShape&, const FwdArgs&, hipStream_t);
template hipError_t launch_bwd_units<128, true, true>(const AttnShape&, const BwdArgs&, int, hipStream_t);
template hipError_t launch_bwd_units<128, false, true>(const AttnShape&, const BwdArgs&, int, hipStream_t);
template hipError_t launch_bwd_units<128, true, false>(const AttnShape&, const BwdArgs&, int, hipStream_t);
template hipError_t launch_bwd_units<128, false, false>(const AttnShape&, const BwdArgs&, int, hipStream_t);
}  // namespace f32
}  // namespace mft
