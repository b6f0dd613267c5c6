// fp32 fast path, padded head dim 256: the combined MAIN launch, without the causal mask.
#include "attn_f32_fast.h"

namespace mft {
namespace f32 {
template hipError_t launch_bwd_units<256, false, true>(const AttnShape&, const BwdArgs&, int, hipStream_t);
}  // namespace f32
}  // namespace mft
