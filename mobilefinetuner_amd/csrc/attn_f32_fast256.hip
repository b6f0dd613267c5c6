// fp32 fast-path instantiations for padded head dim 256: the forward.  The
// backward's kernels are in attn_f32_fast256_{main,stage}_{causal,full}.hip
// (the D = 256 kernels are the slowest to compile; split, they compile in
// parallel).
#include "attn_f32_fast.h"

namespace mft {
namespace f32 {
template hipError_t launch_fwd_dpf<256>(const AttnShape&, const FwdArgs&, hipStream_t);
}  // namespace f32
}  // namespace mft
