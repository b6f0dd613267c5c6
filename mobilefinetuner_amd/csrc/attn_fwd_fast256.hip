// D = 256 instantiation of the bf16 fast forward (attn_fwd_fast.h), in a
// translation unit of its own so that it compiles in parallel with the
// rest; built, like attn_fwd.hip, with MFMA accumulators in VGPRs.  The
// balanced launch on whole tiles runs the 16-row, two-waves-per-SIMD kernel
// of attn_fwd_w16.h; the rest the 32-row kernels.
#include "attn_fwd_w16.h"

namespace mft {
namespace fwd {
hipError_t launch_fwd_fast256(const AttnShape& s, FwdArgs a, hipStream_t st) {
    if (a.part_o == nullptr || !fwd_fast_dma<256>(s)) return launch_fwd_fast_t<256>(s, a, st);
    a.n_qtiles = (int)((s.S + kFwdBM - 1) / kFwdBM);
    const dim3 grid((unsigned)(a.us.units * s.B * s.Hq));
    if (s.causal)
        hipLaunchKernelGGL((attn_fwd_bf16_split16<256, true>), grid, dim3(kW16Threads), 0, st, a);
    else
        hipLaunchKernelGGL((attn_fwd_bf16_split16<256, false>), grid, dim3(kW16Threads), 0, st, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || !a.any_split) return e;
    return launch_fwd_combine(s, a, st);
}
}  // namespace fwd
}  // namespace mft
