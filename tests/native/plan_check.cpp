// Host-side check that the split planners keep every tile within the merge
// kernels' slot limit (kSplitMaxSlots) over a sweep of shapes, masks and
// windows, so that the C ABI's plan check (MFT_ERR_UNSUPPORTED) is never hit
// by a shape the library supports.  Linked against libmft_attn.so and run by
// tests/test_geometry.py without a GPU (the planners then assume 256 CUs);
// prints "ok <cases>" or the first shape over the limit.
#include <cstdio>

#include "attn_kernels.h"

int main() {
    const long long S_list[] = {1, 63, 64, 65, 127, 128, 1000, 2048, 4096, 8192, 32768, 131072, 1 << 20};
    const int shapes[][3] = {{1, 1, 1}, {1, 4, 1}, {2, 14, 2}, {4, 4, 1}, {1, 16, 8}, {8, 32, 8}, {64, 32, 32}};
    const int windows[] = {0, 1, 512, 4096};
    const int dims[] = {64, 128, 256};
    int cases = 0;
    for (long long S : S_list)
        for (const auto& sh : shapes)
            for (int W : windows)
                for (int causal = 0; causal < 2; ++causal)
                    for (int D : dims) {
                        if (W && !causal) continue;
                        mft::AttnShape s{};
                        s.B = sh[0];
                        s.Hq = sh[1];
                        s.Hkv = sh[2];
                        s.S = S;
                        s.D = D;
                        s.scale = 0.1f;
                        s.causal = causal != 0;
                        s.bf16 = true;
                        s.window = W < S ? W : 0;
                        s.contiguous = true;
                        const mft::FwdPlan f = mft::plan_fwd_split(s);
                        const mft::BwdPlan b = mft::plan_bwd_fast(s);
                        if (f.parts_max > mft::kSplitMaxSlots || b.kv_parts_max > mft::kSplitMaxSlots ||
                            b.q_parts_max > mft::kSplitMaxSlots) {
                            std::printf("OVER S=%lld B=%d Hq=%d Hkv=%d D=%d causal=%d W=%d fwd=%d kv=%d q=%d\n", S,
                                        sh[0], sh[1], sh[2], D, causal, W, f.parts_max, b.kv_parts_max,
                                        b.q_parts_max);
                            return 1;
                        }
                        ++cases;
                    }
    std::printf("ok %d\n", cases);
    return 0;
}
