// Host-side check that the split planners keep every tile within the merge
// kernels' slot limit (kSplitMaxSlots) over a sweep of shapes, masks and
// windows, so that the C ABI's plan check (MFT_ERR_UNSUPPORTED) is never hit
// by a shape the library supports, and that every unit split partitions its
// role's iterations with the slots the kernels write and the merges read.  Linked against libmft_attn.so and run by
// tests/test_geometry.py without a GPU (the planners then assume 256 CUs);
// prints "ok <cases>" or the first shape over the limit.
#include <cstdio>

#include "attn_kernels.h"

// The unit split of one role covers its iterations exactly once, in order:
// unit k holds [unit_first(k), unit_first(k + 1)), nonempty (at least
// min_iters iterations when there are several units), unit_of agrees at
// both ends, and for every split tile the slot REDUCE / combine read for
// each unit (split_slot) is the slot the unit writes (2u for its first
// segment, 2u + 1 for its last).
static bool check_split(const mft::FastTiles& g, const mft::UnitSplit& u, const char* role, int min_iters) {
    const int nt = g.nt();
    auto tile_of = [&](int64_t i, int t) {  // from a tile at or before i's
        while (t + 1 < nt && g.start(t + 1) <= i) ++t;
        return t;
    };
    if (mft::unit_first(g, u, 0) != 0 || mft::unit_first(g, u, u.units) != g.total()) {
        std::printf("BAD %s: bounds\n", role);
        return false;
    }
    int t = 0;
    for (int k = 0; k < u.units; ++k) {
        const int64_t f0 = mft::unit_first(g, u, k), f1 = mft::unit_first(g, u, k + 1);
        if (f1 <= f0 || (u.units > 1 && f1 - f0 < min_iters)) {
            std::printf("BAD %s: unit %d holds [%lld, %lld)\n", role, k, (long long)f0, (long long)f1);
            return false;
        }
        t = tile_of(f0, t);
        const int t1 = tile_of(f1 - 1, t);
        if (mft::unit_of(u, f0, t) != k || mft::unit_of(u, f1 - 1, t1) != k) {
            std::printf("BAD %s: unit_of at unit %d\n", role, k);
            return false;
        }
    }
    for (int tt = 0; tt < nt; ++tt) {
        int u0;
        const int nsl = mft::tile_units(g, u, tt, &u0);
        const int64_t s = g.start(tt), e = s + g.n(tt);
        const bool starts = mft::unit_first(g, u, u0) == s;
        for (int p = 0; p < nsl; ++p) {
            const int un = u0 + p;
            const int64_t f = mft::unit_first(g, u, un);
            const int64_t writes = 2 * un + ((f >= s && f < e) ? 0 : 1);
            if (nsl > 1 && mft::split_slot(un, u0, starts) != writes) {
                std::printf("BAD %s: tile %d unit %d slot\n", role, tt, un);
                return false;
            }
        }
        if (mft::unit_of(u, e - 1, tt) != u0 + nsl - 1 || (tt > 0 && mft::unit_of(u, s - 1, tt - 1) > u0)) {
            std::printf("BAD %s: tile %d units\n", role, tt);
            return false;
        }
    }
    return true;
}

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
                    for (int D : dims)
                    for (int bf = 0; bf < 2; ++bf) {
                        if (W && !causal) continue;
                        mft::AttnShape s{};
                        s.B = sh[0];
                        s.Hq = sh[1];
                        s.Hkv = sh[2];
                        s.S = S;
                        s.D = D;
                        s.scale = 0.1f;
                        s.causal = causal != 0;
                        s.bf16 = bf != 0;  // fp32: the fp32 fast path's units (two workgroups each)
                        s.window = W < S ? W : 0;
                        s.contiguous = true;
                        const mft::FwdPlan f = mft::plan_fwd_split(s);
                        const mft::BwdPlan b = mft::plan_bwd_fast(s);
                        if (f.parts_max > mft::kSplitMaxSlots || b.kv_parts_max > mft::kSplitMaxSlots ||
                            b.q_parts_max > mft::kSplitMaxSlots) {
                            std::printf("OVER S=%lld B=%d Hq=%d Hkv=%d D=%d bf16=%d causal=%d W=%d fwd=%d kv=%d q=%d\n", S,
                                        sh[0], sh[1], sh[2], D, bf, causal, W, f.parts_max, b.kv_parts_max,
                                        b.q_parts_max);
                            return 1;
                        }
                        const int G = sh[1] / sh[2], Wv = (int)s.window, Si = (int)S;
                        // a forward planned without the balanced launch (one
                        // workgroup per query tile) has no unit split to check
                        if ((f.balanced &&
                             !check_split(mft::FastTiles{Si, causal, Wv, G, 0}, f.us, "fwd", mft::kMinFwdUnitIters)) ||
                            !check_split(mft::FastTiles{Si, causal, Wv, G, 1}, b.kv, "kv", mft::kMinUnitIters) ||
                            !check_split(mft::FastTiles{Si, causal, Wv, G, 0}, b.q, "q", mft::kMinUnitIters)) {
                            std::printf("  at S=%lld B=%d Hq=%d Hkv=%d D=%d causal=%d W=%d\n", S, sh[0], sh[1],
                                        sh[2], D, causal, W);
                            return 1;
                        }
                        ++cases;
                    }
    std::printf("ok %d\n", cases);
    return 0;
}
