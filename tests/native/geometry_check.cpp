// Host-side check of the closed-form work geometry (attn_geometry.h) against
// brute-force enumeration of the tiles that hold a visible (query, key) pair
// under the causal mask and a causal sliding window.  Built and run by
// tests/test_geometry.py; prints "ok <cases>" or the first mismatch.
#include <algorithm>
#include <cstdio>
#include <cstdlib>

#include "attn_geometry.h"

namespace {

bool visible(int i, int j, int causal, int W) {
    if (causal && j > i) return false;
    if (W > 0 && i - j >= W) return false;
    return true;
}

// Some row of [r0, r1] sees some key of [k0, k1] (all < S).
bool pair_in(int r0, int r1, int k0, int k1, int causal, int W) {
    for (int i = r0; i <= r1; ++i)
        for (int j = k0; j <= k1; ++j)
            if (visible(i, j, causal, W)) return true;
    return false;
}

int fail(const char* what, int S, int causal, int W, int t, long long got, long long want) {
    std::printf("MISMATCH %s S=%d causal=%d W=%d tile=%d got=%lld want=%lld\n", what, S, causal, W, t, got, want);
    return 1;
}

int check(int S, int causal, int W, int group) {
    using namespace mft;
    // query tiles of 128 rows x 64-key tiles
    const int nqt = (S + 127) / 128, nkt64 = (S + 63) / 64;
    long long start = 0;
    for (int qt = 0; qt < nqt; ++qt) {
        const int r0 = 128 * qt, r1 = std::min(S, r0 + 128) - 1;
        int lo = -1, n = 0;
        for (int t = 0; t < nkt64; ++t)
            if (pair_in(r0, r1, 64 * t, std::min(S, 64 * t + 64) - 1, causal, W)) {
                if (lo < 0) lo = t;
                if (t != lo + n) return fail("q tiles not contiguous", S, causal, W, qt, t, lo + n);
                ++n;
            }
        if (fast_q_lo(causal, W, qt) != lo) return fail("fast_q_lo", S, causal, W, qt, fast_q_lo(causal, W, qt), lo);
        if (fast_q_n(S, causal, W, qt) != n) return fail("fast_q_n", S, causal, W, qt, fast_q_n(S, causal, W, qt), n);
        if (fast_q_start(S, causal, W, qt) != start)
            return fail("fast_q_start", S, causal, W, qt, fast_q_start(S, causal, W, qt), start);
        start += n;
    }
    if (fast_q_total(S, causal, W) != start) return fail("fast_q_total", S, causal, W, nqt, fast_q_total(S, causal, W), start);
    // 128-key tiles x 32-row query blocks (x group heads)
    const int nkt = (S + 127) / 128, nb = fast_nb(S);
    start = 0;
    for (int kt = 0; kt <= nkt; ++kt) {
        if (fast_kv_start(S, causal, W, group, kt) != start)
            return fail("fast_kv_start", S, causal, W, kt, fast_kv_start(S, causal, W, group, kt), start);
        if (kt == nkt) break;
        const int k0 = 128 * kt, k1 = std::min(S, k0 + 128) - 1;
        int lo = -1, n = 0;
        for (int qb = 0; qb < nb; ++qb)
            if (pair_in(32 * qb, std::min(S, 32 * qb + 32) - 1, k0, k1, causal, W)) {
                if (lo < 0) lo = qb;
                if (qb != lo + n) return fail("kv blocks not contiguous", S, causal, W, kt, qb, lo + n);
                ++n;
            }
        if (fast_kv_qb0(causal, kt) != lo) return fail("fast_kv_qb0", S, causal, W, kt, fast_kv_qb0(causal, kt), lo);
        if (fast_kv_nqb(S, causal, W, kt) != n)
            return fail("fast_kv_nqb", S, causal, W, kt, fast_kv_nqb(S, causal, W, kt), n);
        if (fast_kv_n(S, causal, W, group, kt) != group * n)
            return fail("fast_kv_n", S, causal, W, kt, fast_kv_n(S, causal, W, group, kt), group * n);
        start += (long long)group * n;
    }
    return 0;
}

}  // namespace

int main() {
    const int Ss[] = {1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 129, 200, 255, 256, 257, 300, 383, 384, 385, 511, 640, 1000};
    const int Ws[] = {0, 1, 2, 31, 32, 33, 63, 64, 65, 66, 96, 127, 128, 129, 130, 191, 192, 255, 256, 257, 300, 512};
    int cases = 0;
    for (int S : Ss)
        for (int causal = 0; causal < 2; ++causal)
            for (int W : Ws) {
                if (W > 0 && (!causal || W >= S)) continue;  // the library normalises these to W = 0
                for (int group : {1, 3}) {
                    if (check(S, causal, W, group)) return 1;
                    ++cases;
                }
            }
    std::printf("ok %d\n", cases);
    return 0;
}
