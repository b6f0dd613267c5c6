// Work geometry of the bf16 fast kernels, shared by host planning and device
// code (identical formulas on both sides).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mft {

// Fast-path work geometry (host and device use the same formulas).
// dK/dV: per (batch, kv head) the iterations (128-key tile kt, query head of
// the group, 32-row query block) are flattened kt-major; tile kt holds
// fast_kv_n(kt) of them starting at fast_kv_start(kt).  dQ: per (batch, query
// head) the iterations (128-row query tile qt, 64-key tile) are flattened
// qt-major.  Work units are equal chunks of these ranges.
__host__ __device__ inline int fast_nb(int S) { return (S + 31) / 32; }
__host__ __device__ inline int fast_kv_n(int S, int causal, int group, int kt) {
    return group * (causal ? fast_nb(S) - 4 * kt : fast_nb(S));
}
__host__ __device__ inline int64_t fast_kv_start(int S, int causal, int group, int kt) {
    const int64_t nb = fast_nb(S);
    return causal ? group * (kt * nb - 2 * (int64_t)kt * (kt - 1)) : (int64_t)group * nb * kt;
}
__host__ __device__ inline int fast_q_n(int S, int causal, int qt) {
    const int kend = causal ? min(S, 128 * (qt + 1)) : S;
    return (kend + 63) / 64;
}
__host__ __device__ inline int64_t fast_q_start(int S, int causal, int qt) {
    return causal ? (int64_t)qt * (qt + 1) : (int64_t)qt * ((S + 63) / 64);
}
// The same query-tile geometry for BM-row query tiles (BM a multiple of 128):
// tile qt holds fastw_q_n<BM>(qt) 64-key tiles, starting at iteration
// fastw_q_start<BM>(qt).  BM = 128 is fast_q_n / fast_q_start.
template <int BM> __host__ __device__ inline int fastw_q_n(int S, int causal, int qt) {
    const int kend = causal ? min(S, BM * (qt + 1)) : S;
    return (kend + 63) / 64;
}
template <int BM> __host__ __device__ inline int64_t fastw_q_start(int S, int causal, int qt) {
    static_assert(BM % 128 == 0, "query tiles of whole 128-row blocks");
    return causal ? (int64_t)(BM / 128) * qt * (qt + 1) : (int64_t)qt * ((S + 63) / 64);
}
// Total iterations of one (batch, head): the start formula counts every tile
// as full, which overcounts when the last tile is partial, so the total is
// the last tile's start plus its own count.
template <int BM> __host__ __device__ inline int64_t fastw_q_total(int S, int causal) {
    const int nqt = (S + BM - 1) / BM;
    return fastw_q_start<BM>(S, causal, nqt - 1) + fastw_q_n<BM>(S, causal, nqt - 1);
}
__host__ __device__ inline int64_t fast_q_total(int S, int causal) { return fastw_q_total<128>(S, causal); }
// Work units per (batch, head) for `pairs` independent (batch, head) ranges
// on `cus` compute units, one workgroup per CU at a time: the u that
// minimises ceil(pairs * u / cus) * (1 / u + 0.02), i.e. rounds of
// workgroups times the unit length plus a fixed per-unit cost (loading the
// rows, writing outputs or partials) of 2% of a (batch, head)'s work; the
// smallest such u.
__host__ __device__ inline int64_t balanced_units(int64_t pairs, int64_t cus) {
    int64_t best = 1;
    double best_t = 1e300;
    const int64_t umax = (4 * cus + pairs - 1) / pairs;
    for (int64_t u = 1; u <= umax; ++u) {
        const double t = (double)((pairs * u + cus - 1) / cus) * (1.0 / (double)u + 0.02);
        if (t < best_t * (1.0 - 1e-9)) {
            best_t = t;
            best = u;
        }
    }
    return best;
}
// Units [first, last] of chunk size `chunk` that touch the range [start, start + n).
__host__ __device__ inline int fast_slots(int64_t start, int n, int64_t chunk) {
    return (int)((start + n - 1) / chunk - start / chunk + 1);
}

// Partial slots.  A work unit has at most two segments in split tiles: the
// tile holding its first iteration and the tile holding its last.  Unit u of
// a (batch, head) keeps their partials in slots 2u (first segment) and 2u + 1
// (last segment, when it differs from the first).  For a split tile starting
// at iteration `start`, touched by units u0 = start / chunk .. u1, unit u's
// partial is in slot split_slot(start, chunk, u, u0): the tile is the first
// segment of every unit except possibly u0 (when the tile starts inside u0).
__host__ __device__ inline int64_t split_slot(int64_t start, int64_t chunk, int64_t u, int64_t u0) {
    return 2 * u + ((u == u0 && start % chunk != 0) ? 1 : 0);
}

}  // namespace mft
