// Work geometry of the bf16 fast kernels, shared by host planning and device
// code (identical formulas on both sides).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mft {

// Fast-path work geometry (host and device use the same formulas).
//
// Visibility: key j is visible to query row i iff j <= i (causal), i - j < W
// (causal sliding window of W keys, W > 0; W = 0: none) and j < len_b (key
// padding, per batch; not part of the geometry, masked inside the tiles).
// The geometry only visits tiles that the causal window can reach:
//
// dK/dV: per (batch, kv head) the iterations (128-key tile kt, query head of
// the group, 32-row query block) are flattened kt-major; tile kt holds
// fast_kv_n(kt) = G * nqb(kt) of them starting at fast_kv_start(kt), its
// query blocks are fast_kv_qb0(kt) .. + nqb(kt) - 1 (head-major inside the
// tile).  dQ and forward: per (batch, query head) the iterations (128-row
// query tile qt, 64-key tile) are flattened qt-major; tile qt holds
// fast_q_n(qt) key tiles fast_q_lo(qt) .. + fast_q_n(qt) - 1 starting at
// iteration fast_q_start(qt).  Work units are equal chunks of these ranges.
__host__ __device__ inline int fast_nb(int S) { return (S + 31) / 32; }

// 64-key tiles a 128-row query tile reaches back beyond its own two:
// ceil((W - 1) / 64), "unbounded" without a window.
__host__ __device__ inline int win_back64(int causal, int W) {
    return (causal && W > 0) ? (W - 1 + 63) / 64 : (1 << 28);
}
// 32-row query blocks a 128-key tile reaches (causal window): the rows
// 128 kt .. 128 kt + 127 + W - 1.
__host__ __device__ inline int win_qblocks(int causal, int W) {
    return (causal && W > 0) ? (126 + W) / 32 + 1 : (1 << 28);
}
__host__ __device__ inline int fast_kv_qb0(int causal, int kt) { return causal ? 4 * kt : 0; }
__host__ __device__ inline int fast_kv_nqb(int S, int causal, int W, int kt) {
    return causal ? min(fast_nb(S) - 4 * kt, win_qblocks(causal, W)) : fast_nb(S);
}
__host__ __device__ inline int fast_kv_n(int S, int causal, int W, int group, int kt) {
    return group * fast_kv_nqb(S, causal, W, kt);
}
// sum_{k < kt} nqb(k): nqb(k) = min(nb - 4k, cmax) is cmax for k < K1 and
// nb - 4k after.
__host__ __device__ inline int64_t fast_kv_start(int S, int causal, int W, int group, int kt) {
    const int64_t nb = fast_nb(S);
    if (!causal) return (int64_t)group * nb * kt;
    const int64_t cmax = win_qblocks(causal, W);
    const int64_t K1 = nb >= cmax ? (nb - cmax) / 4 + 1 : 0;
    const int64_t m = kt < K1 ? kt : K1;
    return group * (m * cmax + (kt - m) * nb - 2 * ((int64_t)kt * (kt - 1) - m * (m - 1)));
}
__host__ __device__ inline int fast_q_lo(int causal, int W, int qt) {
    const int c = win_back64(causal, W);
    return 2 * qt > c ? 2 * qt - c : 0;
}
__host__ __device__ inline int fast_q_n(int S, int causal, int W, int qt) {
    const int kend = causal ? min(S, 128 * (qt + 1)) : S;
    return (kend + 63) / 64 - fast_q_lo(causal, W, qt);
}
// Iterations before query tile qt, counting every earlier tile as full:
// min(2q + 2, c + 2) key tiles for tile q; the first r = min(qt, c/2 + 1)
// tiles are 2q + 2, the rest c + 2.
__host__ __device__ inline int64_t fast_q_start(int S, int causal, int W, int qt) {
    if (!causal) return (int64_t)qt * ((S + 63) / 64);
    const int64_t c = win_back64(causal, W);
    const int64_t r = qt < c / 2 + 1 ? qt : c / 2 + 1;
    return r * (r + 1) + (qt - r) * (c + 2);
}
// Total iterations of one (batch, head): the start formula counts every tile
// as full, which overcounts when the last tile is partial, so the total is
// the last tile's start plus its own count.
__host__ __device__ inline int64_t fast_q_total(int S, int causal, int W) {
    const int nqt = (S + 127) / 128;
    return fast_q_start(S, causal, W, nqt - 1) + fast_q_n(S, causal, W, nqt - 1);
}
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
