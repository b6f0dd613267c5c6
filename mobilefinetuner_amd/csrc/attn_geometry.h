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
// iteration fast_q_start(qt).  Work units are contiguous ranges of these
// iterations of about equal cost (UnitSplit).
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
// The tiles of one (batch, head)'s flattened iterations: 128-key tiles of the
// dK/dV role (kv = 1), or 128-row query tiles of the dQ role and the forward.
struct FastTiles {
    int S, causal, W, group, kv;
    __host__ __device__ int nt() const { return (S + 127) / 128; }
    __host__ __device__ int64_t start(int t) const {
        return kv ? fast_kv_start(S, causal, W, group, t) : fast_q_start(S, causal, W, t);
    }
    __host__ __device__ int n(int t) const {
        return kv ? fast_kv_n(S, causal, W, group, t) : fast_q_n(S, causal, W, t);
    }
    __host__ __device__ int64_t total() const { return start(nt() - 1) + n(nt() - 1); }
};

// Work units sized by cost rather than by iteration count.  An iteration
// costs w and each tile costs c more, for what a tile's segment adds
// (loading its rows, storing its outputs or partial, restarting the
// pipeline), so that units covering many short tiles get fewer iterations.
// F(i) = w (i + 1) + c (t(i) + 1) is the cost through iteration i of tile
// t(i), ctot = F(last); unit u of `units` holds the iterations i with
// ceil(F(i) units / ctot) - 1 == u, a contiguous range.
struct UnitSplit {
    int units, w, c;
    int64_t ctot;
};
__host__ __device__ inline UnitSplit make_unit_split(const FastTiles& g, int units, int w, int c) {
    return UnitSplit{units, w, c, (int64_t)w * g.total() + (int64_t)c * g.nt()};
}
// Unit of iteration i, which lies in tile t.
__host__ __device__ inline int unit_of(const UnitSplit& u, int64_t i, int t) {
    const int64_t F = (int64_t)u.w * (i + 1) + (int64_t)u.c * (t + 1);
    return (int)((F * u.units + u.ctot - 1) / u.ctot - 1);
}
// First iteration of unit k (k = units: one past the last iteration): the
// smallest i with F(i) units > k ctot, found in the first tile whose last
// iteration passes the bound.
__host__ __device__ inline int64_t unit_first(const FastTiles& g, const UnitSplit& u, int k) {
    if (k <= 0) return 0;
    if (k >= u.units) return g.total();
    const int64_t target = (int64_t)k * u.ctot;
    int lo = 0, hi = g.nt() - 1;
    while (lo < hi) {
        const int mid = (lo + hi) / 2;
        const int64_t end_cost = (int64_t)u.w * (g.start(mid) + g.n(mid)) + (int64_t)u.c * (mid + 1);
        if (end_cost * u.units > target)
            hi = mid;
        else
            lo = mid + 1;
    }
    const int64_t s0 = g.start(lo);
    const int64_t num = target - (int64_t)u.c * (lo + 1) * u.units;
    const int64_t i = num < 0 ? 0 : num / ((int64_t)u.w * u.units);
    return i > s0 ? i : s0;
}
// Units that touch tile t (first: *u0).
__host__ __device__ inline int tile_units(const FastTiles& g, const UnitSplit& u, int t, int* u0) {
    const int64_t s = g.start(t);
    *u0 = unit_of(u, s, t);
    return unit_of(u, s + g.n(t) - 1, t) - *u0 + 1;
}
__host__ __device__ inline int tile_units(const FastTiles& g, const UnitSplit& u, int t) {
    int u0;
    return tile_units(g, u, t, &u0);
}
// A split over `units` units with the planners' limits: every unit at least
// kMin iterations and no tile over kMaxSlots units; units is lowered until
// both hold (one unit always does).  *parts_max: the most units of a tile.
inline UnitSplit fit_unit_split(const FastTiles& g, int64_t units, int w, int c, int kMin, int kMaxSlots,
                                int* parts_max) {
    const int64_t n = g.total();
    if (units > n / kMin) units = n / kMin;
    if (units < 1) units = 1;
    for (;; units = units * 15 / 16 < units - 1 ? units * 15 / 16 : units - 1) {
        const UnitSplit u = make_unit_split(g, (int)units, w, c);
        int pm = 1;
        for (int t = 0; t < g.nt(); ++t) {
            const int k = tile_units(g, u, t);
            pm = k > pm ? k : pm;
        }
        bool ok = pm <= kMaxSlots;
        for (int k = 0; ok && k < u.units; ++k) ok = unit_first(g, u, k + 1) - unit_first(g, u, k) >= kMin;
        if (ok || units == 1) {
            *parts_max = pm;
            return u;
        }
    }
}

// Partial slots.  A work unit has at most two segments in split tiles: the
// tile holding its first iteration and the tile holding its last.  Unit u of
// a (batch, head) keeps their partials in slots 2u (first segment) and 2u + 1
// (last segment, when it differs from the first).  For a split tile touched
// by units u0 .. u1, unit u's partial is in slot split_slot(u, u0, starts):
// the tile is the first segment of every unit except possibly u0, whose last
// segment it is when the tile starts inside u0 (starts: the tile begins at
// u0's first iteration).
__host__ __device__ inline int64_t split_slot(int64_t u, int64_t u0, bool starts) {
    return 2 * u + ((u == u0 && !starts) ? 1 : 0);
}

// XCD-aware block order.  The dispatcher hands workgroup i of a launch to
// XCD i % kXcds, and each XCD has its own L2.  xcd_block(i, n) renumbers the
// n workgroups so that XCD x runs one contiguous range of logical indices:
// work units with neighbouring indices (which read the same K/V or Q tiles)
// then share one L2.  A bijection of [0, n) whatever the dispatch order, so
// only the cache behaviour depends on it.
constexpr int kXcds = 8;
__host__ __device__ inline int xcd_block(int i, int n) {
    const int x = i % kXcds, k = i / kXcds, q = n / kXcds, r = n % kXcds;
    return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + k;
}

}  // namespace mft
