// fp32 fast path of the attention forward and backward (fp32 q, k, v, o and
// dO; D % 4 == 0, 32 < D <= 256), on v_mfma_f32_16x16x4_f32.
//
// It runs the same work decomposition as the bf16 fast path (attn_geometry.h:
// 128-row query tiles x 64-key tiles for the forward and the dQ role, 128-key
// tiles x 32-row query blocks for the dK/dV role, cut into units of about
// equal cost), the same fp32 partial slots for split tiles, the forward
// combine and the backward REDUCE.  What differs:
//   - every unit runs as two workgroups, one per 64-row (dQ, forward) or
//     64-key (dK/dV) half of the tile, 4 waves x 16 rows or keys.  An fp32
//     row of D = 256 is 1 KiB, so a wave's 16 K and 16 V rows (dK/dV), or 16
//     Q and 16 dO rows (dQ), fit in 128 registers, next to 128 of
//     accumulators; with 32 per wave they would not;
//   - fp32 MFMAs take 16x the time of bf16 ones per flop, so LDS reads are
//     far from a bound: every operand is read from plain row-major tiles (no
//     transposing reads), with one 16-byte read per four MFMAs.
//
// v_mfma_f32_16x16x4_f32 operand layout, lane l = 16 g + i:
//   A (16 x 4): lane holds A[i][g];  B (4 x 16): lane holds B[g][i];
//   C (16 x 16): lane holds C[4 g + r][i] in register r (r = 0..3).
// A reduction index only has to be assigned to the same (g, step) in A and B.
// Dot products over d take a 16-byte chunk (4 consecutive d) per lane and
// step: MFMA (c, e) of a chain puts d = 16 c + 4 g + e in slot g.  Products
// whose output runs over d (O, dQ, dK, dV) assign output index m of tile
// (u, j) to d = 64 u + 4 m + j, so that one 16-byte read of a row feeds the
// four tiles j = 0..3 and a lane ends up with 4 consecutive d per tile group.
//
// LDS tiles are row-major fp32 rows of DPF floats whose 16-byte chunks are
// XOR-swizzled by row (chunk c of row r at c ^ (r & 15)): both access
// patterns (16 rows x one chunk, one row x 16 chunks per 16 lanes) then hit
// 16 distinct bank groups.  They are filled with global_load_lds_dwordx4 by
// the bf16 path's TileDma, viewing an fp32 row as 2 * DPF bf16 columns.
//
// The kernels are instantiated per padded head dim in attn_f32_fast64.hip,
// attn_f32_fast128.hip and, split by role and causal mode,
// attn_f32_fast256*.hip, so they compile in parallel.
#pragma once
#include "attn_bwd_fast.h"
#include "attn_fwd_fast.h"

namespace mft {
namespace f32 {

using bwd::BwdArgs;
using fwd::FwdArgs;
using fwd::kFwdBM;
using fwd::kFwdBN;

__device__ __forceinline__ f32x4 mma(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
// A zero accumulator the compiler does not see as a constant: a builtin MFMA
// chain that starts from a literal-zero accumulator may get result registers
// that overlap its A/B operands (ROCm 7.2; see mfma_v_first).
__device__ __forceinline__ f32x4 zero4() {
    f32x4 z = {0.f, 0.f, 0.f, 0.f};
    asm volatile("" : "+v"(z));
    return z;
}

// Byte offset of 16-byte chunk c of row r in a swizzled fp32 tile of DPF
// floats per row (swz_row of the bf16 view: CPR = DPF / 4 >= 16 chunks).
template <int DPF> __device__ __forceinline__ uint32_t toff(int r, int c) {
    return (uint32_t)r * (DPF * 4) + 16u * (uint32_t)(c ^ (r & 15));
}
template <int DPF> __device__ __forceinline__ f32x4 tread(const char* tile, int r, int c) {
    return *reinterpret_cast<const f32x4*>(tile + toff<DPF>(r, c));
}

// Direct loads of an fp32 tile of ROWS rows (row0.., row stride ld floats, D
// valid columns) into a swizzled LDS tile; load j of this thread's PER.
template <int DPF, int ROWS> using F32Dma = TileDma<2 * DPF, ROWS, 256, SWZ_ROW>;
// src and row0 are wave-uniform; they pass through readfirstlane so that the
// compiler keeps them in scalar registers (the instruction's address base).
// readfirstlane returns a signed int: each half goes through uint32_t, or the
// low half would sign-extend over the high one.
__device__ __forceinline__ uint64_t uniform_u64(uint64_t p) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)p);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(p >> 32));
    return ((uint64_t)hi << 32) | (uint64_t)lo;
}
template <bool FAST, int DPF, int ROWS>
__device__ __forceinline__ void issue_f32(const F32Dma<DPF, ROWS>& t, const float* src, int row0, int S, int D,
                                          int ld, float* tile, int j) {
    const uint64_t pu = uniform_u64(reinterpret_cast<uint64_t>(src));
    src = reinterpret_cast<const float*>(pu);
    row0 = __builtin_amdgcn_readfirstlane(row0);
    issue_tile_j<FAST, 2 * DPF, ROWS, 256, SWZ_ROW>(t, reinterpret_cast<const bf16*>(src), row0, S, 2 * D, 2 * ld,
                                                    reinterpret_cast<bf16*>(tile), lds_addr(tile), j);
}

// This lane's 16-byte chunks 16 c + 4 g of a global row (zeros past D, and for
// rows that do not exist).
template <int NC>
__device__ __forceinline__ void load_row(f32x4 (&f)[NC], const float* row, bool ok, int D, bool vec_ok) {
    const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
    for (int c = 0; c < NC; ++c) f[c] = load_chunk<float>(row, 16 * c + 4 * g, D, ok, vec_ok);
}

// Store of a transposed-output accumulator set (tiles (u, j), lane (i, g)
// holding output row i at d = 64 u + 16 g + 4 r + j in register r): per (u, r)
// one 16-byte store of 4 consecutive d.
template <int NU>
__device__ __forceinline__ void store_rowT(float* row, const f32x4 (&acc)[4 * NU], int D, float scale) {
    const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
    for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int d0 = 64 * u + 16 * g + 4 * r;
            if (d0 < D)
                *reinterpret_cast<f32x4*>(row + d0) =
                    f32x4{acc[4 * u][r] * scale, acc[4 * u + 1][r] * scale, acc[4 * u + 2][r] * scale,
                          acc[4 * u + 3][r] * scale};
        }
}

// Store of a key-major accumulator set (tiles (u, j), lane (i, g) holding row
// 4 g + r at d = 64 u + 4 i + j): rows base + (4 g + r) * ld.
template <int NU>
__device__ __forceinline__ void store_rows(float* base, int64_t ld, const f32x4 (&acc)[4 * NU], int D, float scale,
                                           int rows_ok) {
    const int lane = threadIdx.x & 63, i = lane & 15, g = lane >> 4;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        if (4 * g + r >= rows_ok) continue;
        float* row = base + (int64_t)(4 * g + r) * ld;
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const int d0 = 64 * u + 4 * i;
            if (d0 < D)
                *reinterpret_cast<f32x4*>(row + d0) =
                    f32x4{acc[4 * u][r] * scale, acc[4 * u + 1][r] * scale, acc[4 * u + 2][r] * scale,
                          acc[4 * u + 3][r] * scale};
        }
    }
}

// An unrolled chain of NI steps: step i reads its operands (R LDS reads)
// PF steps ahead into a ring, then issues its M MFMAs.  The order is pinned
// (pin_read_ahead): left alone, the scheduler either puts each read next to
// its MFMA (exposing the LDS latency) or hoists them all (spilling).
template <int NI, int PF, int R, int M, class Ops, class Read, class Step>
__device__ __forceinline__ void chain(Read read, Step step) {
    Ops ring[PF];
#pragma unroll
    for (int i = 0; i < PF; ++i) ring[i] = read(i);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const Ops o = ring[i % PF];
        if (i + PF < NI) ring[i % PF] = read(i + PF);
        step(i, o);
    }
    pin_read_ahead<NI, PF, R, M>();
}
template <int N> struct Ops {
    f32x4 v[N];
};
constexpr int kPF = 2;

// ===========================================================================
// Forward.  Workgroup = (unit, half): 4 waves x 16 query rows, the rows
// 64 half .. 64 half + 63 of every 128-row query tile of the unit; lane (i, g)
// owns query row 16 w + i.  Per 64-key tile:
//   S^T = K Q^T  (A = K rows from LDS, B = Q from registers), 4 key blocks kb;
//   online softmax in exp2 (the row's 64 scores sit in lanes i, i+16, i+32,
//   i+48);
//   O^T += V^T P^T (A = V rows from LDS, B = the exp'd scores as they are).
// K and V have one LDS buffer each: V of tile i streams in during S^T of
// tile i, K of tile i+1 during P.V of tile i.
template <int DPF, bool CAUSAL, bool FAST>
__global__ __launch_bounds__(256) void attn_fwd_f32_split(FwdArgs a) {
    constexpr int BN = kFwdBN, BM = kFwdBM, NC = DPF / 16, NU = DPF / 64;
    typedef F32Dma<DPF, BN> TD;
    __shared__ __attribute__((aligned(1024))) float smem[2 * BN * DPF];
    float* Kt = smem;
    float* Vt = smem + BN * DPF;

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, i16 = lane & 15, g = lane >> 4;
    const int S = a.S, D = a.D, W = a.window;
    const int bh = a.B * a.Hq, blk = xcd_block((int)blockIdx.x, (int)gridDim.x);  // XCD-major order
    const int unit = blk / (2 * bh), half = (blk / bh) & 1, b = (blk % bh) / a.Hq, h = (blk % bh) % a.Hq;
    const int hk = h / a.group;
    const float* Q = (const float*)a.q + a.sq.at(b, h);
    const float* K = (const float*)a.k + a.sk.at(b, hk);
    const float* V = (const float*)a.v + a.sv.at(b, hk);
    const int lq = a.sq.s, lk = a.sk.s, lv = a.sv.s;
    const bool vec_ok = a.vec_ok != 0;
    TD dk_, dv_;
    dk_.init(lane, wave_id(), 2 * lk);
    dv_.init(lane, wave_id(), 2 * lv);
    const KeyVis vis{S, W, a.kv_len ? min(max(a.kv_len[b], 0), S) : S, CAUSAL};

    const FastTiles tiles{S, CAUSAL, W, a.group, 0};
    const int64_t g0 = unit_first(tiles, a.us, unit);
    const int niter = (int)(unit_first(tiles, a.us, unit + 1) - g0);
    int qt = 0;
    while (fast_q_start(S, CAUSAL, W, qt + 1) <= g0) ++qt;
    int pf_qt = qt, pf_t = (int)(g0 - fast_q_start(S, CAUSAL, W, qt)), pf_n = fast_q_n(S, CAUSAL, W, qt);
    int pf_lo = fast_q_lo(CAUSAL, W, qt);
    auto next_key_tile = [&]() {
        const int t = pf_lo + pf_t;
        if (++pf_t == pf_n) {
            ++pf_qt;
            pf_t = 0;
            pf_n = fast_q_n(S, CAUSAL, W, pf_qt);
            pf_lo = fast_q_lo(CAUSAL, W, pf_qt);
        }
        return t;
    };
    {
        const int k0 = next_key_tile() * BN;
#pragma unroll
        for (int j = 0; j < TD::PER; ++j) issue_f32<FAST, DPF, BN>(dk_, K, k0, S, D, lk, Kt, j);
    }
    int64_t qstart = fast_q_start(S, CAUSAL, W, qt);
    int qn = fast_q_n(S, CAUSAL, W, qt);
    int qlo = fast_q_lo(CAUSAL, W, qt);
    f32x4 qf[NC];
    {
        const int row = qt * BM + 64 * half + 16 * w + i16;
        load_row<NC>(qf, Q + (int64_t)min(row, S - 1) * lq, row < S, D, vec_ok);
    }
    wait_vmcnt<0>();

    f32x4 oacc[4 * NU];
    for (int i = 0, first = 1;; first = 0) {
#pragma unroll
        for (int t = 0; t < 4 * NU; ++t) oacc[t] = zero4();
        float m_run = -INFINITY, l_run = 0.f;
        const int wrow0 = qt * BM + 64 * half + 16 * w, row = wrow0 + i16;
        const int vlo = vis.lo(row), vhi = vis.hi(row);
        const int seg_end = (int)min((int64_t)niter, qstart + qn - g0);
        for (; i < seg_end; ++i) {
            const int kbase = (qlo + (int)(g0 + i - qstart)) * BN;
            // K of this tile has landed everywhere; every wave is done with V.
            wait_vmcnt<0>();
            lds_barrier();
#pragma unroll
            for (int j = 0; j < TD::PER; ++j) issue_f32<FAST, DPF, BN>(dv_, V, kbase, S, D, lv, Vt, j);
            const bool active =
                wave_uniform(wrow0 < S && vis.any(wrow0, min(wrow0 + 15, S - 1), kbase, kbase + BN - 1));
            f32x4 st[4];
            if (active) {
                const char* kt = reinterpret_cast<const char*>(Kt);
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) st[kb] = zero4();
                chain<NC, kPF, 4, 16, Ops<4>>(
                    [&](int c) {
                        Ops<4> o;
#pragma unroll
                        for (int kb = 0; kb < 4; ++kb) o.v[kb] = tread<DPF>(kt, 16 * kb + i16, 4 * c + g);
                        return o;
                    },
                    [&](int c, const Ops<4>& o) {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
#pragma unroll
                            for (int kb = 0; kb < 4; ++kb) st[kb] = mma(o.v[kb][e], qf[c][e], st[kb]);
                    });
                // online softmax of row `row` over this tile's keys
                const bool need_mask = wave_uniform(!vis.all(wrow0, wrow0 + 15, kbase, kbase + BN - 1));
                float mx = -INFINITY;
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float x = st[kb][r] * a.scale_log2;
                        if (need_mask) {
                            const int key = kbase + 16 * kb + 4 * g + r;
                            if (key < vlo || key > vhi) x = -INFINITY;
                        }
                        st[kb][r] = x;
                        mx = fmaxf(mx, x);
                    }
                mx = half_max(row16_max(mx));
                // Lazy rescaling (as the bf16 kernels): the reference point
                // m_run moves, and O and l are rescaled, only when some row
                // of the wave sees a max above m_run + 8, so exp2 arguments
                // stay <= 8.  O = acc / l and LSE = m_run + log2(l) are the
                // same for any reference point; most tiles skip the rescale
                // of the accumulators (which live in AGPRs: a read, a
                // multiply and a write each).
                if (__any(mx > m_run + kLazyRescale)) {
                    const float m_new = fmaxf(m_run, mx);
                    const float alpha = fast_exp2(m_run - (m_new == -INFINITY ? 0.f : m_new));
                    m_run = m_new;
                    l_run *= alpha;
#pragma unroll
                    for (int t = 0; t < 4 * NU; ++t) oacc[t] *= alpha;
                }
                const float msub = m_run == -INFINITY ? 0.f : m_run;
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float p = fast_exp2(st[kb][r] - msub);
                        l_run += p;
                        st[kb][r] = p;
                    }
            }
            // V has landed everywhere; every wave is done with K.
            wait_vmcnt<0>();
            lds_barrier();
            if (i + 1 < niter) {
                const int kn = next_key_tile() * BN;
#pragma unroll
                for (int j = 0; j < TD::PER; ++j) issue_f32<FAST, DPF, BN>(dk_, K, kn, S, D, lk, Kt, j);
            }
            if (active) {
                const char* vt = reinterpret_cast<const char*>(Vt);
                // O^T(u, j) += V^T P^T: step (kb, r) takes keys 16 kb + 4 g + r
                chain<16, kPF, NU, 4 * NU, Ops<NU>>(
                    [&](int s) {
                        Ops<NU> o;
#pragma unroll
                        for (int u = 0; u < NU; ++u) o.v[u] = tread<DPF>(vt, 16 * (s >> 2) + 4 * g + (s & 3), 16 * u + i16);
                        return o;
                    },
                    [&](int s, const Ops<NU>& o) {
#pragma unroll
                        for (int u = 0; u < NU; ++u)
#pragma unroll
                            for (int j = 0; j < 4; ++j) oacc[4 * u + j] = mma(o.v[u][j], st[s >> 2][s & 3], oacc[4 * u + j]);
                    });
            }
        }
        // End of this unit's part of query tile qt: normalised O and LSE, or
        // this unit's partial (unnormalised O, running max, sum).
        const bool more = i < niter;
        const int nsl = tile_units(tiles, a.us, qt);
        const float l_tot = half_sum(row16_sum(l_run));
        if (row < S) {
            if (nsl <= 1) {
                const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
                store_rowT<NU>((float*)a.o + a.so.at(b, h) + (int64_t)row * a.so.s, oacc, D, inv);
                if (a.lse && g == 0)
                    a.lse[(int64_t)(b * a.Hq + h) * S + row] = l_tot > 0.f ? (m_run + log2f(l_tot)) * kLn2 : INFINITY;
            } else {
                const int64_t slot = (int64_t)(b * a.Hq + h) * 2 * a.us.units + 2 * unit + (first ? 0 : 1);
                const int64_t prow = slot * BM + 64 * half + 16 * w + i16;
                store_rowT<NU>(a.part_o + prow * D, oacc, D, 1.f);
                if (g == 0) {
                    a.part_ml[prow * 2] = m_run;
                    a.part_ml[prow * 2 + 1] = l_tot;
                }
            }
        }
        if (!more) {
            wait_vmcnt<0>();  // no direct load is in flight when the workgroup ends
            break;
        }
        ++qt;
        qstart = fast_q_start(S, CAUSAL, W, qt);
        qn = fast_q_n(S, CAUSAL, W, qt);
        qlo = fast_q_lo(CAUSAL, W, qt);
        const int nrow = qt * BM + 64 * half + 16 * w + i16;
        load_row<NC>(qf, Q + (int64_t)min(nrow, S - 1) * lq, nrow < S, D, vec_ok);
    }
}

// ===========================================================================
// Backward, dK/dV role.  Workgroup = (unit, half): 4 waves x 16 keys, the keys
// 64 half .. 64 half + 63 of every 128-key tile of the unit; lane (i, g) holds
// K and V of key 16 w + i in registers.  Per iteration (query head, 32-row
// query block), with Q, dO and the block's row terms double-buffered in LDS:
//   S = Q K^T, dP = dO V^T  (A = Q, dO rows from LDS, B = K, V registers),
//   two 16-row halves qa;
//   P = exp2(S scale log2e - lse log2e), dS = P (dP - delta);
//   dV += P^T dO, dK += dS^T Q  (A = P, dS as they are, B = dO, Q rows).
template <int DPF> struct KvLds {
    static constexpr int TILE = 32 * DPF;                 // floats of a Q or dO block
    static constexpr int ST_OFF = 4 * TILE, ST = 64;      // [Q0][Q1][dO0][dO1][stats0][stats1]
    static constexpr int FLOATS = ST_OFF + 2 * ST;
};
template <int DPF> struct QLds {
    static constexpr int TILE = 64 * DPF;  // [K][V]
    static constexpr int FLOATS = 2 * TILE;
};
template <int DPF> constexpr int main_lds_floats() {
    return KvLds<DPF>::FLOATS > QLds<DPF>::FLOATS ? KvLds<DPF>::FLOATS : QLds<DPF>::FLOATS;
}

template <int DPF, bool CAUSAL, bool FAST>
__device__ __forceinline__ void dkdv_f32_body(const BwdArgs& a, float* smem, int unit, int half, int b, int hk) {
    typedef KvLds<DPF> L;
    typedef F32Dma<DPF, 32> TD;
    constexpr int BNK = 128, NC = DPF / 16, NU = DPF / 64;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, i16 = lane & 15, g = lane >> 4;
    const int S = a.S, D = a.D, G = a.group, W = a.window;
    const bool vec_ok = a.vec_ok != 0;
    const KeyVis vis = bwd::key_vis(a, b, CAUSAL);
    const float* K = (const float*)a.k + a.sk.at(b, hk);
    const float* V = (const float*)a.v + a.sv.at(b, hk);
    const int lk = a.sk.s, lv = a.sv.s;
    TD dq_, dg_;
    dq_.init(lane, wave_id(), 2 * a.sq.s);
    dg_.init(lane, wave_id(), 2 * a.sdo.s);

    const FastTiles tiles{S, CAUSAL, W, G, 1};
    const int64_t g0 = unit_first(tiles, a.kv_us, unit);
    const int niter = (int)(unit_first(tiles, a.kv_us, unit + 1) - g0);
    int kt = 0;
    while (fast_kv_start(S, CAUSAL, W, G, kt + 1) <= g0) ++kt;
    // prefetch cursor: key tile, query head of the group, query block
    int pf_kt = kt, pf_nqb = fast_kv_nqb(S, CAUSAL, W, kt), pf_h, pf_qi;
    {
        const int it0 = (int)(g0 - fast_kv_start(S, CAUSAL, W, G, kt));
        pf_h = it0 / pf_nqb;
        pf_qi = it0 - pf_h * pf_nqb;
    }
    // Issues the next block's loads into buffer par; returns its first row.
    auto issue = [&](int par) {
        const int h = hk * G + pf_h, qb = (CAUSAL ? pf_kt * BNK : 0) + pf_qi * 32;
        if (++pf_qi == pf_nqb) {
            pf_qi = 0;
            if (++pf_h == G) {
                pf_h = 0;
                ++pf_kt;
                pf_nqb = fast_kv_nqb(S, CAUSAL, W, pf_kt);
            }
        }
        const float* q = (const float*)a.q + a.sq.at(b, h);
        const float* go = (const float*)a.dO + a.sdo.at(b, h);
#pragma unroll
        for (int j = 0; j < TD::PER; ++j) {
            issue_f32<FAST, DPF, 32>(dq_, q, qb, S, D, a.sq.s, smem + par * L::TILE, j);
            issue_f32<FAST, DPF, 32>(dg_, go, qb, S, D, a.sdo.s, smem + (2 + par) * L::TILE, j);
        }
        // the block's row terms: 256 bytes, lanes 0..15 of wave 0
        if (threadIdx.x < 16)
            load_lds_16(a.stats + ((int64_t)(b * a.Hq + h) * a.nqb_total + qb / 32) * 64 + 4 * threadIdx.x,
                        smem + L::ST_OFF + par * L::ST);
        return qb;
    };

    f32x4 kf[NC], vf[NC];
    auto load_keys = [&](int t) {
        const int key = t * BNK + 64 * half + 16 * w + i16, keyc = min(key, S - 1);
        load_row<NC>(kf, K + (int64_t)keyc * lk, key < S, D, vec_ok);
        load_row<NC>(vf, V + (int64_t)keyc * lv, key < S, D, vec_ok);
    };
    load_keys(kt);
    int cur_qb = issue(0);
    wait_vmcnt<0>();

    f32x4 dk[4 * NU], dv[4 * NU];
#pragma unroll
    for (int t = 0; t < 4 * NU; ++t) {
        dk[t] = zero4();
        dv[t] = zero4();
    }
    int64_t kstart = fast_kv_start(S, CAUSAL, W, G, kt);
    int kn = fast_kv_n(S, CAUSAL, W, G, kt);
    for (int i = 0, first = 1;; first = 0) {
        const int seg_end = (int)min((int64_t)niter, kstart + kn - g0);
        const int wkey0 = kt * BNK + 64 * half + 16 * w, key = wkey0 + i16;
        for (; i < seg_end; ++i) {
            const int par = i & 1;
            // this block has landed everywhere; every wave is done with the other buffer
            wait_vmcnt<0>();
            lds_barrier();
            const int qb = cur_qb;
            if (i + 1 < niter) cur_qb = issue(par ^ 1);
            if (!wave_uniform(wkey0 < S && vis.any(qb, min(qb + 31, S - 1), wkey0, min(wkey0 + 15, S - 1))))
                continue;
            const char* qt = reinterpret_cast<const char*>(smem + par * L::TILE);
            const char* gt = reinterpret_cast<const char*>(smem + (2 + par) * L::TILE);
            const float* stt = smem + L::ST_OFF + par * L::ST;
            f32x4 sc[2], dp[2];
#pragma unroll
            for (int qa = 0; qa < 2; ++qa) {
                sc[qa] = zero4();
                dp[qa] = zero4();
            }
            // step c: [Q qa0, Q qa1, dO qa0, dO qa1] chunks 4 c + g
            chain<NC, kPF, 4, 16, Ops<4>>(
                [&](int c) {
                    Ops<4> o;
#pragma unroll
                    for (int qa = 0; qa < 2; ++qa) {
                        o.v[qa] = tread<DPF>(qt, 16 * qa + i16, 4 * c + g);
                        o.v[2 + qa] = tread<DPF>(gt, 16 * qa + i16, 4 * c + g);
                    }
                    return o;
                },
                [&](int c, const Ops<4>& o) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
#pragma unroll
                        for (int qa = 0; qa < 2; ++qa) {
                            sc[qa] = mma(o.v[qa][e], kf[c][e], sc[qa]);
                            dp[qa] = mma(o.v[2 + qa][e], vf[c][e], dp[qa]);
                        }
                });
            // register r of half qa: query row qb + 16 qa + 4 g + r, key `key`
            const bool need_mask = wave_uniform(!vis.all(qb, qb + 31, wkey0, wkey0 + 15));
            const int r_lo = vis.rlo(key) - qb, r_hi = vis.rhi(key) - qb;
#pragma unroll
            for (int qa = 0; qa < 2; ++qa) {
                const f32x4 l4 = *reinterpret_cast<const f32x4*>(stt + 16 * qa + 4 * g);
                const f32x4 d4 = *reinterpret_cast<const f32x4*>(stt + 32 + 16 * qa + 4 * g);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float p = fast_exp2(sc[qa][r] * a.scale_log2 - l4[r]);
                    if (need_mask) {
                        const int rr = 16 * qa + 4 * g + r;
                        if (rr < r_lo || rr >= r_hi) p = 0.f;
                    }
                    sc[qa][r] = p;
                    dp[qa][r] = p * (dp[qa][r] - d4[r]);
                }
            }
            // dV(u, j) += P^T dO, dK(u, j) += dS^T Q: step (qa, r, u) reads dO and
            // Q of block row 16 qa + 4 g + r, chunk 16 u + i (the d-range of tiles (u, *))
            chain<8 * NU, kPF, 2, 8, Ops<2>>(
                [&](int st8) {
                    const int row = 16 * (st8 / (4 * NU)) + 4 * g + ((st8 / NU) & 3), u = st8 % NU;
                    Ops<2> o;
                    o.v[0] = tread<DPF>(gt, row, 16 * u + i16);
                    o.v[1] = tread<DPF>(qt, row, 16 * u + i16);
                    return o;
                },
                [&](int st8, const Ops<2>& o) {
                    const int qa = st8 / (4 * NU), r = (st8 / NU) & 3, u = st8 % NU;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        dv[4 * u + j] = mma(sc[qa][r], o.v[0][j], dv[4 * u + j]);
                        dk[4 * u + j] = mma(dp[qa][r], o.v[1][j], dk[4 * u + j]);
                    }
                });
        }
        // End of this unit's part of key tile kt: dK/dV rows (or this unit's
        // slot, rows 64 half + 16 w + 4 g + r of the [dK | dV] slot tiles).
        if (wkey0 < S) {
            const int rows_ok = min(16, S - wkey0);
            if (tile_units(tiles, a.kv_us, kt) > 1) {
                const int64_t slot = (int64_t)(b * a.Hkv + hk) * 2 * a.kv_us.units + 2 * unit + (first ? 0 : 1);
                float* dkp = a.kv_part + (slot * 2 * BNK + 64 * half + 16 * w) * D;
                store_rows<NU>(dkp, D, dk, D, a.scale, rows_ok);
                store_rows<NU>(dkp + BNK * D, D, dv, D, 1.f, rows_ok);
            } else {
                store_rows<NU>(a.dk + a.sdk.at(b, hk) + (int64_t)wkey0 * a.sdk.s, a.sdk.s, dk, D, a.scale, rows_ok);
                store_rows<NU>(a.dv + a.sdv.at(b, hk) + (int64_t)wkey0 * a.sdv.s, a.sdv.s, dv, D, 1.f, rows_ok);
            }
        }
        if (i >= niter) {
            wait_vmcnt<0>();
            break;
        }
        ++kt;
        kstart = fast_kv_start(S, CAUSAL, W, G, kt);
        kn = fast_kv_n(S, CAUSAL, W, G, kt);
#pragma unroll
        for (int t = 0; t < 4 * NU; ++t) {
            dk[t] = zero4();
            dv[t] = zero4();
        }
        load_keys(kt);
    }
}

// ===========================================================================
// Backward, dQ role.  Workgroup = (unit, half): 4 waves x 16 query rows, the
// rows 64 half .. 64 half + 63 of every 128-row query tile of the unit; lane
// (i, g) holds Q and dO of row 16 w + i in registers.  Per 64-key tile, K and
// V in LDS (one buffer each):
//   dP^T = V dO^T, S^T = K Q^T  (A = V, K rows from LDS, B = registers);
//   P = exp2(S^T scale log2e - lse log2e), dS = P (dP - delta);
//   dQ^T += K^T dS^T  (A = K rows from LDS, B = dS as it is).
// V of tile i+1 streams in during S^T and dQ of tile i, K of tile i+1 during
// dP^T of tile i+1.
template <int DPF, bool CAUSAL, bool FAST>
__device__ __forceinline__ void dq_f32_body(const BwdArgs& a, float* smem, int unit, int half, int b, int h) {
    typedef QLds<DPF> L;
    typedef F32Dma<DPF, 64> TD;
    constexpr int BN = 64, BM = 128, NC = DPF / 16, NU = DPF / 64;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, i16 = lane & 15, g = lane >> 4;
    const int S = a.S, D = a.D, W = a.window;
    const bool vec_ok = a.vec_ok != 0;
    const KeyVis vis = bwd::key_vis(a, b, CAUSAL);
    const int hk = h / a.group;
    const float* K = (const float*)a.k + a.sk.at(b, hk);
    const float* V = (const float*)a.v + a.sv.at(b, hk);
    const float* Q = (const float*)a.q + a.sq.at(b, h);
    const float* G = (const float*)a.dO + a.sdo.at(b, h);
    const int lk = a.sk.s, lv = a.sv.s;
    float* Kt = smem;
    float* Vt = smem + L::TILE;
    TD dk_, dv_;
    dk_.init(lane, wave_id(), 2 * lk);
    dv_.init(lane, wave_id(), 2 * lv);

    const FastTiles tiles{S, CAUSAL, W, a.group, 0};
    const int64_t g0 = unit_first(tiles, a.q_us, unit);
    const int niter = (int)(unit_first(tiles, a.q_us, unit + 1) - g0);
    int qt = 0;
    while (fast_q_start(S, CAUSAL, W, qt + 1) <= g0) ++qt;
    int pf_qt = qt, pf_t = (int)(g0 - fast_q_start(S, CAUSAL, W, qt)), pf_n = fast_q_n(S, CAUSAL, W, qt);
    int pf_lo = fast_q_lo(CAUSAL, W, qt);
    auto next_key_tile = [&]() {
        const int t = pf_lo + pf_t;
        if (++pf_t == pf_n) {
            ++pf_qt;
            pf_t = 0;
            pf_n = fast_q_n(S, CAUSAL, W, pf_qt);
            pf_lo = fast_q_lo(CAUSAL, W, pf_qt);
        }
        return t;
    };
    // The V tile of the next iteration is issued before its K tile (kv_next
    // remembers the K tile's first key between the two).
    int kv_next = next_key_tile() * BN;
#pragma unroll
    for (int j = 0; j < TD::PER; ++j) issue_f32<FAST, DPF, BN>(dv_, V, kv_next, S, D, lv, Vt, j);
#pragma unroll
    for (int j = 0; j < TD::PER; ++j) issue_f32<FAST, DPF, BN>(dk_, K, kv_next, S, D, lk, Kt, j);

    f32x4 qf[NC], gf[NC];
    float lse2 = 0.f, dlt = 0.f;
    auto load_rows_of = [&](int t) {
        const int row = t * BM + 64 * half + 16 * w + i16, rowc = min(row, S - 1);
        load_row<NC>(qf, Q + (int64_t)rowc * a.sq.s, row < S, D, vec_ok);
        load_row<NC>(gf, G + (int64_t)rowc * a.sdo.s, row < S, D, vec_ok);
        const float* st = a.stats + ((int64_t)(b * a.Hq + h) * a.nqb_total + rowc / 32) * 64;
        lse2 = st[rowc % 32];
        dlt = st[32 + rowc % 32];
    };
    load_rows_of(qt);
    int64_t qstart = fast_q_start(S, CAUSAL, W, qt);
    int qn = fast_q_n(S, CAUSAL, W, qt);
    int qlo = fast_q_lo(CAUSAL, W, qt);

    f32x4 dq[4 * NU];
    for (int i = 0, first = 1;; first = 0) {
#pragma unroll
        for (int t = 0; t < 4 * NU; ++t) dq[t] = zero4();
        const int wrow0 = qt * BM + 64 * half + 16 * w, row = wrow0 + i16;
        const int vlo = vis.lo(row), vhi = vis.hi(row);
        const int seg_end = (int)min((int64_t)niter, qstart + qn - g0);
        for (; i < seg_end; ++i) {
            const int kbase = (qlo + (int)(g0 + i - qstart)) * BN;
            const bool active =
                wave_uniform(wrow0 < S && vis.any(wrow0, min(wrow0 + 15, S - 1), kbase, kbase + BN - 1));
            // V of this tile has landed everywhere (its K may still stream in)
            lds_barrier_vm<TD::PER>();
            f32x4 sacc[4], dpa[4];
            if (active) {
                const char* vt = reinterpret_cast<const char*>(Vt);
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) dpa[kb] = zero4();
                chain<NC, kPF, 4, 16, Ops<4>>(
                    [&](int c) {
                        Ops<4> o;
#pragma unroll
                        for (int kb = 0; kb < 4; ++kb) o.v[kb] = tread<DPF>(vt, 16 * kb + i16, 4 * c + g);
                        return o;
                    },
                    [&](int c, const Ops<4>& o) {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
#pragma unroll
                            for (int kb = 0; kb < 4; ++kb) dpa[kb] = mma(o.v[kb][e], gf[c][e], dpa[kb]);
                    });
            }
            // K has landed everywhere; every wave is done with V, whose next
            // tile streams in now.
            lds_barrier_vm<0>();
            if (i + 1 < niter) {
                kv_next = next_key_tile() * BN;
#pragma unroll
                for (int j = 0; j < TD::PER; ++j) issue_f32<FAST, DPF, BN>(dv_, V, kv_next, S, D, lv, Vt, j);
            }
            if (active) {
                const char* kt = reinterpret_cast<const char*>(Kt);
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) sacc[kb] = zero4();
                chain<NC, kPF, 4, 16, Ops<4>>(
                    [&](int c) {
                        Ops<4> o;
#pragma unroll
                        for (int kb = 0; kb < 4; ++kb) o.v[kb] = tread<DPF>(kt, 16 * kb + i16, 4 * c + g);
                        return o;
                    },
                    [&](int c, const Ops<4>& o) {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
#pragma unroll
                            for (int kb = 0; kb < 4; ++kb) sacc[kb] = mma(o.v[kb][e], qf[c][e], sacc[kb]);
                    });
                // register r of key block kb: key kbase + 16 kb + 4 g + r, row `row`
                const bool need_mask = wave_uniform(!vis.all(wrow0, wrow0 + 15, kbase, kbase + BN - 1));
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float p = fast_exp2(sacc[kb][r] * a.scale_log2 - lse2);
                        if (need_mask) {
                            const int key = kbase + 16 * kb + 4 * g + r;
                            if (key < vlo || key > vhi) p = 0.f;
                        }
                        sacc[kb][r] = p * (dpa[kb][r] - dlt);
                    }
                // dQ^T(u, j) += K^T dS^T: step (kb, r) takes key 16 kb + 4 g + r
                chain<16, kPF, NU, 4 * NU, Ops<NU>>(
                    [&](int s) {
                        Ops<NU> o;
#pragma unroll
                        for (int u = 0; u < NU; ++u) o.v[u] = tread<DPF>(kt, 16 * (s >> 2) + 4 * g + (s & 3), 16 * u + i16);
                        return o;
                    },
                    [&](int s, const Ops<NU>& o) {
#pragma unroll
                        for (int u = 0; u < NU; ++u)
#pragma unroll
                            for (int j = 0; j < 4; ++j) dq[4 * u + j] = mma(o.v[u][j], sacc[s >> 2][s & 3], dq[4 * u + j]);
                    });
            }
            // every wave is done with K, whose next tile streams in now
            lds_barrier();
            if (i + 1 < niter) {
#pragma unroll
                for (int j = 0; j < TD::PER; ++j) issue_f32<FAST, DPF, BN>(dk_, K, kv_next, S, D, lk, Kt, j);
            }
        }
        const bool more = i < niter;
        if (row < S) {
            if (tile_units(tiles, a.q_us, qt) > 1) {
                const int64_t slot = (int64_t)(b * a.Hq + h) * 2 * a.q_us.units + 2 * unit + (first ? 0 : 1);
                store_rowT<NU>(a.q_part + (slot * BM + 64 * half + 16 * w + i16) * D, dq, D, a.scale);
            } else {
                store_rowT<NU>(a.dq + a.sdq.at(b, h) + (int64_t)row * a.sdq.s, dq, D, a.scale);
            }
        }
        if (!more) {
            wait_vmcnt<0>();
            break;
        }
        ++qt;
        qstart = fast_q_start(S, CAUSAL, W, qt);
        qn = fast_q_n(S, CAUSAL, W, qt);
        qlo = fast_q_lo(CAUSAL, W, qt);
        load_rows_of(qt);
    }
}

// Workgroups: (unit, half, batch, head), dK/dV units first (both roles' units
// are sized to take about equally long, plan_bwd_fast).
template <int DPF, bool CAUSAL, bool FAST>
__global__ __launch_bounds__(256) void attn_bwd_main_f32(BwdArgs a) {
    __shared__ __attribute__((aligned(1024))) float smem[main_lds_floats<DPF>()];
    const int nkv = 2 * a.kv_us.units * a.B * a.Hkv, i = xcd_block((int)blockIdx.x, (int)gridDim.x);
    if (i < nkv) {
        const int bh = a.B * a.Hkv;
        dkdv_f32_body<DPF, CAUSAL, FAST>(a, smem, i / (2 * bh), (i / bh) & 1, (i % bh) / a.Hkv, (i % bh) % a.Hkv);
    } else {
        const int j = i - nkv, bh = a.B * a.Hq;
        dq_f32_body<DPF, CAUSAL, FAST>(a, smem, j / (2 * bh), (j / bh) & 1, (j % bh) / a.Hq, (j % bh) % a.Hq);
    }
}
template <int DPF, bool CAUSAL, bool FAST>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_f32_fast(BwdArgs a) {
    __shared__ __attribute__((aligned(1024))) float smem[KvLds<DPF>::FLOATS];
    const int bh = a.B * a.Hkv, i = (int)blockIdx.x;
    dkdv_f32_body<DPF, CAUSAL, FAST>(a, smem, i / (2 * bh), (i / bh) & 1, (i % bh) / a.Hkv, (i % bh) % a.Hkv);
}
template <int DPF, bool CAUSAL, bool FAST>
__global__ __launch_bounds__(256) void attn_bwd_dq_f32_fast(BwdArgs a) {
    __shared__ __attribute__((aligned(1024))) float smem[QLds<DPF>::FLOATS];
    const int bh = a.B * a.Hq, j = (int)blockIdx.x;
    dq_f32_body<DPF, CAUSAL, FAST>(a, smem, j / (2 * bh), (j / bh) & 1, (j % bh) / a.Hq, (j % bh) % a.Hq);
}

// FAST (TileDma offsets): every tile whole, D == DPF and S a multiple of 64.
template <int DPF> bool whole_tiles(const AttnShape& s) { return s.D == DPF && s.S % 64 == 0; }

template <int DPF>
hipError_t launch_fwd(const AttnShape& s, FwdArgs a, hipStream_t st) {
    a.n_qtiles = (int)((s.S + kFwdBM - 1) / kFwdBM);
    const dim3 grid((unsigned)(2 * a.us.units * s.B * s.Hq));
    const bool fast = whole_tiles<DPF>(s);
    if (s.causal) {
        if (fast) hipLaunchKernelGGL((attn_fwd_f32_split<DPF, true, true>), grid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((attn_fwd_f32_split<DPF, true, false>), grid, dim3(256), 0, st, a);
    } else {
        if (fast) hipLaunchKernelGGL((attn_fwd_f32_split<DPF, false, true>), grid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((attn_fwd_f32_split<DPF, false, false>), grid, dim3(256), 0, st, a);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || !a.any_split) return e;
    return fwd::launch_fwd_combine(s, a, st);
}

// The work-unit kernels of one causal mode: MAIN = the combined launch of
// both roles, otherwise the DKDV or DQ stage alone (stages).  Instantiated
// per (DPF, CAUSAL, MAIN) in the attn_f32_fast*.hip translation units, so
// that the D = 256 kernels compile in parallel.
template <int DPF, bool CAUSAL, bool MAIN>
hipError_t launch_bwd_units(const AttnShape& s, const BwdArgs& a, int stages, hipStream_t st) {
    const bool fast = whole_tiles<DPF>(s);
    const unsigned nkv = (unsigned)(2 * a.kv_us.units * s.B * s.Hkv), nq = (unsigned)(2 * a.q_us.units * s.B * s.Hq);
#define MFT_F32_LAUNCH(KERNEL, GRID)                                                       \
    do {                                                                                   \
        if (fast) hipLaunchKernelGGL((KERNEL<DPF, CAUSAL, true>), GRID, dim3(256), 0, st, a); \
        else hipLaunchKernelGGL((KERNEL<DPF, CAUSAL, false>), GRID, dim3(256), 0, st, a);     \
    } while (0)
    if constexpr (MAIN)
        MFT_F32_LAUNCH(attn_bwd_main_f32, dim3(nkv + nq));
    else if (stages & BWD_STAGE_DKDV)
        MFT_F32_LAUNCH(attn_bwd_dkdv_f32_fast, dim3(nkv));
    else if (stages & BWD_STAGE_DQ)
        MFT_F32_LAUNCH(attn_bwd_dq_f32_fast, dim3(nq));
#undef MFT_F32_LAUNCH
    return hipGetLastError();
}

// Launchers for one padded head dim (DPF = 64, 128, 256), instantiated in the
// attn_f32_fast*.hip translation units.
template <int DPF> hipError_t launch_fwd_dpf(const AttnShape& s, const FwdArgs& a, hipStream_t st) {
    return launch_fwd<DPF>(s, a, st);
}
#define MFT_F32_EXTERN(DPF)                                                                                  \
    extern template hipError_t launch_fwd_dpf<DPF>(const AttnShape&, const FwdArgs&, hipStream_t);          \
    extern template hipError_t launch_bwd_units<DPF, true, true>(const AttnShape&, const BwdArgs&, int,     \
                                                                 hipStream_t);                               \
    extern template hipError_t launch_bwd_units<DPF, false, true>(const AttnShape&, const BwdArgs&, int,    \
                                                                  hipStream_t);                              \
    extern template hipError_t launch_bwd_units<DPF, true, false>(const AttnShape&, const BwdArgs&, int,    \
                                                                  hipStream_t);                              \
    extern template hipError_t launch_bwd_units<DPF, false, false>(const AttnShape&, const BwdArgs&, int,   \
                                                                   hipStream_t);
MFT_F32_EXTERN(64)
MFT_F32_EXTERN(128)
MFT_F32_EXTERN(256)
#undef MFT_F32_EXTERN

// DELTA, the work-unit launch of the stages asked for, then REDUCE.
template <int DPF>
hipError_t launch_bwd_dpf(const AttnShape& s, const BwdArgs& a, int stages, hipStream_t st) {
    if (stages & BWD_STAGE_DELTA) {
        constexpr int RPB = 256 / (DPF / 4);
        const int64_t rows = s.B * s.Hq * (int64_t)a.nqb_total * 32;
        hipLaunchKernelGGL((bwd::attn_bwd_stats_kernel<float, DPF>), dim3((unsigned)((rows + RPB - 1) / RPB)),
                           dim3(256), 0, st, a);
    }
    hipError_t e = hipSuccess;
    const bool main = (stages & BWD_STAGE_MAIN) == BWD_STAGE_MAIN;
    if (main)
        e = s.causal ? launch_bwd_units<DPF, true, true>(s, a, stages, st)
                     : launch_bwd_units<DPF, false, true>(s, a, stages, st);
    else if (stages & BWD_STAGE_MAIN)
        e = s.causal ? launch_bwd_units<DPF, true, false>(s, a, stages, st)
                     : launch_bwd_units<DPF, false, false>(s, a, stages, st);
    if (e != hipSuccess) return e;
    if ((stages & BWD_STAGE_REDUCE) && (a.kv_parts_max > 1 || a.q_parts_max > 1)) {
        const int64_t nt = (s.S + 127) / 128;
        const int64_t blocks = (s.B * s.Hkv + s.B * s.Hq) * nt * (128 / merge_rows(s.D));
        if (s.causal)
            hipLaunchKernelGGL(bwd::attn_bwd_fast_reduce<true>, dim3((unsigned)blocks), dim3(256), 0, st, a);
        else
            hipLaunchKernelGGL(bwd::attn_bwd_fast_reduce<false>, dim3((unsigned)blocks), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

}  // namespace f32
}  // namespace mft
