// Balanced bf16 forward at D = 256 with two waves per SIMD.
//
// The 32-row waves of attn_fwd_fast.h hold O (128 registers), Q (64) and the
// score tile: more than the 256 registers that leave room for a second wave
// on the SIMD, so each SIMD runs one wave and idles its MFMA unit through
// every softmax, address and wait instruction of that wave.  Here a wave
// owns 16 query rows and uses v_mfma_f32_16x16x32_bf16 (the same MAC rate as
// 32x32x16): O^T is 16 tiles of 16 x 16 (64 registers), Q 32 registers, and
// the workgroup is 8 waves (two per SIMD) over the same 128-row query tile,
// 64-key K/V tiles, split plan and partial-slot layout as the 32-row kernel
// (attn_fwd_combine merges the partials unchanged).
//
// 16x16x32 operand layout (lane l, g = l / 16, n = l % 16): A is row n, k
// 8g..8g+7; B is column n, k 8g..8g+7; C holds rows 4g..4g+3 of column n.
//   S^T = K Q^T per 16-key block kb: A = K row 16kb + n (ds_read_b128 of a
//        SWZ_ROW tile), B = Q^T (this lane's query row, from registers); the
//        result holds keys 16kb + 4g + i of query n.
//   O^T += V^T P^T per 32-key step s2: B = P^T with the k-slots the lane
//        already holds, keys {32s2 + 4g + t} (t < 4) and {32s2 + 16 + 4g + t-4}
//        (t >= 4); A = V^T in the same key order, two ds_read_b64_tr_b16 (four
//        consecutive keys each) of a SWZ_TR16 tile.
// A query's row statistics are spread over its four lane groups; the tile
// maximum is reduced across them (xor 16, 32) and the sum only at the end.
#pragma once

#include "attn_fwd_fast.h"

namespace mft {
namespace fwd {

constexpr int kW16Threads = 512;  // 8 waves x 16 rows = the 128-row query tile

namespace {

// Per-lane, loop-invariant LDS read offsets (bytes, relative to the tile).
//  kr[jj]: K row read of block kb, k-step j: row 16kb + n, chunk (4j + g) ^ n:
//          n*ROWB + 64*((j & 3) ^ (n >> 2)) + 16*(g ^ (n & 3)) + 256*(j >> 2)
//          + kb*16*ROWB, i.e. kr[j & 3] + 256 (j >> 2) + kb*16*ROWB.
//  vr[dd]: transposed V read of column tile dt, key step s2, half h: reading
//          lane n reads row 32s2 + 16h + 4g + n/4, columns 16dt + 4(n%4) ..:
//          (4g + n/4)*ROWB + 32*((dt & 7) ^ z) + 16*((n & 3) >> 1) + 8*(n & 1)
//          + 256*(dt >> 3) + (32s2 + 16h)*ROWB with z = 4(g & 1) + n/4 (the
//          row's swz_tr16 bits), i.e. vr[dt & 7] + 256 (dt >> 3) + ....
template <int DP> struct W16Lane {
    static constexpr int CPR = DP / 8, ROWB = DP * 2;
    static_assert(DP == 256, "the 16-row forward is laid out for D = 256");
    uint32_t kr[4];
    uint32_t vr[8];
    TileDma<DP, kFwdBN, kW16Threads, SWZ_ROW> dk;
    TileDma<DP, kFwdBN, kW16Threads, SWZ_TR16> dv;

    __host__ __device__ void init(int lane, int w, int lk, int lv) {
        const int n = lane & 15, g = lane >> 4;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
            kr[jj] = (uint32_t)n * ROWB + 64u * (uint32_t)(jj ^ (n >> 2)) + 16u * (uint32_t)(g ^ (n & 3));
        const int z = 4 * (g & 1) + (n >> 2);
#pragma unroll
        for (int dd = 0; dd < 8; ++dd)
            vr[dd] = (uint32_t)(4 * g + (n >> 2)) * ROWB + 32u * (uint32_t)(dd ^ z) + 16u * (uint32_t)((n & 3) >> 1) +
                     8u * (uint32_t)(n & 1);
        dk.init(lane, w, lk);
        dv.init(lane, w, lv);
    }
    __host__ __device__ uint32_t k_off(int kb, int j) const { return kr[j & 3] + 256 * (j >> 2) + kb * 16 * ROWB; }
    __host__ __device__ uint32_t v_off(int dt, int s2, int h) const {
        return vr[dt & 7] + 256 * (dt >> 3) + (32 * s2 + 16 * h) * ROWB;
    }
};

template <int N> __device__ __forceinline__ void pin_vgpr4(f32x4 (&acc)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("" : "+v"(acc[i]));
}

// The next tile's direct loads (K, then V) into the buffer of parity npar.
template <int DP>
struct W16Issue {
    const W16Lane<DP>& ln;
    const bf16* K;
    const bf16* V;
    uint32_t smem_addr;
    int lk, lv, nrow, npar;
    static constexpr int PER = kFwdBN * (DP / 8) / kW16Threads, NPARTS = 2 * PER;
    __device__ __forceinline__ void operator()(int j) const {
        constexpr int TILE = kFwdBN * DP;
        if (j < PER)
            issue_tile_j<true, DP, kFwdBN, kW16Threads, SWZ_ROW>(ln.dk, K, nrow, 0, DP, lk, nullptr,
                                                                smem_addr + 2u * npar * TILE, j);
        else
            issue_tile_j<true, DP, kFwdBN, kW16Threads, SWZ_TR16>(ln.dv, V, nrow, 0, DP, lv, nullptr,
                                                                 smem_addr + 2u * (2 + npar) * TILE, j - PER);
    }
};

// S^T = K Q^T of one 64-key tile for this wave's 16 rows: the four 16-key
// blocks' chains interleaved, K through a ring; issue(j) for the next tile's
// loads j < Issue::NPARTS go between the steps.
template <int DP, class Issue>
__device__ __forceinline__ void fwd16_s(const char* kb_, const W16Lane<DP>& ln, const bf16x8 (&qf)[DP / 32],
                                        f32x4 (&s)[kFwdBN / 16], const Issue& issue) {
    constexpr int NJ = DP / 32, NKB = kFwdBN / 16, PF = 4;
    constexpr int NPARTS = Issue::NPARTS;
    constexpr int NI = NKB * NJ;
    auto kread = [&](int it) { return *reinterpret_cast<const bf16x8*>(kb_ + ln.k_off(it % NKB, it / NKB)); };
    bf16x8 ring[PF];
#pragma unroll
    for (int it = 0; it < PF; ++it) ring[it] = kread(it);
#pragma unroll
    for (int it = 0; it < NI; ++it) {
        const bf16x8 ka = ring[it % PF];
        if (it + PF < NI) ring[it % PF] = kread(it + PF);
        if (it < NKB)
            mfma16_first(s[it], ka, qf[0]);
        else
            s[it % NKB] = mfma16(ka, qf[it / NKB], s[it % NKB]);
        if ((it & 3) == 3 && (it >> 2) < NPARTS) issue(it >> 2);
    }
#pragma unroll
    for (int j = NI / 4; j < NPARTS; ++j) issue(j);
}

// Mask, online softmax and O^T += V^T P^T of one tile whose S^T is in s.
template <int DP>
__device__ __forceinline__ void fwd16_pv(const FwdArgs& a, const char* vb_, const W16Lane<DP>& ln, bool need_mask,
                                         int kbase, int vlo, int vhi, f32x4 (&s)[kFwdBN / 16], f32x4 (&oacc)[DP / 16],
                                         float& m_run, float& l_run) {
    constexpr int NDT = DP / 16, NKB = kFwdBN / 16, PF = 4;
    const int g = (threadIdx.x & 63) >> 4;
    if (need_mask) {  // keys outside [vlo, vhi]
        int hi = vhi - kbase, lo = vlo - kbase;
        asm volatile("" : "+v"(hi), "+v"(lo));
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int kl = 16 * kb + 4 * g + i;
                s[kb][i] = (kl > hi || kl < lo) ? -INFINITY : s[kb][i];
            }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[kb][i]);
    mx = half_max(row16_max(mx)) * a.scale_log2;
    // Lazy rescaling as in fwd_tile: the reference point moves (and O, l
    // are rescaled) only when some row's tile max exceeds it by 8.
    if (__any(mx > m_run + kLazyRescale)) {
        const float m_new = fmaxf(m_run, mx);
        const float alpha = fast_exp2(m_run - (m_new == -INFINITY ? 0.f : m_new));
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) oacc[dt][i] *= alpha;
        pin_vgpr4(oacc);
        m_run = m_new;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    float psum = 0.f;
    bf16x8 pb[NKB / 2];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float p = fast_exp2(s[kb][i] * a.scale_log2 - m_use);
            psum += p;
            pb[kb / 2][4 * (kb & 1) + i] = (bf16)p;
        }
    l_run += psum;

    // O^T += V^T P^T; the two 8-byte halves of each V^T operand through
    // rings of their own, joined at the MFMA.
    {
        constexpr int NI = 2 * NDT;  // (s2, dt)
        auto vread = [&](int it, int h) {
            return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(vb_ + ln.v_off(it % NDT, it / NDT, h)));
        };
        v4i16 rl[PF], rh[PF];
#pragma unroll
        for (int it = 0; it < PF; ++it) {
            rl[it] = vread(it, 0);
            rh[it] = vread(it, 1);
        }
#pragma unroll
        for (int it = 0; it < NI; ++it) {
            const bf16x8 va =
                __builtin_bit_cast(bf16x8, __builtin_shufflevector(rl[it % PF], rh[it % PF], 0, 1, 2, 3, 4, 5, 6, 7));
            if (it + PF < NI) {
                rl[it % PF] = vread(it + PF, 0);
                rh[it % PF] = vread(it + PF, 1);
            }
            oacc[it % NDT] = mfma16(va, pb[it / NDT], oacc[it % NDT]);
        }
        pin_read_ahead<NI, PF, 2>();
    }
}

// One 64-key tile for this wave's 16 rows (see the header comment).
template <int DP, class Issue>
__device__ __forceinline__ void fwd16_tile(const FwdArgs& a, const char* smem, const W16Lane<DP>& ln, int par,
                                           bool need_mask, int kbase, int vlo, int vhi, const bf16x8 (&qf)[DP / 32],
                                           f32x4 (&oacc)[DP / 16], float& m_run, float& l_run, const Issue& issue) {
    constexpr int TILEB = kFwdBN * DP * 2;
    f32x4 s[kFwdBN / 16];
    fwd16_s<DP>(smem + par * TILEB, ln, qf, s, issue);
    fwd16_pv<DP>(a, smem + (2 + par) * TILEB, ln, need_mask, kbase, vlo, vhi, s, oacc, m_run, l_run);
}

// Normalised O row and LSE of this lane's query (row < S): lane group g
// holds columns 16dt + 4g .. +3 of every column tile dt.
template <int DP>
__device__ __forceinline__ void fwd16_store_row(const FwdArgs& a, int b, int h, int row, const f32x4 (&oacc)[DP / 16],
                                                float m_run, float l_tot) {
    const int g = (threadIdx.x & 63) >> 4;
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    bf16* O = (bf16*)a.o + a.so.at(b, h) + (int64_t)row * a.so.s;
#pragma unroll
    for (int dt = 0; dt < DP / 16; ++dt)
        store4<bf16>(O, 16 * dt + 4 * g, a.D, oacc[dt][0] * inv, oacc[dt][1] * inv, oacc[dt][2] * inv,
                     oacc[dt][3] * inv, true);
    if (a.lse && g == 0)
        a.lse[(int64_t)(b * a.Hq + h) * a.S + row] = l_tot > 0.f ? (m_run + log2f(l_tot)) * kLn2 : INFINITY;
}

// The balanced launch (see attn_fwd_bf16_split) with 16-row waves; every
// tile whole (D == DP, S a multiple of 64).
template <int DP, bool CAUSAL>
__global__ __launch_bounds__(kW16Threads) void attn_fwd_bf16_split16(FwdArgs a) {
    constexpr int BN = kFwdBN, BM = kFwdBM;
    constexpr int NJ = DP / 32, NDT = DP / 16, TILE = BN * DP;
    __shared__ __attribute__((aligned(1024))) bf16 smem[4 * TILE];

    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6, n = lane & 15, g = lane >> 4;
    const int S = a.S, D = a.D;
    // XCD-major block order (xcd_block): the query heads of one unit index,
    // which read the same K/V tiles, and neighbouring units share one L2.
    const int bh = a.B * a.Hq, blk = xcd_block((int)blockIdx.x, (int)gridDim.x);
    const int unit = blk / bh, b = (blk % bh) / a.Hq, h = (blk % bh) % a.Hq, hk = h / a.group;

    const bf16* __restrict__ Q = (const bf16*)a.q + a.sq.at(b, h);
    const bf16* __restrict__ K = (const bf16*)a.k + a.sk.at(b, hk);
    const bf16* __restrict__ Vg = (const bf16*)a.v + a.sv.at(b, hk);
    const int lq = a.sq.s, lk = a.sk.s, lv = a.sv.s;
    W16Lane<DP> ln;
    ln.init(lane, wave_id(), lk, lv);
    const uint32_t smem_addr = lds_addr(smem);

    const int W = a.window;
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
        const W16Issue<DP> first{ln, K, Vg, smem_addr, lk, lv, next_key_tile() * BN, 0};
#pragma unroll
        for (int j = 0; j < W16Issue<DP>::NPARTS; ++j) first(j);
    }

    // This lane's query row: Q fragments of k-steps j (B operand of S^T).
    bf16x8 qf[NJ];
    auto load_q = [&](int qtile) {
        const int row = qtile * BM + 16 * w + n, rowc = row < S ? row : S - 1;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
            qf[j] = *reinterpret_cast<const bf16x8*>(Q + (int64_t)rowc * lq + 32 * j + 8 * g);
    };
    f32x4 oacc[NDT];
    float m_run, l_run;
    int64_t qstart = fast_q_start(S, CAUSAL, W, qt);
    int qn = fast_q_n(S, CAUSAL, W, qt);
    int qlo = fast_q_lo(CAUSAL, W, qt);
    load_q(qt);
    wait_vmcnt<0>();

    for (int i = 0, first = 1;; first = 0) {
#pragma unroll
        for (int d = 0; d < NDT; ++d) oacc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
        pin_vgpr4(oacc);
        m_run = -INFINITY;
        l_run = 0.f;
        const int wrow0 = qt * BM + 16 * w, row = wrow0 + n;
        const int vlo = vis.lo(row), vhi = vis.hi(row);
        const int seg_end = (int)min((int64_t)niter, qstart + qn - g0);
        for (; i < seg_end; ++i) {
            const int par = i & 1;
            // This tile's direct loads (and, at a segment's first tile, its Q
            // and the last segment's stores) have landed.  The wait is
            // unconditional so that the compiler sees Q complete here: the
            // direct loads are inline asm it does not count, so any wait it
            // placed for Q inside the S^T loop would also wait for the direct
            // loads issued there for the next tile.
            wait_vmcnt<0>();
            lds_barrier();
            const W16Issue<DP> issue{ln, K, Vg, smem_addr, lk, lv, i + 1 < niter ? next_key_tile() * BN : 0, par ^ 1};
            const int kbase = (qlo + (int)(g0 + i - qstart)) * BN;
            if (wave_uniform(wrow0 < S && vis.any(wrow0, min(wrow0 + 15, S - 1), kbase, kbase + BN - 1))) {
                const bool need_mask = wave_uniform(!vis.all(wrow0, wrow0 + 15, kbase, kbase + BN - 1));
                fwd16_tile<DP>(a, (const char*)smem, ln, par, need_mask, kbase, vlo, vhi, qf, oacc, m_run, l_run,
                               issue);
            } else {
#pragma unroll
                for (int j = 0; j < W16Issue<DP>::NPARTS; ++j) issue(j);
            }
        }
        const bool more = i < niter;
        const int nsl = tile_units(tiles, a.us, qt);
        if (more) {
            ++qt;
            qstart = fast_q_start(S, CAUSAL, W, qt);
            qn = fast_q_n(S, CAUSAL, W, qt);
            qlo = fast_q_lo(CAUSAL, W, qt);
            load_q(qt);
        }
        if (wave_uniform(wrow0 < S)) {
            const float l_tot = half_sum(row16_sum(l_run));
            if (nsl <= 1) {
                fwd16_store_row<DP>(a, b, h, row, oacc, m_run, l_tot);
            } else {
                const int64_t slot = (int64_t)(b * a.Hq + h) * 2 * a.us.units + 2 * unit + (first ? 0 : 1);
                float* po = a.part_o + (slot * BM + 16 * w + n) * D;
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt)
                    store4<float>(po, 16 * dt + 4 * g, D, oacc[dt][0], oacc[dt][1], oacc[dt][2], oacc[dt][3], true);
                if (g == 0) {
                    float* pml = a.part_ml + (slot * BM + 16 * w + n) * 2;
                    pml[0] = m_run;
                    pml[1] = l_tot;
                }
            }
        }
        if (!more) {
            wait_vmcnt<0>();
            break;
        }
    }
}

}  // namespace
}  // namespace fwd
}  // namespace mft
