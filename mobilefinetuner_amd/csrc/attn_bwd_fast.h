// bf16 fast path of the attention backward (D % 8 == 0, 32 < D <= 256).
// Included by attn_bwd_fast64.hip (D <= 128 instantiations) and
// attn_bwd_fast256.hip, which are compiled with different MFMA register
// forms (see mobilefinetuner_amd/build.py).
#pragma once

#include "attn_bwd_common.h"

namespace mft {
namespace bwd {
namespace {

// ===========================================================================
// bf16 fast path (D % 8 == 0, 32 < D <= 256)
//
// The same two roles, with all tile traffic moved HBM -> LDS by
// global_load_lds_dwordx4 into double buffers (the next block streams in
// while the current one is multiplied), unpadded XOR-swizzled LDS tiles, and
// every transposed operand (dO^T, Q^T for dV/dK, K^T for dQ) read with
// ds_read_b64_tr_b16 from the row-major tile instead of being stored twice.
//
// STATS stage: stats[(b*Hq + h) * nqb + blk][0..31] = lse * log2(e) of rows
// 32*blk + 0..31 (+inf past S), [32..63] = delta (0 past S).  256-byte blocks
// let the dK/dV role fetch a query block's row terms with one direct load.
template <typename T, int DP>
__global__ __launch_bounds__(256) void attn_bwd_stats_kernel(BwdArgs a) {
    typedef typename Elt<T>::vec V;
    constexpr int VEC = Elt<T>::VEC;
    constexpr int TPR = DP / VEC;
    constexpr int RPB = 256 / TPR;
    const int64_t spad = (int64_t)a.nqb_total * 32;
    const int64_t total = (int64_t)a.B * a.Hq * spad;
    const int64_t prow = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;  // padded row index
    const int c = threadIdx.x % TPR;
    const int64_t bh = prow / spad;
    const int i = (int)(prow - bh * spad);
    const bool valid = prow < total && i < a.S;
    float acc = 0.f;
    if (valid) {
        const int bb = (int)(bh / a.Hq), hq = (int)(bh % a.Hq);
        const V x = load_chunk<T>((const T*)a.o + a.so.at(bb, hq) + i * a.so.s, c * VEC, a.D, true, a.vec_ok != 0);
        const V y = load_chunk<T>((const T*)a.dO + a.sdo.at(bb, hq) + i * a.sdo.s, c * VEC, a.D, true,
                                  a.vec_ok != 0);
#pragma unroll
        for (int k = 0; k < VEC; ++k) acc += (float)x[k] * (float)y[k];
    }
#pragma unroll
    for (int off = TPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (prow < total && c == 0) {
        float* blk = a.stats + (bh * a.nqb_total + i / 32) * 64;
        blk[i % 32] = valid ? a.lse[bh * a.S + i] * kLog2e : INFINITY;
        blk[32 + i % 32] = valid ? acc : 0.f;
    }
}

template <int DP> struct BwdFastLds {
    // V_LDS: at D = 256 the dK/dV role reads V of its 128 keys from LDS (B
    // operand of dP) instead of registers: K, dK and dV already take 320 of
    // a wave's 512 registers and the LDS operand pipeline needs the rest.
    static constexpr bool V_LDS = DP >= 256;
    static constexpr int KV_BUF = 2 * 32 * DP + 4 * 512;  // Q, dO tiles + 4 waves x 1 KiB stats (elements)
    static constexpr int KV_ELEMS = 2 * KV_BUF + (V_LDS ? 128 * DP : 0);
    static constexpr int Q_BUF = 2 * 64 * DP;             // K, V tiles
    static constexpr int Q_ELEMS = 2 * Q_BUF;
    static constexpr int ELEMS = KV_ELEMS > Q_ELEMS ? KV_ELEMS : Q_ELEMS;
};

template <int DP, bool CAUSAL, bool STRIDED>
__device__ __forceinline__ void dkdv_fast_body(const BwdArgs& a, bf16* smem, int unit, int b, int hk) {
    constexpr int NT = 256, BNK = 128, CPR = DP / 8, NC = DP / 16, NDT = DP / 32;
    constexpr int QT = 32 * DP;
    constexpr int BUF = BwdFastLds<DP>::KV_BUF;
    constexpr bool V_LDS = BwdFastLds<DP>::V_LDS;
    constexpr int PF = 4;  // LDS operand prefetch depth

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 31, hh = lane >> 5;
    const int i16 = lane & 15, nh = (lane >> 4) & 1;
    const int S = a.S, D = a.D, G = a.group, W = a.window;
    const KeyVis vis = key_vis(a, b, CAUSAL);
    const bf16* K = (const bf16*)a.k + op_base<STRIDED>(a.sk, b, hk, a.Hkv, S, D);
    const bf16* Vg = (const bf16*)a.v + op_base<STRIDED>(a.sv, b, hk, a.Hkv, S, D);
    // K and V share one sequence stride on this path (bwd_fast_path): a
    // second stride live across the loop costs the dK/dV accumulators their
    // registers (the compiler then shuffles them every block).
    const int lk = op_ld<STRIDED>(a.sk, D), lv = lk;
    const int lq = op_ld<STRIDED>(a.sq, D), lg = op_ld<STRIDED>(a.sdo, D);

    // This unit's chunk of the flattened (key tile, query head, query block)
    // iterations; it may start inside one key tile and end inside a later one.
    const int nkt = (S + BNK - 1) / BNK;
    const int64_t g0 = (int64_t)unit * a.kv_chunk;
    const int niter = (int)min((int64_t)a.kv_chunk, fast_kv_start(S, CAUSAL, W, G, nkt) - g0);
    int kt = 0;
    while (fast_kv_start(S, CAUSAL, W, G, kt + 1) <= g0) ++kt;

    // Prefetch cursor of the next iteration to load: key tile, query head of
    // the group, query block (iterations of a key tile run head-major over
    // its nqb = fast_kv_n / G query blocks); advanced without divisions.
    int pf_kt = kt, pf_nqb = fast_kv_nqb(S, CAUSAL, W, kt);
    int pf_h, pf_qi;
    {
        const int it0 = (int)(g0 - fast_kv_start(S, CAUSAL, W, G, kt));
        pf_h = it0 / pf_nqb;
        pf_qi = it0 - pf_h * pf_nqb;
    }
    // The next block's loads: issue_begin resolves its sources (and advances
    // the cursor), issue_part(j) issues load j of NPARTS, so that the loads
    // can be spread between the MFMAs of the current block.
    constexpr int PER = 32 * CPR / NT, NPARTS = 2 * PER + 1;
    struct Pending {
        const bf16* q;
        const bf16* g;
        const float* st;
        bf16* buf;
        int qb;
    };
    auto issue_begin = [&](bf16* buf) {
        const int h = hk * G + pf_h, qb = (CAUSAL ? pf_kt * BNK : 0) + pf_qi * 32;
        if (++pf_qi == pf_nqb) {
            pf_qi = 0;
            if (++pf_h == G) {
                pf_h = 0;
                ++pf_kt;
                pf_nqb = fast_kv_nqb(S, CAUSAL, W, pf_kt);
            }
        }
        return Pending{(const bf16*)a.q + op_base<STRIDED>(a.sq, b, h, a.Hq, S, D),
                       (const bf16*)a.dO + op_base<STRIDED>(a.sdo, b, h, a.Hq, S, D),
                       a.stats + ((int64_t)(b * a.Hq + h) * a.nqb_total + qb / 32) * 64, buf, qb};
    };
    auto issue_part = [&](const Pending& p, int j) {
        if (j < PER)
            issue_tile_part<DP, 32, NT, SWZ_DUAL>(p.q, p.qb, S, D, lq, p.buf, j);
        else if (j < 2 * PER)
            issue_tile_part<DP, 32, NT, SWZ_DUAL>(p.g, p.qb, S, D, lg, p.buf + QT, j - PER);
        else
            load_lds_16(p.st + 4 * i16, p.buf + 2 * QT + w * 512);
    };
    auto issue = [&](bf16* buf) {
        const Pending p = issue_begin(buf);
#pragma unroll
        for (int j = 0; j < NPARTS; ++j) issue_part(p, j);
        return p.qb;
    };

    bf16* Vl = smem + 2 * BUF;  // V rows of the current key tile (V_LDS only)
    bf16x8 kf[NC], vf[V_LDS ? 1 : NC];
    // Per key tile: this lane's K (and V) fragments, and with V_LDS the V tile.
    auto load_keys = [&](int t) {
        const int key = t * BNK + 32 * w + n, keyc = key < S ? key : S - 1;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            kf[c] = load_chunk<bf16>(K + (int64_t)keyc * lk, 16 * c + 8 * hh, D, key < S, true);
            if constexpr (!V_LDS) vf[c] = load_chunk<bf16>(Vg + (int64_t)keyc * lv, 16 * c + 8 * hh, D, key < S, true);
        }
        if constexpr (V_LDS) {
            issue_tile<DP, BNK, NT, SWZ_ROW>(Vg, t * BNK, S, D, lv, Vl);
            if (D < DP) {
                // Staged columns >= D hold copies of column chunk 0, and so do
                // those of the dO tiles: zero them so that dP = dO V^T sums
                // only the D real columns.
                lds_barrier_vm<0>();
                const bf16x8 z = zero_vec<bf16x8>();
                for (int idx = tid; idx < BNK * CPR; idx += NT) {
                    const int r = idx / CPR, c = idx % CPR;
                    if (8 * c >= D) *reinterpret_cast<bf16x8*>(Vl + r * DP + ((c ^ swz_row<CPR>(r)) << 3)) = z;
                }
            }
        }
    };
    load_keys(kt);
    int cur_qb = issue(smem);  // query block of the block in the current buffer
    // The key fragments are complete before the loop (the compiler then sees
    // nothing pending inside it; the direct loads are untracked, see load_lds_16).
    wait_vmcnt<0>();

    f32x16 dk[NDT], dv[NDT];
#pragma unroll
    for (int i = 0; i < NDT; ++i) {
        dk[i] = zero16();
        dv[i] = zero16();
    }
    int64_t kstart = fast_kv_start(S, CAUSAL, W, G, kt);
    int kn = fast_kv_n(S, CAUSAL, W, G, kt);

    for (int i = 0, first = 1;; first = 0) {
      // Iterations of key tile kt inside this unit, then its dK/dV store.
      const int seg_end = (int)min((int64_t)niter, kstart + kn - g0);
      for (; i < seg_end; ++i) {
        const bf16* Qb = smem + (i & 1) * BUF;
        const bf16* Gb = Qb + QT;
        const float* stt = reinterpret_cast<const float*>(Qb + 2 * QT + w * 512);
        // This wave's loads of buffer i&1 (issued one iteration ago) have
        // landed; after the barrier every wave's have, and every wave is done
        // with buffer (i+1)&1, which the next block then streams into.
        wait_vmcnt<0>();
        lds_barrier();
        // The last block prefetches a harmless copy of itself into the idle
        // buffer, so that the load schedule below needs no branch (the unit
        // waits for it before it ends).
        const Pending pend = i + 1 < niter ? issue_begin(smem + ((i + 1) & 1) * BUF)
                                           : Pending{(const bf16*)a.q, (const bf16*)a.dO, a.stats,
                                                     smem + ((i + 1) & 1) * BUF, 0};
        const int qb = cur_qb;
        cur_qb = pend.qb;
        const int wkey0 = kt * BNK + 32 * w;
        const int key = wkey0 + n;
        // Waves whose keys are past S, or none of which a row of this query
        // block sees, skip it.
        if (wave_uniform(wkey0 < S && vis.any(qb, min(qb + 31, S - 1), wkey0, min(wkey0 + 31, S - 1)))) {
        // S = Q K^T and dP = dO V^T, one chunk of both per step; the steps'
        // LDS operands (Q, dO and, with V_LDS, V) are read PF steps ahead.
        f32x16 s = zero16(), dp = zero16();
        {
            constexpr int R = V_LDS ? 3 : 2;
            struct Ops { bf16x8 q, g, v; };
            auto sread = [&](int c) {
                const int col = 16 * c + 8 * hh;
                Ops o;
                o.q = *reinterpret_cast<const bf16x8*>(Qb + tile_off<CPR, SWZ_DUAL>(n, col));
                o.g = *reinterpret_cast<const bf16x8*>(Gb + tile_off<CPR, SWZ_DUAL>(n, col));
                if constexpr (V_LDS)
                    o.v = *reinterpret_cast<const bf16x8*>(Vl + tile_off<CPR, SWZ_ROW>(32 * w + n, col));
                return o;
            };
            Ops ring[PF];
#pragma unroll
            for (int c = 0; c < PF; ++c) ring[c] = sread(c);
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const Ops o = ring[c % PF];
                if (c + PF < NC) ring[c % PF] = sread(c + PF);
                s = mfma_bf16(o.q, kf[c], s);
                if constexpr (V_LDS)
                    dp = mfma_bf16(o.g, o.v, dp);
                else
                    dp = mfma_bf16(o.g, vf[c], dp);
                // next block's loads, one per step, behind this step's MFMAs
                if (c < NPARTS) issue_part(pend, c);
            }
#pragma unroll
            for (int j = NC; j < NPARTS; ++j) issue_part(pend, j);
        }
        // lane column n = key; register r = query qb + row_of_reg(r, hh)
        const bool need_mask = wave_uniform(!vis.all(qb, qb + 31, wkey0, wkey0 + 31));
        // this lane's key is seen by rows qb + [r_lo, r_hi)
        const int r_lo = need_mask ? vis.rlo(key) - qb : -64, r_hi = need_mask ? vis.rhi(key) - qb : 64;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f32x4 l4 = *reinterpret_cast<const f32x4*>(stt + 8 * g + 4 * hh);
            const f32x4 d4 = *reinterpret_cast<const f32x4*>(stt + 32 + 8 * g + 4 * hh);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = 4 * g + i;
                float p = fast_exp2(s[r] * a.scale_log2 - l4[i]);
                const int rr = 8 * g + 4 * hh + i;
                p = (rr < r_lo || rr >= r_hi) ? 0.f : p;
                dp[r] = p * (dp[r] - d4[i]);
                s[r] = p;
            }
        }
#pragma unroll 1
        for (int e = 0; e < 2; ++e) {
            bf16x8 pb, db;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                pb[j] = (bf16)s[8 * e + j];
                db[j] = (bf16)dp[8 * e + j];
            }
            // dV^T += dO^T P (even steps) and dK^T += Q^T dS (odd steps); the
            // transposed A operands come two ds_read_b64_tr_b16 per step.
            const int r0 = 16 * e + 4 * hh + (i16 >> 2);
            constexpr int NI = 2 * NDT;
            auto tread = [&](int it) {
                const bf16* t = (it & 1) ? Qb : Gb;
                const int col = 32 * (it >> 1) + 16 * nh + 4 * (i16 & 3);
                const bf16x4 lo = ds_read_tr4(t + tile_off<CPR, SWZ_DUAL>(r0, col));
                const bf16x4 hi = ds_read_tr4(t + tile_off<CPR, SWZ_DUAL>(r0 + 8, col));
                return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            };
            bf16x8 ring[PF];
#pragma unroll
            for (int it = 0; it < PF; ++it) ring[it] = tread(it);
#pragma unroll
            for (int it = 0; it < NI; ++it) {
                const bf16x8 av = ring[it % PF];
                if (it + PF < NI) ring[it % PF] = tread(it + PF);
                if (it & 1)
                    dk[it >> 1] = mfma_bf16(av, db, dk[it >> 1]);
                else
                    dv[it >> 1] = mfma_bf16(av, pb, dv[it >> 1]);
            }
            pin_read_ahead<NI, PF, 2>();
        }
        } else {
#pragma unroll
            for (int j = 0; j < NPARTS; ++j) issue_part(pend, j);
        }  // active wave
      }
      // End of this unit's part of key tile kt: a tile covered by one unit
      // writes dK/dV, otherwise this unit's slot (split_slot): [dK | dV]
      // tiles of 128 key rows.
      const int key = kt * BNK + 32 * w + n;
      if (key < S) {
          float* dkp = a.dk + op_base<STRIDED>(a.sdk, b, hk, a.Hkv, S, D) + (int64_t)key * op_ld<STRIDED>(a.sdk, D);
          float* dvp = a.dv + op_base<STRIDED>(a.sdv, b, hk, a.Hkv, S, D) + (int64_t)key * op_ld<STRIDED>(a.sdv, D);
          if (fast_slots(kstart, kn, a.kv_chunk) > 1) {
              const int64_t slot = (int64_t)(b * a.Hkv + hk) * 2 * a.kv_units + 2 * unit + (first ? 0 : 1);
              dkp = a.kv_part + (slot * 2 * BNK + (32 * w + n)) * D;
              dvp = dkp + BNK * D;
          }
          store_dkdv<NDT>(a, dkp, dvp, hh, dk, dv);
      }
      if (i >= niter) {
          wait_vmcnt<0>();  // the last block's self-copy has landed before the unit ends
          break;
      }
      ++kt;
      kstart = fast_kv_start(S, CAUSAL, W, G, kt);
      kn = fast_kv_n(S, CAUSAL, W, G, kt);
#pragma unroll
      for (int d = 0; d < NDT; ++d) {
          dk[d] = zero16();
          dv[d] = zero16();
      }
      if constexpr (V_LDS) lds_barrier_vm<0>();  // all waves done with the old V tile
      load_keys(kt);
      if constexpr (V_LDS) lds_barrier_vm<0>();
      wait_vmcnt<0>();
    }
}

template <int DP, bool CAUSAL, bool STRIDED>
__device__ __forceinline__ void dq_fast_body(const BwdArgs& a, bf16* smem, int unit, int b, int h) {
    constexpr int NT = 256, BN = 64, BM = 128, CPR = DP / 8, NC = DP / 16, NDT = DP / 32, NKK = BN / 32;
    constexpr int TILE = BN * DP;
    constexpr int PER = BN * CPR / NT;  // loads per thread of a K (V) tile: the K tile's are spread
                                        // over the S/dP steps of kk = 0, the V tile's over kk = 1
    static_assert(NKK == 2, "one tile's loads per 32-key block");
    constexpr int BUF = BwdFastLds<DP>::Q_BUF;
    constexpr int PF = 4;  // LDS operand prefetch depth

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 31, hh = lane >> 5;
    const int i16 = lane & 15, nh = (lane >> 4) & 1;
    const int wu = wave_id();
    const int S = a.S, D = a.D, W = a.window;
    const KeyVis vis = key_vis(a, b, CAUSAL);
    const int hk = h / a.group;
    const bf16* K = (const bf16*)a.k + op_base<STRIDED>(a.sk, b, hk, a.Hkv, S, D);
    const bf16* Vg = (const bf16*)a.v + op_base<STRIDED>(a.sv, b, hk, a.Hkv, S, D);
    const bf16* Q = (const bf16*)a.q + op_base<STRIDED>(a.sq, b, h, a.Hq, S, D);
    const bf16* G = (const bf16*)a.dO + op_base<STRIDED>(a.sdo, b, h, a.Hq, S, D);
    const int lk = op_ld<STRIDED>(a.sk, D), lv = lk;  // one K/V sequence stride, as in dkdv_fast_body

    // This unit's chunk of the flattened (query tile, key tile) iterations.
    const int64_t g0 = (int64_t)unit * a.q_chunk;
    const int niter = (int)min((int64_t)a.q_chunk, fast_q_total(S, CAUSAL, W) - g0);
    int qt = 0;
    while (fast_q_start(S, CAUSAL, W, qt + 1) <= g0) ++qt;
    // Prefetch cursor: query tile and key tile of the next iteration to load
    // (pf_t counts from the tile's first key tile pf_lo).
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
        const int kt0 = next_key_tile();
        issue_tile<DP, BN, NT, SWZ_DUAL>(K, kt0 * BN, S, D, lk, smem);
        issue_tile<DP, BN, NT, SWZ_ROW>(Vg, kt0 * BN, S, D, lv, smem + TILE);
    }

    bf16x8 qf[NC], gf[NC];
    float lse2, dlt;
    auto load_rows = [&](int t) {  // this lane's query row of tile t: Q, dO fragments and row terms
        const int row = t * BM + 32 * w + n, rowc = row < S ? row : S - 1;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            qf[c] = load_chunk<bf16>(Q + (int64_t)rowc * op_ld<STRIDED>(a.sq, D), 16 * c + 8 * hh, D, row < S, true);
            gf[c] = load_chunk<bf16>(G + (int64_t)rowc * op_ld<STRIDED>(a.sdo, D), 16 * c + 8 * hh, D, row < S, true);
        }
        const float* blk = a.stats + ((int64_t)(b * a.Hq + h) * a.nqb_total + rowc / 32) * 64;
        lse2 = row < S ? blk[rowc % 32] : INFINITY;
        dlt = row < S ? blk[32 + rowc % 32] : 0.f;
    };
    load_rows(qt);
    wait_vmcnt<0>();
    int64_t qstart = fast_q_start(S, CAUSAL, W, qt);
    int qn = fast_q_n(S, CAUSAL, W, qt);
    int qlo = fast_q_lo(CAUSAL, W, qt);

    f32x16 dq[NDT];
#pragma unroll
    for (int i = 0; i < NDT; ++i) dq[i] = zero16();

    for (int i = 0, first = 1;; first = 0) {
      // Iterations of query tile qt inside this unit, then its dQ store.
      const int seg_end = (int)min((int64_t)niter, qstart + qn - g0);
      for (; i < seg_end; ++i) {
        const bf16* Kb = smem + (i & 1) * BUF;
        const bf16* Vb = Kb + TILE;
        wait_vmcnt<0>();  // see dkdv_fast_body
        lds_barrier();
        // Next key tile's loads (K then V, NPARTS per thread), spread over the
        // S/dP steps below; the last block re-loads key tile 0 into the idle
        // buffer so that the schedule has no branch (waited for at the end).
        bf16* const nbuf = smem + ((i + 1) & 1) * BUF;
        const int ktn = i + 1 < niter ? next_key_tile() : 0;
        // Load j of the K tile (v = 0) or of the V tile (v = 1; v may be a
        // runtime value: the two tiles differ only in source, destination
        // and swizzle, which are selected without a branch).
        auto issue_part = [&](int v, int j) {
            const int m = wu * PER + j, P = m * 64 + lane;
            const int r = P / CPR, p = P % CPR;
            const int c = p ^ (v ? swz<CPR, SWZ_ROW>(r) : swz<CPR, SWZ_DUAL>(r));
            const int gr = min(ktn * BN + r, S - 1);
            const int col = 8 * c < D ? 8 * c : 0;
            if constexpr (STRIDED)
                load_lds_16((v ? Vg : K) + (gr * (v ? lv : lk) + col), (v ? nbuf + TILE : nbuf) + m * 512);
            else
                load_lds_16((v ? Vg : K) + (int64_t)gr * D + col, (v ? nbuf + TILE : nbuf) + m * 512);
        };
        const int kbase = (qlo + (int)(g0 + i - qstart)) * BN;
        const int wrow0 = qt * BM + 32 * w, row = wrow0 + n;
        if (wave_uniform(wrow0 < S && vis.any(wrow0, min(wrow0 + 31, S - 1), kbase, kbase + BN - 1))) {
        const bool need_mask = wave_uniform(!vis.all(wrow0, wrow0 + 31, kbase, kbase + BN - 1));
#pragma unroll 1
        for (int kk = 0; kk < NKK; ++kk) {
            f32x16 s = zero16(), dp = zero16();
            const int r = 32 * kk + n;
            {
                // S^T = K Q^T (even steps), dP^T = V dO^T (odd steps)
                constexpr int NI = 2 * NC;
                auto aread = [&](int it) {
                    const int col = 16 * (it >> 1) + 8 * hh;
                    return (it & 1) ? *reinterpret_cast<const bf16x8*>(Vb + tile_off<CPR, SWZ_ROW>(r, col))
                                    : *reinterpret_cast<const bf16x8*>(Kb + tile_off<CPR, SWZ_DUAL>(r, col));
                };
                bf16x8 ring[PF];
#pragma unroll
                for (int it = 0; it < PF; ++it) ring[it] = aread(it);
#pragma unroll
                for (int it = 0; it < NI; ++it) {
                    const bf16x8 av = ring[it % PF];
                    if (it + PF < NI) ring[it % PF] = aread(it + PF);
                    if (it & 1)
                        dp = mfma_bf16(av, gf[it >> 1], dp);
                    else
                        s = mfma_bf16(av, qf[it >> 1], s);
                    if ((it & 1) && (it >> 1) < PER) issue_part(kk, it >> 1);
                }
#pragma unroll
                for (int j = NI / 2; j < PER; ++j) issue_part(kk, j);
            }
            // lane column n = query row; register r = key kbase + 32kk + row_of_reg(r, hh),
            // visible iff lo <= row_of_reg(r, hh) <= hi
            const int hi = need_mask ? vis.hi(row) - kbase - 32 * kk : 64;
            const int lo = need_mask ? vis.lo(row) - kbase - 32 * kk : -1;
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                float p = fast_exp2(s[q] * a.scale_log2 - lse2);
                p = (row_of_reg(q, hh) > hi || row_of_reg(q, hh) < lo) ? 0.f : p;
                s[q] = p * (dp[q] - dlt);
            }
            {
                // dQ^T += K^T dS^T over the two 16-key halves (e) of this block
                bf16x8 db[2];
#pragma unroll
                for (int e = 0; e < 2; ++e)
#pragma unroll
                    for (int j = 0; j < 8; ++j) db[e][j] = (bf16)s[8 * e + j];
                constexpr int NI = 2 * NDT;
                auto tread = [&](int it) {
                    const int r0 = 32 * kk + 16 * (it / NDT) + 4 * hh + (i16 >> 2);
                    const int col = 32 * (it % NDT) + 16 * nh + 4 * (i16 & 3);
                    const bf16x4 lo = ds_read_tr4(Kb + tile_off<CPR, SWZ_DUAL>(r0, col));
                    const bf16x4 hi = ds_read_tr4(Kb + tile_off<CPR, SWZ_DUAL>(r0 + 8, col));
                    return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                };
                bf16x8 ring[PF];
#pragma unroll
                for (int it = 0; it < PF; ++it) ring[it] = tread(it);
#pragma unroll
                for (int it = 0; it < NI; ++it) {
                    const bf16x8 av = ring[it % PF];
                    if (it + PF < NI) ring[it % PF] = tread(it + PF);
                    dq[it % NDT] = mfma_bf16(av, db[it / NDT], dq[it % NDT]);
                }
                pin_read_ahead<NI, PF, 2>();
            }
        }
        } else {
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                issue_part(0, j);
                issue_part(1, j);
            }
        }  // active wave
      }
      // End of this unit's part of query tile qt: a tile covered by one unit
      // writes dQ, otherwise slot (unit - first unit of qt).
      const int row = qt * BM + 32 * w + n;
      if (row < S) {
          float* dqp = a.dq + op_base<STRIDED>(a.sdq, b, h, a.Hq, S, D) + (int64_t)row * op_ld<STRIDED>(a.sdq, D);
          if (fast_slots(qstart, qn, a.q_chunk) > 1) {
              const int64_t slot = (int64_t)(b * a.Hq + h) * 2 * a.q_units + 2 * unit + (first ? 0 : 1);
              dqp = a.q_part + (slot * BM + 32 * w + n) * D;
          }
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
              for (int g = 0; g < 4; ++g)
                  store4<float>(dqp, 32 * dt + 8 * g + 4 * hh, D, dq[dt][4 * g] * a.scale,
                                dq[dt][4 * g + 1] * a.scale, dq[dt][4 * g + 2] * a.scale,
                                dq[dt][4 * g + 3] * a.scale, true);
      }
      if (i >= niter) {
          wait_vmcnt<0>();  // the last block's re-load has landed before the unit ends
          break;
      }
      ++qt;
      qstart = fast_q_start(S, CAUSAL, W, qt);
      qn = fast_q_n(S, CAUSAL, W, qt);
      qlo = fast_q_lo(CAUSAL, W, qt);
#pragma unroll
      for (int d = 0; d < NDT; ++d) dq[d] = zero16();
      load_rows(qt);
      wait_vmcnt<0>();
    }
}

// One workgroup per unit; unit u of every (batch, head) precedes unit u+1.
template <int DP, bool CAUSAL, bool STRIDED>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_bf16_fast(BwdArgs a) {
    __shared__ __attribute__((aligned(1024))) bf16 smem[BwdFastLds<DP>::KV_ELEMS];
    const int bh = a.B * a.Hkv, i = (int)blockIdx.x;
    dkdv_fast_body<DP, CAUSAL, STRIDED>(a, smem, i / bh, (i % bh) / a.Hkv, (i % bh) % a.Hkv);
}

template <int DP, bool CAUSAL, bool STRIDED>
__global__ __launch_bounds__(256) void attn_bwd_dq_bf16_fast(BwdArgs a) {
    __shared__ __attribute__((aligned(1024))) bf16 smem[BwdFastLds<DP>::Q_ELEMS];
    const int bh = a.B * a.Hq, i = (int)blockIdx.x;
    dq_fast_body<DP, CAUSAL, STRIDED>(a, smem, i / bh, (i % bh) / a.Hq, (i % bh) % a.Hq);
}

// Both roles in one grid: the first kv_units * B * Hkv workgroups run dK/dV
// units, the rest dQ units (the units of both are sized to take about equally
// long, see plan_bwd_fast).
template <int DP, bool CAUSAL, bool STRIDED>
__global__ __launch_bounds__(256) void attn_bwd_main_bf16_fast(BwdArgs a) {
    __shared__ __attribute__((aligned(1024))) bf16 smem[BwdFastLds<DP>::ELEMS];
    const int nkv = a.kv_units * a.B * a.Hkv;
    const int i = (int)blockIdx.x;
    if (i < nkv) {
        const int bh = a.B * a.Hkv;
        dkdv_fast_body<DP, CAUSAL, STRIDED>(a, smem, i / bh, (i % bh) / a.Hkv, (i % bh) % a.Hkv);
    } else {
        const int j = i - nkv, bh = a.B * a.Hq;
        dq_fast_body<DP, CAUSAL, STRIDED>(a, smem, j / bh, (j % bh) / a.Hq, (j % bh) % a.Hq);
    }
}

// REDUCE: sum the partial slots of every split tile in unit order.  One
// workgroup per (batch, head, 128-row tile, 16-row group) of the dK/dV role
// (rows = keys; dK and dV) and then of the dQ role (rows = queries);
// workgroups of unsplit tiles return at once.
constexpr int kRedRows = 16, kRedMaxSlots = 64;

__device__ __forceinline__ void reduce_rows(const float* part, const int64_t* slot_of, int nsl, int64_t tile_elems,
                                            int64_t row_in_tile, int D, float* dst) {
    // thread -> 16-byte column chunks (tid % 16) + 16 j of row tid / 16
    const int cl = threadIdx.x % 16, cg = D / 4;
    constexpr int MAXJ = 256 / 4 / 16;
    f32x4 acc[MAXJ];
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int p = 0; p < nsl; ++p) {
        const float* src = part + slot_of[p] * tile_elems + row_in_tile * D;
        f32x4 x[MAXJ];
#pragma unroll
        for (int j = 0; j < MAXJ; ++j) {
            const int c = cl + 16 * j;
            x[j] = c < cg ? *reinterpret_cast<const f32x4*>(src + 4 * c) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int j = 0; j < MAXJ; ++j) acc[j] += x[j];
    }
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) {
        const int c = cl + 16 * j;
        if (c < cg) *reinterpret_cast<f32x4*>(dst + 4 * c) = acc[j];
    }
}

template <bool CAUSAL>
__global__ __launch_bounds__(256) void attn_bwd_fast_reduce(BwdArgs a) {
    constexpr int RG = 128 / kRedRows;
    __shared__ int64_t slot_of[kRedMaxSlots];
    const int S = a.S, D = a.D, nt = (S + 127) / 128;
    const int64_t kv_blocks = (int64_t)a.B * a.Hkv * nt * RG;
    int64_t blk = blockIdx.x;
    const bool kv = blk < kv_blocks;
    if (!kv) blk -= kv_blocks;
    const int rg = (int)(blk % RG), t = (int)((blk / RG) % nt), bh = (int)(blk / (RG * nt));
    const int64_t start = kv ? fast_kv_start(S, CAUSAL, a.window, a.group, t) : fast_q_start(S, CAUSAL, a.window, t);
    const int n = kv ? fast_kv_n(S, CAUSAL, a.window, a.group, t) : fast_q_n(S, CAUSAL, a.window, t);
    const int64_t chunk = kv ? a.kv_chunk : a.q_chunk;
    const int nsl = fast_slots(start, n, chunk);
    const int r0 = t * 128 + rg * kRedRows;
    if (nsl <= 1 || r0 >= S) return;
    const int64_t u0 = start / chunk, head_slots = (int64_t)bh * 2 * (kv ? a.kv_units : a.q_units);
    if ((int)threadIdx.x < nsl) slot_of[threadIdx.x] = head_slots + split_slot(start, chunk, u0 + threadIdx.x, u0);
    __syncthreads();
    const int r = threadIdx.x / 16;
    if (r0 + r >= S) return;
    const int64_t row = r0 + r;
    const int64_t rit = rg * kRedRows + r;  // row inside the tile
    if (kv) {
        // slot layout [dK rows 0..127][dV rows 0..127]
        const int bb = bh / a.Hkv, hk = bh % a.Hkv;
        reduce_rows(a.kv_part, slot_of, nsl, 2 * 128 * (int64_t)D, rit, D,
                    a.dk + a.sdk.at(bb, hk) + row * a.sdk.s);
        reduce_rows(a.kv_part, slot_of, nsl, 2 * 128 * (int64_t)D, 128 + rit, D,
                    a.dv + a.sdv.at(bb, hk) + row * a.sdv.s);
    } else {
        const int bb = bh / a.Hq, h = bh % a.Hq;
        reduce_rows(a.q_part, slot_of, nsl, 128 * (int64_t)D, rit, D, a.dq + a.sdq.at(bb, h) + row * a.sdq.s);
    }
}

template <int DP>
hipError_t launch_bwd_fast(const AttnShape& s, BwdArgs a, int stages, hipStream_t st) {
    if (stages & BWD_STAGE_DELTA) {
        constexpr int RPB = 256 / (DP / 8);
        const int64_t rows = s.B * s.Hq * (int64_t)a.nqb_total * 32;
        hipLaunchKernelGGL((attn_bwd_stats_kernel<bf16, DP>), dim3((unsigned)((rows + RPB - 1) / RPB)), dim3(256), 0,
                           st, a);
    }
    const BwdPlan pl = plan_bwd_fast(s);
    const bool strided = !s.contiguous;
    // (causal, strided) -> instantiation
#define MFT_BWD_LAUNCH(KERNEL, GRID)                                                      \
    do {                                                                                  \
        if (s.causal && strided)                                                          \
            hipLaunchKernelGGL((KERNEL<DP, true, true>), GRID, dim3(256), 0, st, a);      \
        else if (s.causal)                                                                \
            hipLaunchKernelGGL((KERNEL<DP, true, false>), GRID, dim3(256), 0, st, a);     \
        else if (strided)                                                                 \
            hipLaunchKernelGGL((KERNEL<DP, false, true>), GRID, dim3(256), 0, st, a);     \
        else                                                                              \
            hipLaunchKernelGGL((KERNEL<DP, false, false>), GRID, dim3(256), 0, st, a);    \
    } while (0)
    if ((stages & BWD_STAGE_MAIN) == BWD_STAGE_MAIN) {
        MFT_BWD_LAUNCH(attn_bwd_main_bf16_fast, dim3((unsigned)(pl.kv_units * s.B * s.Hkv + pl.q_units * s.B * s.Hq)));
    } else if (stages & BWD_STAGE_DKDV) {
        MFT_BWD_LAUNCH(attn_bwd_dkdv_bf16_fast, dim3((unsigned)(pl.kv_units * s.B * s.Hkv)));
    } else if (stages & BWD_STAGE_DQ) {
        MFT_BWD_LAUNCH(attn_bwd_dq_bf16_fast, dim3((unsigned)(pl.q_units * s.B * s.Hq)));
    }
#undef MFT_BWD_LAUNCH
    if ((stages & BWD_STAGE_REDUCE) && (pl.kv_parts_max > 1 || pl.q_parts_max > 1)) {
        const int64_t nt = (s.S + 127) / 128;
        const int64_t blocks = (s.B * s.Hkv + s.B * s.Hq) * nt * (128 / kRedRows);
        if (s.causal)
            hipLaunchKernelGGL(attn_bwd_fast_reduce<true>, dim3((unsigned)blocks), dim3(256), 0, st, a);
        else
            hipLaunchKernelGGL(attn_bwd_fast_reduce<false>, dim3((unsigned)blocks), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}


}  // namespace
}  // namespace bwd
}  // namespace mft
