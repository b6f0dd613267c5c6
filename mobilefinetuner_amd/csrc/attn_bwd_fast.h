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
    // a wave's 512 registers.
    static constexpr bool V_LDS = DP >= 256;
    // dK/dV role, in elements: [Q tile 0][Q tile 1][dO tile 0][dO tile 1]
    // (32 x DP each), [stats 0][stats 1] (4 waves x 1 KiB each), then V of the
    // key tile (128 x DP).  Keeping the four operand tiles first keeps every
    // read's tile and step offsets inside the 16-bit immediate.
    static constexpr int QT = 32 * DP;
    static constexpr int ST_OFF = 4 * QT, ST = 4 * 512;
    static constexpr int V_OFF = ST_OFF + 2 * ST;
    static constexpr int KV_ELEMS = V_OFF + (V_LDS ? 128 * DP : 0);
    // dQ role: [K tile 0][K tile 1][V tile 0][V tile 1], 64 x DP each.
    static constexpr int KT = 64 * DP;
    static constexpr int Q_ELEMS = 4 * KT;
    static constexpr int ELEMS = KV_ELEMS > Q_ELEMS ? KV_ELEMS : Q_ELEMS;
};

// Per-lane, loop-invariant LDS read offsets (bytes) of the fast backward's
// SWZ_DUAL tiles, shared by both roles (tests/native/offsets_check.cpp checks
// them against tile_off):
//  rr[j]: row reads.  Row 32k + n, column chunk 2c + hh:
//         n*ROWB + (32c ^ 16 (hh ^ swz_dual(n))) + 32k*ROWB, and c, c + 8 differ
//         by 256 bytes: rr[c % 8].
//  tr[hi][j]: transposing reads (ds_read_b64_tr_b16) of rows
//         32k + 16e + 8hi + 4hh + i16/4, columns 32dt + 16nh + 4 (i16 & 3):
//         the row's swizzle depends on (hi, lane) only, so the offset is
//         tr[hi][dt % 4] + (32k + 16e)*ROWB + 256 (dt / 4).
template <int DP> struct BwdLane {
    static constexpr int CPR = DP / 8, ROWB = DP * 2, NC = DP / 16, NDT = DP / 32;
    static constexpr int KC = NC < 8 ? NC : 8;
    static constexpr int VC = NDT < 4 ? NDT : 4;
    uint32_t rr[KC];
    uint32_t tr[2][VC];
    __host__ __device__ void init(int lane) {
        const int n = lane & 31, hh = lane >> 5, i16 = lane & 15, nh = (lane >> 4) & 1;
        const uint32_t y16 = 16u * (uint32_t)(hh ^ swz_dual<CPR>(n));
#pragma unroll
        for (int j = 0; j < KC; ++j) rr[j] = (uint32_t)n * ROWB + ((32u * j) ^ y16);
        const int W = 2 * nh + ((i16 & 3) >> 1);
#pragma unroll
        for (int hi = 0; hi < 2; ++hi) {
            const int rlow = 8 * hi + 4 * hh + (i16 >> 2);
            const int sw = swz_dual<CPR>(rlow);
#pragma unroll
            for (int j = 0; j < VC; ++j)
                tr[hi][j] = (uint32_t)rlow * ROWB + 16u * (uint32_t)((4 * j + W) ^ sw) + 8u * (i16 & 1);
        }
    }
    __host__ __device__ uint32_t row(int k, int c) const { return rr[c % KC] + k * 32 * ROWB + (c / KC) * 256; }
    __host__ __device__ uint32_t trn(int k, int e, int dt, int hi) const {
        return tr[hi][dt % VC] + (32 * k + 16 * e) * ROWB + (dt / VC) * 256;
    }
};

// The score products S and dP of one step.  ASM: the VGPR-form inline-asm
// MFMAs (attn_common.h), used where the loop-carried accumulators fill the
// AGPRs (D = 256); otherwise the builtin.  The first product of a chain is
// always the asm form (see mfma_v_first).
template <bool ASM>
__device__ __forceinline__ void mm_score(f32x16& c, const bf16x8& a, const bf16x8& b, bool first) {
    if (first)
        mfma_v_first(c, a, b);
    else if constexpr (ASM)
        mfma_v(c, a, b);
    else
        c = mfma_bf16(a, b, c);
}

template <int DP, bool CAUSAL, bool STRIDED, bool FAST>
__device__ __forceinline__ void dkdv_fast_body(const BwdArgs& a, bf16* smem, int unit, int b, int hk) {
    typedef BwdFastLds<DP> L;
    constexpr int NT = 256, BNK = 128, CPR = DP / 8, NC = DP / 16, NDT = DP / 32;
    constexpr bool V_LDS = L::V_LDS, ASM = DP >= 256;
    constexpr int PF = 2;  // LDS operand prefetch depth
    constexpr int QTB = L::QT * 2;  // bytes of one Q or dO tile

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 31, hh = lane >> 5;
    const int i16 = lane & 15;
    const int S = a.S, D = a.D, G = a.group, W = a.window;
    const KeyVis vis = key_vis(a, b, CAUSAL);
    const bf16* K = (const bf16*)a.k + op_base<STRIDED>(a.sk, b, hk, a.Hkv, S, D);
    const bf16* Vg = (const bf16*)a.v + op_base<STRIDED>(a.sv, b, hk, a.Hkv, S, D);
    // K and V share one sequence stride on this path (bwd_fast_path): a
    // second stride live across the loop costs the dK/dV accumulators their
    // registers (the compiler then shuffles them every block).
    const int lk = op_ld<STRIDED>(a.sk, D), lv = lk;
    const int lq = op_ld<STRIDED>(a.sq, D), lg = op_ld<STRIDED>(a.sdo, D);
    BwdLane<DP> ln;
    ln.init(lane);
    const uint32_t smem_addr = lds_addr(smem);
    TileDma<DP, 32, NT, SWZ_DUAL> dmq, dmg;
    dmq.init(lane, wave_id(), lq);
    dmg.init(lane, wave_id(), lg);

    // This unit's chunk of the flattened (key tile, query head, query block)
    // iterations; it may start inside one key tile and end inside a later one.
    const FastTiles tiles{S, CAUSAL, W, G, 1};
    const int64_t g0 = unit_first(tiles, a.kv_us, unit);
    const int niter = (int)(unit_first(tiles, a.kv_us, unit + 1) - g0);
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
        int par, qb;
    };
    auto issue_begin = [&](int par) {
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
                       a.stats + ((int64_t)(b * a.Hq + h) * a.nqb_total + qb / 32) * 64, par, qb};
    };
    auto issue_part = [&](const Pending& p, int j) {
        if (j < PER)
            issue_tile_j<FAST, DP, 32, NT, SWZ_DUAL>(dmq, p.q, p.qb, S, D, lq, smem + p.par * L::QT,
                                                     smem_addr + 2u * p.par * L::QT, j);
        else if (j < 2 * PER)
            issue_tile_j<FAST, DP, 32, NT, SWZ_DUAL>(dmg, p.g, p.qb, S, D, lg, smem + (2 + p.par) * L::QT,
                                                     smem_addr + 2u * (2 + p.par) * L::QT, j - PER);
        else
            load_lds_16(p.st + 4 * i16, smem + L::ST_OFF + p.par * L::ST + w * 512);
    };
    auto issue = [&](int par) {
        const Pending p = issue_begin(par);
#pragma unroll
        for (int j = 0; j < NPARTS; ++j) issue_part(p, j);
        return p.qb;
    };

    bf16* Vl = smem + L::V_OFF;  // V rows of the current key tile (V_LDS only)
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
            issue_tile<DP, BNK, NT, SWZ_DUAL>(Vg, t * BNK, S, D, lv, Vl);
            if (D < DP) {
                // Staged columns >= D hold copies of column chunk 0, and so do
                // those of the dO tiles: zero them so that dP = dO V^T sums
                // only the D real columns.
                lds_barrier_vm<0>();
                const bf16x8 z = zero_vec<bf16x8>();
                for (int idx = tid; idx < BNK * CPR; idx += NT) {
                    const int r = idx / CPR, c = idx % CPR;
                    if (8 * c >= D) *reinterpret_cast<bf16x8*>(Vl + r * DP + ((c ^ swz_dual<CPR>(r)) << 3)) = z;
                }
            }
        }
    };
    load_keys(kt);
    int cur_qb = issue(0);  // query block of the block in the current buffer
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
        const int par = i & 1;
        const char* Qb = reinterpret_cast<const char*>(smem) + par * QTB;   // Q tile; dO tile at + 2 QTB
        const float* stt = reinterpret_cast<const float*>(smem + L::ST_OFF + par * L::ST + w * 512);
        // This wave's loads of buffer par (issued one iteration ago) have
        // landed; after the barrier every wave's have, and every wave is done
        // with buffer par ^ 1, which the next block then streams into.
        wait_vmcnt<0>();
        lds_barrier();
        // The last block prefetches a harmless copy of itself into the idle
        // buffer, so that the load schedule below needs no branch (the unit
        // waits for it before it ends).
        const Pending pend = i + 1 < niter ? issue_begin(par ^ 1)
                                           : Pending{(const bf16*)a.q, (const bf16*)a.dO, a.stats, par ^ 1, 0};
        const int qb = cur_qb;
        cur_qb = pend.qb;
        const int wkey0 = kt * BNK + 32 * w;
        const int key = wkey0 + n;
        // Waves whose keys are past S, or none of which a row of this query
        // block sees, skip it.
        if (wave_uniform(wkey0 < S && vis.any(qb, min(qb + 31, S - 1), wkey0, min(wkey0 + 31, S - 1)))) {
        // S = Q K^T and dP = dO V^T, one chunk of both per step; the steps'
        // LDS operands (Q, dO and, with V_LDS, V) are read PF steps ahead.
        f32x16 s, dp;
        {
            const char* Vw = reinterpret_cast<const char*>(Vl) + 32 * w * 2 * DP;  // this wave's 32 V rows
            struct Ops { bf16x8 q, g, v; };
            auto sread = [&](int c) {
                Ops o;
                o.q = *reinterpret_cast<const bf16x8*>(Qb + ln.row(0, c));
                o.g = *reinterpret_cast<const bf16x8*>(Qb + 2 * QTB + ln.row(0, c));
                if constexpr (V_LDS) o.v = *reinterpret_cast<const bf16x8*>(Vw + ln.row(0, c));
                return o;
            };
            Ops ring[PF];
#pragma unroll
            for (int c = 0; c < PF; ++c) ring[c] = sread(c);
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const Ops o = ring[c % PF];
                if (c + PF < NC) ring[c % PF] = sread(c + PF);
                mm_score<ASM>(s, o.q, kf[c], c == 0);
                if constexpr (V_LDS)
                    mm_score<ASM>(dp, o.g, o.v, c == 0);
                else
                    mm_score<ASM>(dp, o.g, vf[c], c == 0);
                // next block's loads, one per step, behind this step's MFMAs
                if (c < NPARTS) issue_part(pend, c);
            }
#pragma unroll
            for (int j = NC; j < NPARTS; ++j) issue_part(pend, j);
            if constexpr (ASM) mfma_v_drain(s, dp);
        }
        // lane column n = key; register r = query qb + row_of_reg(r, hh)
        float lse_r[16], dlt_r[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f32x4 l4 = *reinterpret_cast<const f32x4*>(stt + 8 * g + 4 * hh);
            const f32x4 d4 = *reinterpret_cast<const f32x4*>(stt + 32 + 8 * g + 4 * hh);
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2) {
                lse_r[4 * g + i2] = l4[i2];
                dlt_r[4 * g + i2] = d4[i2];
            }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = fast_exp2(s[r] * a.scale_log2 - lse_r[r]);
        if (wave_uniform(!vis.all(qb, qb + 31, wkey0, wkey0 + 31))) {
            // this lane's key is seen by rows qb + [r_lo, r_hi); the bounds
            // pass through an asm statement inside the branch so that the
            // selects stay in it (blocks without masked pairs skip them)
            int r_lo = vis.rlo(key) - qb, r_hi = vis.rhi(key) - qb;
            asm volatile("" : "+v"(r_lo), "+v"(r_hi));
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int rr = row_of_reg(r, hh);
                s[r] = (rr < r_lo || rr >= r_hi) ? 0.f : s[r];
            }
        }
        bf16x8 pb[2], db[2];
#pragma unroll
        for (int e = 0; e < 2; ++e)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int r = 8 * e + j;
                pb[e][j] = (bf16)s[r];
                db[e][j] = (bf16)(s[r] * (dp[r] - dlt_r[r]));
            }
        // dV^T += dO^T P (even steps) and dK^T += Q^T dS (odd steps); the
        // transposed A operands come two ds_read_b64_tr_b16 per step, their
        // halves through rings of their own (see the forward).
        {
            constexpr int NI = 4 * NDT;  // (e, dt, operand)
            auto tread = [&](int it, int hi) {
                const int e = it / (2 * NDT), dt = (it / 2) % NDT;
                const char* t = (it & 1) ? Qb : Qb + 2 * QTB;
                return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(t + ln.trn(0, e, dt, hi)));
            };
            v4i16 rl[PF], rh[PF];
#pragma unroll
            for (int it = 0; it < PF; ++it) {
                rl[it] = tread(it, 0);
                rh[it] = tread(it, 1);
            }
#pragma unroll
            for (int it = 0; it < NI; ++it) {
                const bf16x8 av =
                    __builtin_bit_cast(bf16x8, __builtin_shufflevector(rl[it % PF], rh[it % PF], 0, 1, 2, 3, 4, 5, 6, 7));
                if (it + PF < NI) {
                    rl[it % PF] = tread(it + PF, 0);
                    rh[it % PF] = tread(it + PF, 1);
                }
                const int e = it / (2 * NDT), dt = (it / 2) % NDT;
                if (it & 1)
                    dk[dt] = mfma_bf16(av, db[e], dk[dt]);
                else
                    dv[dt] = mfma_bf16(av, pb[e], dv[dt]);
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
      const int key0 = kt * BNK + 32 * w;
      if constexpr (V_LDS && FAST) {
          // Whole tiles (FAST: D == DP, 16-byte rows, and key0 < S means all
          // 32 rows are): through LDS (store_acc32_staged), this wave's
          // quarter of the V tile as its staging area once every wave is done
          // with V.
          lds_barrier();
          if (wave_uniform(key0 < S)) {
              float* dkp = a.dk + op_base<STRIDED>(a.sdk, b, hk, a.Hkv, S, D) + (int64_t)key0 * op_ld<STRIDED>(a.sdk, D);
              float* dvp = a.dv + op_base<STRIDED>(a.sdv, b, hk, a.Hkv, S, D) + (int64_t)key0 * op_ld<STRIDED>(a.sdv, D);
              int64_t ldk = op_ld<STRIDED>(a.sdk, D), ldv = op_ld<STRIDED>(a.sdv, D);
              if (tile_units(tiles, a.kv_us, kt) > 1) {
                  const int64_t slot = (int64_t)(b * a.Hkv + hk) * 2 * a.kv_us.units + 2 * unit + (first ? 0 : 1);
                  dkp = a.kv_part + (slot * 2 * BNK + 32 * w) * D;
                  dvp = dkp + BNK * D;
                  ldk = ldv = D;
              }
              char* stage = reinterpret_cast<char*>(Vl) + w * (32 * DP * 2);
              store_acc32_staged<NDT, 4>(stage, dkp, ldk, dk, a.scale);
              store_acc32_staged<NDT, 4>(stage, dvp, ldv, dv, 1.f);
          }
      } else if (key0 + n < S) {
          const int key = key0 + n;
          float* dkp = a.dk + op_base<STRIDED>(a.sdk, b, hk, a.Hkv, S, D) + (int64_t)key * op_ld<STRIDED>(a.sdk, D);
          float* dvp = a.dv + op_base<STRIDED>(a.sdv, b, hk, a.Hkv, S, D) + (int64_t)key * op_ld<STRIDED>(a.sdv, D);
          if (tile_units(tiles, a.kv_us, kt) > 1) {
              const int64_t slot = (int64_t)(b * a.Hkv + hk) * 2 * a.kv_us.units + 2 * unit + (first ? 0 : 1);
              dkp = a.kv_part + (slot * 2 * BNK + key - kt * BNK) * D;
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

template <int DP, bool CAUSAL, bool STRIDED, bool FAST>
__device__ __forceinline__ void dq_fast_body(const BwdArgs& a, bf16* smem, int unit, int b, int h) {
    typedef BwdFastLds<DP> L;
    constexpr int NT = 256, BN = 64, BM = 128, CPR = DP / 8, NC = DP / 16, NDT = DP / 32, NKK = BN / 32;
    constexpr int KTB = L::KT * 2;  // bytes of one K or V tile
    constexpr int PER = BN * CPR / NT;  // loads per thread of a K (V) tile: the K tile's are spread
                                        // over the S/dP steps of kk = 0, the V tile's over kk = 1
    static_assert(NKK == 2, "one tile's loads per 32-key block");
    constexpr bool ASM = DP >= 256;
    constexpr int PF = 2;  // LDS operand prefetch depth

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 31, hh = lane >> 5;
    const int S = a.S, D = a.D, W = a.window;
    const KeyVis vis = key_vis(a, b, CAUSAL);
    const int hk = h / a.group;
    const bf16* K = (const bf16*)a.k + op_base<STRIDED>(a.sk, b, hk, a.Hkv, S, D);
    const bf16* Vg = (const bf16*)a.v + op_base<STRIDED>(a.sv, b, hk, a.Hkv, S, D);
    const bf16* Q = (const bf16*)a.q + op_base<STRIDED>(a.sq, b, h, a.Hq, S, D);
    const bf16* G = (const bf16*)a.dO + op_base<STRIDED>(a.sdo, b, h, a.Hq, S, D);
    const int lk = op_ld<STRIDED>(a.sk, D), lv = lk;  // one K/V sequence stride, as in dkdv_fast_body
    BwdLane<DP> ln;
    ln.init(lane);
    const uint32_t smem_addr = lds_addr(smem);
    TileDma<DP, BN, NT, SWZ_DUAL> dmk;
    dmk.init(lane, wave_id(), lk);

    // This unit's range of the flattened (query tile, key tile) iterations.
    const FastTiles tiles{S, CAUSAL, W, a.group, 0};
    const int64_t g0 = unit_first(tiles, a.q_us, unit);
    const int niter = (int)(unit_first(tiles, a.q_us, unit + 1) - g0);
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
    // Load j of the K tile (v = 0) or of the V tile (v = 1) of key tile ktn
    // into buffer par.
    auto issue_kv = [&](int v, int ktn, int par, int j) {
        if (v)
            issue_tile_j<FAST, DP, BN, NT, SWZ_DUAL>(dmk, Vg, ktn * BN, S, D, lv, smem + (2 + par) * L::KT,
                                                     smem_addr + 2u * (2 + par) * L::KT, j);
        else
            issue_tile_j<FAST, DP, BN, NT, SWZ_DUAL>(dmk, K, ktn * BN, S, D, lk, smem + par * L::KT,
                                                     smem_addr + 2u * par * L::KT, j);
    };
    {
        const int kt0 = next_key_tile();
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            issue_kv(0, kt0, 0, j);
            issue_kv(1, kt0, 0, j);
        }
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
        const int par = i & 1;
        const char* Kb = reinterpret_cast<const char*>(smem) + par * KTB;  // K tile; V tile at + 2 KTB
        wait_vmcnt<0>();  // see dkdv_fast_body
        lds_barrier();
        // Next key tile's loads (K then V, PER each per thread), spread over
        // the S/dP steps below; the last block re-loads key tile 0 into the
        // idle buffer so that the schedule has no branch (waited for at the end).
        const int ktn = i + 1 < niter ? next_key_tile() : 0;
        const int kbase = (qlo + (int)(g0 + i - qstart)) * BN;
        const int wrow0 = qt * BM + 32 * w, row = wrow0 + n;
        if (wave_uniform(wrow0 < S && vis.any(wrow0, min(wrow0 + 31, S - 1), kbase, kbase + BN - 1))) {
        const bool need_mask = wave_uniform(!vis.all(wrow0, wrow0 + 31, kbase, kbase + BN - 1));
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
            f32x16 s, dp;
            {
                // S^T = K Q^T and dP^T = V dO^T, one chunk of both per step
                struct Ops { bf16x8 k, v; };
                auto aread = [&](int c) {
                    Ops o;
                    o.k = *reinterpret_cast<const bf16x8*>(Kb + ln.row(kk, c));
                    o.v = *reinterpret_cast<const bf16x8*>(Kb + 2 * KTB + ln.row(kk, c));
                    return o;
                };
                Ops ring[PF];
#pragma unroll
                for (int c = 0; c < PF; ++c) ring[c] = aread(c);
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    const Ops o = ring[c % PF];
                    if (c + PF < NC) ring[c % PF] = aread(c + PF);
                    mm_score<ASM>(s, o.k, qf[c], c == 0);
                    mm_score<ASM>(dp, o.v, gf[c], c == 0);
                    if (c < PER) issue_kv(kk, ktn, par ^ 1, c);
                }
#pragma unroll
                for (int j = NC; j < PER; ++j) issue_kv(kk, ktn, par ^ 1, j);
                if constexpr (ASM) mfma_v_drain(s, dp);
            }
            // lane column n = query row; register r = key kbase + 32kk + row_of_reg(r, hh)
#pragma unroll
            for (int q = 0; q < 16; ++q) s[q] = fast_exp2(s[q] * a.scale_log2 - lse2);
            if (need_mask) {
                // visible iff lo <= row_of_reg(r, hh) <= hi; the bounds pass
                // through an asm statement so that the selects stay in the branch
                int hi = vis.hi(row) - kbase - 32 * kk, lo = vis.lo(row) - kbase - 32 * kk;
                asm volatile("" : "+v"(hi), "+v"(lo));
#pragma unroll
                for (int q = 0; q < 16; ++q)
                    s[q] = (row_of_reg(q, hh) > hi || row_of_reg(q, hh) < lo) ? 0.f : s[q];
            }
            bf16x8 db[2];
#pragma unroll
            for (int e = 0; e < 2; ++e)
#pragma unroll
                for (int j = 0; j < 8; ++j) db[e][j] = (bf16)(s[8 * e + j] * (dp[8 * e + j] - dlt));
            {
                // dQ^T += K^T dS^T over the two 16-key halves (e) of this block
                constexpr int NI = 2 * NDT;
                auto tread = [&](int it, int hi) {
                    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_v4i16_t*)(Kb + ln.trn(kk, it / NDT, it % NDT, hi)));
                };
                v4i16 rl[PF], rh[PF];
#pragma unroll
                for (int it = 0; it < PF; ++it) {
                    rl[it] = tread(it, 0);
                    rh[it] = tread(it, 1);
                }
#pragma unroll
                for (int it = 0; it < NI; ++it) {
                    const bf16x8 av = __builtin_bit_cast(
                        bf16x8, __builtin_shufflevector(rl[it % PF], rh[it % PF], 0, 1, 2, 3, 4, 5, 6, 7));
                    if (it + PF < NI) {
                        rl[it % PF] = tread(it + PF, 0);
                        rh[it % PF] = tread(it + PF, 1);
                    }
                    dq[it % NDT] = mfma_bf16(av, db[it / NDT], dq[it % NDT]);
                }
                pin_read_ahead<NI, PF, 2>();
            }
        }
        } else {
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                issue_kv(0, ktn, par ^ 1, j);
                issue_kv(1, ktn, par ^ 1, j);
            }
        }  // active wave
      }
      // End of this unit's part of query tile qt: a tile covered by one unit
      // writes dQ, otherwise slot (unit - first unit of qt).
      const int row0 = qt * BM + 32 * w;
      if constexpr (FAST) {
          // Whole tiles (FAST: D == DP, 16-byte rows, and row0 < S means all
          // 32 rows are): through LDS
          // (store_acc32_staged), the buffer of the segment's last tile is
          // idle (the next tile streams into the other); waves 0 and 1 stage
          // in its K tile, waves 2 and 3 in its V tile.
          lds_barrier();
          if (wave_uniform(row0 < S)) {
              float* dqp = a.dq + op_base<STRIDED>(a.sdq, b, h, a.Hq, S, D) + (int64_t)row0 * op_ld<STRIDED>(a.sdq, D);
              int64_t ldq = op_ld<STRIDED>(a.sdq, D);
              if (tile_units(tiles, a.q_us, qt) > 1) {
                  const int64_t slot = (int64_t)(b * a.Hq + h) * 2 * a.q_us.units + 2 * unit + (first ? 0 : 1);
                  dqp = a.q_part + (slot * BM + 32 * w) * D;
                  ldq = D;
              }
              constexpr int SB = KTB / 2;  // staging bytes per wave
              char* stage = reinterpret_cast<char*>(smem) + (((i - 1) & 1) + 2 * (w >> 1)) * KTB + (w & 1) * SB;
              store_acc32_staged<NDT, SB / 4096 < NDT ? SB / 4096 : NDT>(stage, dqp, ldq, dq, a.scale);
          }
      } else if (row0 + n < S) {
          float* dqp = a.dq + op_base<STRIDED>(a.sdq, b, h, a.Hq, S, D) + (int64_t)(row0 + n) * op_ld<STRIDED>(a.sdq, D);
          if (tile_units(tiles, a.q_us, qt) > 1) {
              const int64_t slot = (int64_t)(b * a.Hq + h) * 2 * a.q_us.units + 2 * unit + (first ? 0 : 1);
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
    dkdv_fast_body<DP, CAUSAL, STRIDED, false>(a, smem, i / bh, (i % bh) / a.Hkv, (i % bh) % a.Hkv);
}

template <int DP, bool CAUSAL, bool STRIDED>
__global__ __launch_bounds__(256) void attn_bwd_dq_bf16_fast(BwdArgs a) {
    __shared__ __attribute__((aligned(1024))) bf16 smem[BwdFastLds<DP>::Q_ELEMS];
    const int bh = a.B * a.Hq, i = (int)blockIdx.x;
    dq_fast_body<DP, CAUSAL, STRIDED, false>(a, smem, i / bh, (i % bh) / a.Hq, (i % bh) % a.Hq);
}

// Both roles in one grid: the first kv_us.units * B * Hkv workgroups run dK/dV
// units, the rest dQ units (the units of both are sized to take about equally
// long, see plan_bwd_fast).  Block ids are renumbered XCD-major (xcd_block):
// units with neighbouring ids, which read the same K/V tiles (the group's
// query heads' units of one index) or the same query blocks, then share one
// XCD's L2.  FAST: every operand tile is whole (D == DP and S
// a multiple of 64), so the direct loads take TileDma's precomputed offsets.
template <int DP, bool CAUSAL, bool STRIDED, bool FAST>
__global__ __launch_bounds__(256) void attn_bwd_main_bf16_fast(BwdArgs a) {
    __shared__ __attribute__((aligned(1024))) bf16 smem[BwdFastLds<DP>::ELEMS];
    const int nkv = a.kv_us.units * a.B * a.Hkv;
    const int i = xcd_block((int)blockIdx.x, (int)gridDim.x);
    if (i < nkv) {
        const int bh = a.B * a.Hkv;
        dkdv_fast_body<DP, CAUSAL, STRIDED, FAST>(a, smem, i / bh, (i % bh) / a.Hkv, (i % bh) % a.Hkv);
    } else {
        const int j = i - nkv, bh = a.B * a.Hq;
        dq_fast_body<DP, CAUSAL, STRIDED, FAST>(a, smem, j / bh, (j % bh) / a.Hq, (j % bh) % a.Hq);
    }
}

// REDUCE: sum the partial slots of every split tile in unit order.  One
// workgroup per (batch, head, 128-row tile, group of merge_rows(D) rows) of
// the dK/dV role (rows = keys; dK and dV) and then of the dQ role (rows =
// queries); workgroups of unsplit tiles return at once.
constexpr int kRedMaxSlots = kSplitMaxSlots, kRedBatch = 4;

// dst row r (r < rows, row stride ld) = sum over the slots, in slot order, of
// row row0 + r of the slot tiles (rows <= RW = merge_rows(D)).  256 / RW
// threads share a row: thread t sums its row's 16-byte chunks
// t % (256 / RW) + (256 / RW) j (j < 4), kRedBatch slots' loads in flight
// together.
__device__ __forceinline__ void reduce_rows(const float* part, const int64_t* slot_of, int nsl, int64_t tile_elems,
                                            int row0, int rows, int D, float* dst, int64_t ld) {
    constexpr int MAXJ = 4;
    const int tpr = 256 / merge_rows(D), r = (int)threadIdx.x / tpr, cl = (int)threadIdx.x % tpr, cg = D / 4;
    if (r >= rows) return;
    f32x4 acc[MAXJ];
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int p0 = 0; p0 < nsl; p0 += kRedBatch) {
        f32x4 x[kRedBatch][MAXJ];
#pragma unroll
        for (int q = 0; q < kRedBatch; ++q) {
            if (p0 + q >= nsl) break;
            const float* src = part + slot_of[p0 + q] * tile_elems + (int64_t)(row0 + r) * D;
#pragma unroll
            for (int j = 0; j < MAXJ; ++j) {
                const int c = cl + tpr * j;
                x[q][j] = c < cg ? *reinterpret_cast<const f32x4*>(src + 4 * c) : f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
#pragma unroll
        for (int q = 0; q < kRedBatch; ++q) {
            if (p0 + q >= nsl) break;
#pragma unroll
            for (int j = 0; j < MAXJ; ++j) acc[j] += x[q][j];
        }
    }
    float* out = dst + (int64_t)r * ld;
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) {
        const int c = cl + tpr * j;
        if (c < cg) *reinterpret_cast<f32x4*>(out + 4 * c) = acc[j];
    }
}

template <bool CAUSAL>
__global__ __launch_bounds__(256) void attn_bwd_fast_reduce(BwdArgs a) {
    __shared__ int64_t slot_of[kRedMaxSlots];
    const int S = a.S, D = a.D, nt = (S + 127) / 128, RW = merge_rows(D), RG = 128 / RW;
    const int64_t kv_blocks = (int64_t)a.B * a.Hkv * nt * RG;
    int64_t blk = blockIdx.x;
    const bool kv = blk < kv_blocks;
    if (!kv) blk -= kv_blocks;
    const int rg = (int)(blk % RG), t = (int)((blk / RG) % nt), bh = (int)(blk / (RG * nt));
    const FastTiles tiles{S, CAUSAL, a.window, a.group, kv ? 1 : 0};
    const UnitSplit us = kv ? a.kv_us : a.q_us;
    int u0;
    const int nsl = tile_units(tiles, us, t, &u0);
    const int r0 = t * 128 + rg * RW;
    if (nsl <= 1 || r0 >= S) return;
    const bool starts = unit_first(tiles, us, u0) == tiles.start(t);
    const int64_t head_slots = (int64_t)bh * 2 * us.units;
    if ((int)threadIdx.x < nsl) slot_of[threadIdx.x] = head_slots + split_slot(u0 + threadIdx.x, u0, starts);
    __syncthreads();
    const int rows = min(RW, S - r0), rit = rg * RW;  // rows, first row inside the tile
    if (kv) {
        // slot layout [dK rows 0..127][dV rows 0..127]
        const int bb = bh / a.Hkv, hk = bh % a.Hkv;
        reduce_rows(a.kv_part, slot_of, nsl, 2 * 128 * (int64_t)D, rit, rows, D,
                    a.dk + a.sdk.at(bb, hk) + (int64_t)r0 * a.sdk.s, a.sdk.s);
        reduce_rows(a.kv_part, slot_of, nsl, 2 * 128 * (int64_t)D, 128 + rit, rows, D,
                    a.dv + a.sdv.at(bb, hk) + (int64_t)r0 * a.sdv.s, a.sdv.s);
    } else {
        const int bb = bh / a.Hq, h = bh % a.Hq;
        reduce_rows(a.q_part, slot_of, nsl, 128 * (int64_t)D, rit, rows, D,
                    a.dq + a.sdq.at(bb, h) + (int64_t)r0 * a.sdq.s, a.sdq.s);
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
        const dim3 grid((unsigned)(a.kv_us.units * s.B * s.Hkv + a.q_us.units * s.B * s.Hq));
        if (s.D == DP && s.S % 64 == 0) {
#define MFT_MAIN_FAST(CAUSAL, STRIDED, FAST) \
    hipLaunchKernelGGL((attn_bwd_main_bf16_fast<DP, CAUSAL, STRIDED, FAST>), grid, dim3(256), 0, st, a)
            if (s.causal && strided)
                MFT_MAIN_FAST(true, true, true);
            else if (s.causal)
                MFT_MAIN_FAST(true, false, true);
            else if (strided)
                MFT_MAIN_FAST(false, true, true);
            else
                MFT_MAIN_FAST(false, false, true);
        } else {
            if (s.causal && strided)
                MFT_MAIN_FAST(true, true, false);
            else if (s.causal)
                MFT_MAIN_FAST(true, false, false);
            else if (strided)
                MFT_MAIN_FAST(false, true, false);
            else
                MFT_MAIN_FAST(false, false, false);
#undef MFT_MAIN_FAST
        }
    } else if (stages & BWD_STAGE_DKDV) {
        MFT_BWD_LAUNCH(attn_bwd_dkdv_bf16_fast, dim3((unsigned)(a.kv_us.units * s.B * s.Hkv)));
    } else if (stages & BWD_STAGE_DQ) {
        MFT_BWD_LAUNCH(attn_bwd_dq_bf16_fast, dim3((unsigned)(a.q_us.units * s.B * s.Hq)));
    }
#undef MFT_BWD_LAUNCH
    if ((stages & BWD_STAGE_REDUCE) && (a.kv_parts_max > 1 || a.q_parts_max > 1)) {
        const int64_t nt = (s.S + 127) / 128;
        const int64_t blocks = (s.B * s.Hkv + s.B * s.Hq) * nt * (128 / merge_rows(s.D));
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
