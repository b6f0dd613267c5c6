// Fused causal GQA attention backward for gfx950.
//
// Replaces Engine::run_backward over the composite's nodes
// (core/autograd_engine.cpp:144-273): MatmulBackward for P.V and Q.K^T
// (core/backward_functions.cpp:94-147), SoftmaxBackward (:306-349),
// ScaleBackward (:981-985), AddBackward (:36-72), TransposeBackward
// (:422-426) and RepeatKVHeadsBackward (:693-726).  Nothing of size S x S is
// read: P is recomputed from the saved row log-sum-exp, and the softmax row
// term sum_j dP_ij P_ij is computed as delta_i = dO_i . O_i (equal in exact
// arithmetic; the reference forms it in double from dP and P).
//
// Stages (each a launch; mft_attn_bwd runs all three in order):
//   DELTA  : delta[b,h,i] = sum_d dO[i,d] * O[i,d]                  (HBM bound)
//   MAIN   : one launch holding two kinds of workgroup (bf16; fp32 uses two
//            launches of the same bodies):
//     dK/dV role — one workgroup per (32*NW keys, kv head, head-group split);
//       wave w owns 32 keys, one key per lane column.  It loops over the
//       query heads of its group and over 32-row query blocks (causal: from
//       its first key on), recomputing S = Q K^T and dP = dO V^T with keys
//       along the accumulator columns, and accumulates
//         dV^T += dO^T P,   dK^T += Q^T dS
//       in registers.  GQA: the group's heads sum in registers, so dK/dV come
//       out already reduced over repeat_kv (no atomics).
//     dQ role — one workgroup per (32*NW query rows, query head): recomputes
//       S^T and dP^T with one query row per lane (like the forward) and
//       accumulates dQ^T += K^T dS^T.  No atomics; deterministic.
//     The two roles are independent (both only need delta), so running them
//     in one grid fills the 256 CUs even when B*Hkv is 1.  Blocks alternate
//     between roles, heaviest causal tiles first.
//   REDUCE : when a group is split across workgroups for parallelism, each
//            split wrote fp32 dK/dV partials; sum them in split order.
// bf16 inputs use v_mfma_f32_32x32x16_bf16 with fp32 accumulation; operands
// that must be read along the reduction dimension are staged transposed in
// LDS.  fp32 inputs use v_mfma_f32_32x32x2_f32 and need no transposes.
#include "attn_bwd_common.h"

#include <algorithm>
#include <atomic>

namespace mft {
namespace {
using namespace bwd;

// Row terms of a query row for the P recompute, in log2 units:
// P = exp2(x * lc - t0 - t1).  Plain: x is the raw dot product, lc =
// scale * log2(e), t0 = lse * log2(e), t1 = 0.  Mask mode: x is the
// mask_score (natural units), lc = log2(e), (t0, t1) = (row max, ln sum) *
// log2(e) from the forward's lse pair; x * lc - t0 is exactly 0 at the row
// max, so a uniform row (all scores equal and huge) still gets P = 1 / n.
template <bool MASK>
__device__ __forceinline__ void row_terms(const float* lse, int64_t ri, bool valid, float* t0, float* t1) {
    if constexpr (MASK) {
        *t0 = valid ? lse[2 * ri] * kLog2e : INFINITY;
        *t1 = valid ? lse[2 * ri + 1] * kLog2e : 0.f;
    } else {
        *t0 = valid ? lse[ri] * kLog2e : INFINITY;
        *t1 = 0.f;
    }
}

// ------------------------------------------------------------------ DELTA
template <typename T, int DP>
__global__ __launch_bounds__(256) void attn_bwd_delta_kernel(BwdArgs a) {
    typedef typename Elt<T>::vec V;
    constexpr int VEC = Elt<T>::VEC;
    constexpr int TPR = DP / VEC;  // threads per row, a power of two <= 64
    constexpr int RPB = 256 / TPR;
    const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
    const int c = threadIdx.x % TPR;
    float acc = 0.f;
    if (row < a.total_rows) {
        const int64_t bh = row / a.S, i = row % a.S;
        const int bb = (int)(bh / a.Hq), hq = (int)(bh % a.Hq);
        const T* o = (const T*)a.o + a.so.at(bb, hq) + i * a.so.s;
        const T* g = (const T*)a.dO + a.sdo.at(bb, hq) + i * a.sdo.s;
        const V x = load_chunk<T>(o, c * VEC, a.D, true, a.vec_ok != 0);
        const V y = load_chunk<T>(g, c * VEC, a.D, true, a.vec_ok != 0);
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc += (float)x[i] * (float)y[i];
    }
#pragma unroll
    for (int off = TPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (row < a.total_rows && c == 0) a.delta[row] = acc;
}

// ------------------------------------------------------- dK/dV role (bf16)
template <int DP> struct DkdvBf16Lds {
    static constexpr int QSTR = DP + 8;  // row-major 32-row tiles of Q and dO
    static constexpr int TSTR = 32 + 4;  // transposed tiles Q^T, dO^T: [DP][32 + 4]
    static constexpr int BYTES = 2 * (2 * 32 * QSTR + 2 * DP * TSTR) + 3 * 32 * 4;  // + row terms
};

template <int DP, int NW, bool CAUSAL, bool MASK>
__device__ __forceinline__ void dkdv_bf16_body(const BwdArgs& a, char* smem, int kt, int ysplit, int b) {
    typedef DkdvBf16Lds<DP> L;
    constexpr int NC = DP / 16, NDT = DP / 32, NT = NW * 64, BNK = 32 * NW;
    constexpr int QSTR = L::QSTR, TSTR = L::TSTR;
    bf16* Qs = reinterpret_cast<bf16*>(smem);
    bf16* Gs = Qs + 32 * QSTR;
    bf16* Qt = Gs + 32 * QSTR;
    bf16* Gt = Qt + DP * TSTR;
    float* Ls = reinterpret_cast<float*>(Gt + DP * TSTR);
    float* Dl = Ls + 32;
    float* L1 = Dl + 32;  // second row term (mask mode)

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 31, hh = lane >> 5;
    const int S = a.S, D = a.D;
    const bool vec_ok = a.vec_ok != 0;
    const int j0 = kt * BNK;
    const int hk = ysplit / a.splits, split = ysplit % a.splits;
    const int h_begin = hk * a.group + split * a.heads_per_split;
    const int h_end = min(h_begin + a.heads_per_split, (hk + 1) * a.group);
    const int wkey0 = j0 + 32 * w;
    const int key = wkey0 + n;
    const int keyc = key < S ? key : S - 1;

    const bf16* K = (const bf16*)a.k + a.sk.at(b, hk);
    const bf16* Vg = (const bf16*)a.v + a.sv.at(b, hk);
    bf16x8 kf[NC], vf[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        kf[c] = load_chunk<bf16>(K + (int64_t)keyc * a.sk.s, 16 * c + 8 * hh, D, key < S, vec_ok);
        vf[c] = load_chunk<bf16>(Vg + (int64_t)keyc * a.sv.s, 16 * c + 8 * hh, D, key < S, vec_ok);
    }
    f32x16 dk[NDT], dv[NDT];
#pragma unroll
    for (int i = 0; i < NDT; ++i) {
        dk[i] = zero16();
        dv[i] = zero16();
    }

    const KeyVis vis = key_vis(a, b, CAUSAL);
    // Causal: rows from the first key on; window: up to the last key + W - 1.
    const int qstart = CAUSAL ? j0 : 0;
    const int qend = (CAUSAL && a.window > 0) ? min(S, j0 + BNK - 1 + a.window) : S;
    for (int h = h_begin; h < h_end; ++h) {
        const bf16* Q = (const bf16*)a.q + a.sq.at(b, h);
        const bf16* G = (const bf16*)a.dO + a.sdo.at(b, h);
        const float* lse = a.lse + (int64_t)(b * a.Hq + h) * S * (MASK ? 2 : 1);
        const float* dl = a.delta + (int64_t)(b * a.Hq + h) * S;
        for (int qb = qstart; qb < qend; qb += 32) {
            __syncthreads();
            {   // stage 32 query rows: row-major and transposed (4 rows x 8 columns per item)
                constexpr int DG = DP / 8;
                for (int idx = tid; idx < 8 * DG; idx += NT) {
                    const int rg = idx / DG, c = idx - rg * DG;
                    bf16x8 xq[4], xg[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int r = qb + 4 * rg + i;
                        const int rc = r < S ? r : S - 1;
                        xq[i] = load_chunk<bf16>(Q + (int64_t)rc * a.sq.s, 8 * c, D, r < S, vec_ok);
                        xg[i] = load_chunk<bf16>(G + (int64_t)rc * a.sdo.s, 8 * c, D, r < S, vec_ok);
                        *reinterpret_cast<bf16x8*>(Qs + (4 * rg + i) * QSTR + 8 * c) = xq[i];
                        *reinterpret_cast<bf16x8*>(Gs + (4 * rg + i) * QSTR + 8 * c) = xg[i];
                    }
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const bf16x4 tq = {xq[0][j], xq[1][j], xq[2][j], xq[3][j]};
                        const bf16x4 tg = {xg[0][j], xg[1][j], xg[2][j], xg[3][j]};
                        *reinterpret_cast<bf16x4*>(Qt + (8 * c + j) * TSTR + 4 * rg) = tq;
                        *reinterpret_cast<bf16x4*>(Gt + (8 * c + j) * TSTR + 4 * rg) = tg;
                    }
                }
                if (tid < 32) {
                    const int r = qb + tid;
                    row_terms<MASK>(lse, r, r < S, &Ls[tid], &L1[tid]);
                    Dl[tid] = r < S ? dl[r] : 0.f;
                }
            }
            __syncthreads();
            if (wkey0 >= S) continue;  // no valid keys in this wave
            // no row of the block sees a key of this wave
            if (!vis.any(qb, min(qb + 31, S - 1), wkey0, min(wkey0 + 31, S - 1))) continue;

            f32x16 s, dp;
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const bf16x8 qa = *reinterpret_cast<const bf16x8*>(Qs + n * QSTR + 16 * c + 8 * hh);
                const bf16x8 ga = *reinterpret_cast<const bf16x8*>(Gs + n * QSTR + 16 * c + 8 * hh);
                if (c == 0) {
                    mfma_chunk_first<true>(s, qa, kf[c]);
                    mfma_chunk_first<true>(dp, ga, vf[c]);
                } else {
                    s = mfma_bf16(qa, kf[c], s);
                    dp = mfma_bf16(ga, vf[c], dp);
                }
            }
            // lane column n = key; register r = query qb + row_of_reg(r, hh)
            const bool need_mask = !vis.all(qb, qb + 31, wkey0, wkey0 + 31);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 l4 = *reinterpret_cast<const f32x4*>(Ls + 8 * g + 4 * hh);
                const f32x4 d4 = *reinterpret_cast<const f32x4*>(Dl + 8 * g + 4 * hh);
                const f32x4 e4 = MASK ? *reinterpret_cast<const f32x4*>(L1 + 8 * g + 4 * hh) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = 4 * g + i;
                    float p;
                    if constexpr (MASK) {
                        const int qr = qb + 8 * g + 4 * hh + i;
                        const float x = qr < S && key < S
                                            ? mask_score(s[r], a.scale, a.mask_causal, a.m0, a.m1, b, h, qr, key)
                                            : -INFINITY;
                        p = fast_exp2((x * kLog2e - l4[i]) - e4[i]);
                    } else {
                        p = fast_exp2(s[r] * a.scale_log2 - l4[i]);
                        if (need_mask && !vis.visible(qb + 8 * g + 4 * hh + i, key)) p = 0.f;
                    }
                    dp[r] = p * (dp[r] - d4[i]);
                    s[r] = p;
                }
            }
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                bf16x8 pb, db;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    pb[j] = (bf16)s[8 * e + j];
                    db[j] = (bf16)dp[8 * e + j];
                }
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
                    const bf16* gp = Gt + (32 * dt + n) * TSTR + 16 * e + 4 * hh;
                    const bf16x4 glo = *reinterpret_cast<const bf16x4*>(gp);
                    const bf16x4 ghi = *reinterpret_cast<const bf16x4*>(gp + 8);
                    const bf16x8 ga = {glo[0], glo[1], glo[2], glo[3], ghi[0], ghi[1], ghi[2], ghi[3]};
                    dv[dt] = mfma_bf16(ga, pb, dv[dt]);
                    const bf16* qp = Qt + (32 * dt + n) * TSTR + 16 * e + 4 * hh;
                    const bf16x4 qlo = *reinterpret_cast<const bf16x4*>(qp);
                    const bf16x4 qhi = *reinterpret_cast<const bf16x4*>(qp + 8);
                    const bf16x8 qa = {qlo[0], qlo[1], qlo[2], qlo[3], qhi[0], qhi[1], qhi[2], qhi[3]};
                    dk[dt] = mfma_bf16(qa, db, dk[dt]);
                }
            }
        }
    }
    if (key >= S) return;
    float *dkp, *dvp;
    dkdv_out_rows(a, b, hk, split, key, &dkp, &dvp);
    store_dkdv<NDT>(a, dkp, dvp, hh, dk, dv);
}

// ------------------------------------------------------- dK/dV role (fp32)
template <int DP, int NW> struct DkdvF32Lds {
    static constexpr int STR = DP + 4;
    static constexpr int BYTES = 4 * (2 * 32 * NW * STR + 2 * 32 * STR + 96);
};

template <int DP, int NW, bool CAUSAL, bool MASK>
__device__ __forceinline__ void dkdv_f32_body(const BwdArgs& a, char* smem, int kt, int ysplit, int b) {
    constexpr int NC = DP / 8, NDT = DP / 32, NT = NW * 64, BNK = 32 * NW;
    constexpr int STR = DkdvF32Lds<DP, NW>::STR;
    float* Ks = reinterpret_cast<float*>(smem);
    float* Vs = Ks + BNK * STR;
    float* Qs = Vs + BNK * STR;
    float* Gs = Qs + 32 * STR;
    float* Ls = Gs + 32 * STR;
    float* Dl = Ls + 32;
    float* L1 = Dl + 32;  // second row term (mask mode)

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 31, hh = lane >> 5;
    const int S = a.S, D = a.D;
    const bool vec_ok = a.vec_ok != 0;
    const int j0 = kt * BNK;
    const int hk = ysplit / a.splits, split = ysplit % a.splits;
    const int h_begin = hk * a.group + split * a.heads_per_split;
    const int h_end = min(h_begin + a.heads_per_split, (hk + 1) * a.group);
    const int wkey0 = j0 + 32 * w;
    const int key = wkey0 + n;

    const float* K = (const float*)a.k + a.sk.at(b, hk);
    const float* Vg = (const float*)a.v + a.sv.at(b, hk);
    {
        constexpr int CPR = DP / 4;
        for (int idx = tid; idx < BNK * CPR; idx += NT) {
            const int rr = idx / CPR, c = idx - rr * CPR;
            const int kr = j0 + rr, krc = kr < S ? kr : S - 1;
            *reinterpret_cast<f32x4*>(Ks + rr * STR + 4 * c) =
                load_chunk<float>(K + (int64_t)krc * a.sk.s, 4 * c, D, kr < S, vec_ok);
            *reinterpret_cast<f32x4*>(Vs + rr * STR + 4 * c) =
                load_chunk<float>(Vg + (int64_t)krc * a.sv.s, 4 * c, D, kr < S, vec_ok);
        }
    }
    f32x16 dk[NDT], dv[NDT];
#pragma unroll
    for (int i = 0; i < NDT; ++i) {
        dk[i] = zero16();
        dv[i] = zero16();
    }
    const float* Kw = Ks + (32 * w + n) * STR;
    const float* Vw = Vs + (32 * w + n) * STR;

    const KeyVis vis = key_vis(a, b, CAUSAL);
    const int qstart = CAUSAL ? j0 : 0;
    const int qend = (CAUSAL && a.window > 0) ? min(S, j0 + BNK - 1 + a.window) : S;
    for (int h = h_begin; h < h_end; ++h) {
        const float* Q = (const float*)a.q + a.sq.at(b, h);
        const float* G = (const float*)a.dO + a.sdo.at(b, h);
        const float* lse = a.lse + (int64_t)(b * a.Hq + h) * S * (MASK ? 2 : 1);
        const float* dl = a.delta + (int64_t)(b * a.Hq + h) * S;
        for (int qb = qstart; qb < qend; qb += 32) {
            __syncthreads();
            {
                constexpr int CPR = DP / 4;
                for (int idx = tid; idx < 32 * CPR; idx += NT) {
                    const int rr = idx / CPR, c = idx - rr * CPR;
                    const int r = qb + rr, rc = r < S ? r : S - 1;
                    *reinterpret_cast<f32x4*>(Qs + rr * STR + 4 * c) =
                        load_chunk<float>(Q + (int64_t)rc * a.sq.s, 4 * c, D, r < S, vec_ok);
                    *reinterpret_cast<f32x4*>(Gs + rr * STR + 4 * c) =
                        load_chunk<float>(G + (int64_t)rc * a.sdo.s, 4 * c, D, r < S, vec_ok);
                }
                if (tid < 32) {
                    const int r = qb + tid;
                    row_terms<MASK>(lse, r, r < S, &Ls[tid], &L1[tid]);
                    Dl[tid] = r < S ? dl[r] : 0.f;
                }
            }
            __syncthreads();
            if (wkey0 >= S) continue;
            if (!vis.any(qb, min(qb + 31, S - 1), wkey0, min(wkey0 + 31, S - 1))) continue;

            f32x16 s, dp;
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const f32x4 qa = *reinterpret_cast<const f32x4*>(Qs + n * STR + 8 * c + 4 * hh);
                const f32x4 kb = *reinterpret_cast<const f32x4*>(Kw + 8 * c + 4 * hh);
                const f32x4 ga = *reinterpret_cast<const f32x4*>(Gs + n * STR + 8 * c + 4 * hh);
                const f32x4 vb = *reinterpret_cast<const f32x4*>(Vw + 8 * c + 4 * hh);
                if (c == 0) {
                    mfma_chunk_first<true>(s, qa, kb);
                    mfma_chunk_first<true>(dp, ga, vb);
                } else {
                    s = mfma_chunk(qa, kb, s);
                    dp = mfma_chunk(ga, vb, dp);
                }
            }
            const bool need_mask = !vis.all(qb, qb + 31, wkey0, wkey0 + 31);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 l4 = *reinterpret_cast<const f32x4*>(Ls + 8 * g + 4 * hh);
                const f32x4 d4 = *reinterpret_cast<const f32x4*>(Dl + 8 * g + 4 * hh);
                const f32x4 e4 = MASK ? *reinterpret_cast<const f32x4*>(L1 + 8 * g + 4 * hh) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = 4 * g + i;
                    float p;
                    if constexpr (MASK) {
                        const int qr = qb + 8 * g + 4 * hh + i;
                        const float x = qr < S && key < S
                                            ? mask_score(s[r], a.scale, a.mask_causal, a.m0, a.m1, b, h, qr, key)
                                            : -INFINITY;
                        p = fast_exp2((x * kLog2e - l4[i]) - e4[i]);
                    } else {
                        p = fast_exp2(s[r] * a.scale_log2 - l4[i]);
                        if (need_mask && !vis.visible(qb + 8 * g + 4 * hh + i, key)) p = 0.f;
                    }
                    dp[r] = p * (dp[r] - d4[i]);
                    s[r] = p;
                }
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int ql = row_of_reg(r, hh);
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
                    dv[dt] = mfma_f32(Gs[ql * STR + 32 * dt + n], s[r], dv[dt]);
                    dk[dt] = mfma_f32(Qs[ql * STR + 32 * dt + n], dp[r], dk[dt]);
                }
            }
        }
    }
    if (key >= S) return;
    float *dkp, *dvp;
    dkdv_out_rows(a, b, hk, split, key, &dkp, &dvp);
    store_dkdv<NDT>(a, dkp, dvp, hh, dk, dv);
}

// ------------------------------------------------------------- dQ role
template <typename T, int DP, int BN> struct DqLds {
    static constexpr bool KT = sizeof(T) == 2;  // K^T staged (bf16)
    static constexpr int STR = DP + Elt<T>::VEC;
    static constexpr int TSTR = BN + 4;
    static constexpr int KV_ELEMS = BN * STR;
    static constexpr int KT_ELEMS = KT ? DP * TSTR : 0;
    static constexpr int BYTES = (int)sizeof(T) * (2 * KV_ELEMS + KT_ELEMS);
};

template <typename T, int DP, int NW, int BN, bool CAUSAL, bool MASK>
__device__ __forceinline__ void dq_body(const BwdArgs& a, char* smem, int qt, int h, int b) {
    typedef typename Elt<T>::vec V;
    typedef DqLds<T, DP, BN> L;
    constexpr int VEC = Elt<T>::VEC;
    constexpr int NC = DP / (2 * VEC);
    constexpr int NDT = DP / 32, NKK = BN / 32, BM = 32 * NW, NT = NW * 64;
    T* Ks = reinterpret_cast<T*>(smem);
    T* Vs = Ks + L::KV_ELEMS;
    T* Kt = Vs + L::KV_ELEMS;

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 31, hh = lane >> 5;
    const int S = a.S, D = a.D;
    const bool vec_ok = a.vec_ok != 0;
    const int hk = h / a.group;
    const int m0 = qt * BM, wrow0 = m0 + 32 * w, row = wrow0 + n;
    const int rowc = row < S ? row : S - 1;

    const T* Q = (const T*)a.q + a.sq.at(b, h);
    const T* G = (const T*)a.dO + a.sdo.at(b, h);
    const T* K = (const T*)a.k + a.sk.at(b, hk);
    const T* Vg = (const T*)a.v + a.sv.at(b, hk);
    // fp32 at D > 128: this lane's dO row is re-read (L1/L2) per key tile
    // instead of held in 128 more registers, which would spill most of the
    // kernel's state.
    constexpr bool GF_REG = !(sizeof(T) == 4 && DP > 128);
    const T* grow = G + (int64_t)rowc * a.sdo.s;
    V qf[NC], gf[GF_REG ? NC : 1];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        qf[c] = load_chunk<T>(Q + (int64_t)rowc * a.sq.s, 2 * VEC * c + VEC * hh, D, row < S, vec_ok);
        if constexpr (GF_REG) gf[c] = load_chunk<T>(grow, 2 * VEC * c + VEC * hh, D, row < S, vec_ok);
    }
    const int64_t rbase = (int64_t)(b * a.Hq + h) * S;
    float lse2, lse2b;
    row_terms<MASK>(a.lse, rbase + row, row < S, &lse2, &lse2b);
    const float dlt = row < S ? a.delta[rbase + row] : 0.f;

    f32x16 dq[NDT];
#pragma unroll
    for (int i = 0; i < NDT; ++i) dq[i] = zero16();

    const KeyVis vis = key_vis(a, b, CAUSAL);
    const int kend = CAUSAL ? min(S, m0 + BM) : S;
    const int ntiles = (kend + BN - 1) / BN;
    const int t0 = (CAUSAL && a.window > 0) ? max(0, m0 - a.window + 1) / BN : 0;
    for (int t = t0; t < ntiles; ++t) {
        const int kbase = t * BN;
        __syncthreads();
        {
            constexpr int CPR = DP / VEC;
            for (int idx = tid; idx < BN * CPR; idx += NT) {
                const int rr = idx / CPR, c = idx - rr * CPR;
                const int kr = kbase + rr, krc = kr < S ? kr : S - 1;
                *reinterpret_cast<V*>(Ks + rr * L::STR + c * VEC) =
                    load_chunk<T>(K + (int64_t)krc * a.sk.s, c * VEC, D, kr < S, vec_ok);
                *reinterpret_cast<V*>(Vs + rr * L::STR + c * VEC) =
                    load_chunk<T>(Vg + (int64_t)krc * a.sv.s, c * VEC, D, kr < S, vec_ok);
            }
        }
        if constexpr (L::KT) {
            constexpr int DG = DP / 8;
            for (int idx = tid; idx < (BN / 4) * DG; idx += NT) {
                const int kg = idx / DG, c = idx - kg * DG;
                bf16x8 x[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int kr = kbase + 4 * kg + i, krc = kr < S ? kr : S - 1;
                    x[i] = load_chunk<bf16>((const bf16*)K + (int64_t)krc * a.sk.s, 8 * c, D, kr < S, vec_ok);
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const bf16x4 tv = {x[0][j], x[1][j], x[2][j], x[3][j]};
                    *reinterpret_cast<bf16x4*>((bf16*)Kt + (8 * c + j) * L::TSTR + 4 * kg) = tv;
                }
            }
        }
        __syncthreads();
        if (wrow0 >= S || !vis.any(wrow0, min(wrow0 + 31, S - 1), kbase, kbase + BN - 1)) continue;

        const bool need_mask = !vis.all(wrow0, wrow0 + 31, kbase, kbase + BN - 1);
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
            f32x16 s, dp;
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const V ka = *reinterpret_cast<const V*>(Ks + (32 * kk + n) * L::STR + 2 * VEC * c + VEC * hh);
                const V va = *reinterpret_cast<const V*>(Vs + (32 * kk + n) * L::STR + 2 * VEC * c + VEC * hh);
                V gb;
                if constexpr (GF_REG)
                    gb = gf[c];
                else
                    gb = load_chunk<T>(grow, 2 * VEC * c + VEC * hh, D, row < S, vec_ok);
                if (c == 0) {
                    mfma_chunk_first<true>(s, ka, qf[c]);
                    mfma_chunk_first<true>(dp, va, gb);
                } else {
                    s = mfma_chunk(ka, qf[c], s);
                    dp = mfma_chunk(va, gb, dp);
                }
            }
            // lane column n = query row; register r = key kbase + 32kk + row_of_reg(r, hh)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = kbase + 32 * kk + row_of_reg(r, hh);
                float p;
                if constexpr (MASK) {
                    const float x = row < S && key < S
                                        ? mask_score(s[r], a.scale, a.mask_causal, a.m0, a.m1, b, h, row, key)
                                        : -INFINITY;
                    p = fast_exp2((x * kLog2e - lse2) - lse2b);
                } else {
                    p = fast_exp2(s[r] * a.scale_log2 - lse2);
                    if (need_mask && !vis.visible(row, key)) p = 0.f;
                }
                s[r] = p * (dp[r] - dlt);
            }
            if constexpr (L::KT) {
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    bf16x8 db;
#pragma unroll
                    for (int j = 0; j < 8; ++j) db[j] = (bf16)s[8 * e + j];
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt) {
                        const bf16* kp = (const bf16*)Kt + (32 * dt + n) * L::TSTR + 32 * kk + 16 * e + 4 * hh;
                        const bf16x4 lo = *reinterpret_cast<const bf16x4*>(kp);
                        const bf16x4 hi = *reinterpret_cast<const bf16x4*>(kp + 8);
                        const bf16x8 ka = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                        dq[dt] = mfma_bf16(ka, db, dq[dt]);
                    }
                }
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int kl = 32 * kk + row_of_reg(r, hh);
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt)
                        dq[dt] = mfma_f32((float)Ks[kl * L::STR + 32 * dt + n], s[r], dq[dt]);
                }
            }
        }
    }
    if (row >= S) return;
    float* dqp = a.dq + a.sdq.at(b, h) + (int64_t)row * a.sdq.s;
    const bool v4 = a.vec4_ok != 0;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g)
            store4<float>(dqp, 32 * dt + 8 * g + 4 * hh, D, dq[dt][4 * g] * a.scale,
                          dq[dt][4 * g + 1] * a.scale, dq[dt][4 * g + 2] * a.scale,
                          dq[dt][4 * g + 3] * a.scale, v4);
}

// bf16 (head dims the fast path does not take): one launch per role.
// MASK: mask mode (AttnShape::masked; CAUSAL false, every key).
template <int DP, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_bf16(BwdArgs a) {
    __shared__ __attribute__((aligned(16))) char smem[DkdvBf16Lds<DP>::BYTES];
    const int i = blockIdx.x;
    const int yb = a.Hkv * a.splits * a.B;
    const int t = i / yb, rest = i - t * yb;
    dkdv_bf16_body<DP, 4, CAUSAL, MASK>(a, smem, t, rest % (a.Hkv * a.splits), rest / (a.Hkv * a.splits));
}

template <int DP, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(256) void attn_bwd_dq_bf16(BwdArgs a) {
    __shared__ __attribute__((aligned(16))) char smem[DqLds<bf16, DP, 64>::BYTES];
    const int i = blockIdx.x;
    const int yb = a.Hq * a.B;
    const int ti = i / yb, rest = i - ti * yb;
    dq_body<bf16, DP, 4, 64, CAUSAL, MASK>(a, smem, a.n_qtiles - 1 - ti, rest % a.Hq, rest / a.Hq);
}

// fp32: the roles use different block sizes, so they are two launches.
template <int DP, int NW, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(NW * 64) void attn_bwd_dkdv_f32(BwdArgs a) {
    __shared__ __attribute__((aligned(16))) char smem[DkdvF32Lds<DP, NW>::BYTES];
    const int i = blockIdx.x;
    const int yb = a.Hkv * a.splits * a.B;
    const int t = i / yb, rest = i - t * yb;
    dkdv_f32_body<DP, NW, CAUSAL, MASK>(a, smem, t, rest % (a.Hkv * a.splits), rest / (a.Hkv * a.splits));
}

template <int DP, int BN, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(256) void attn_bwd_dq_f32(BwdArgs a) {
    __shared__ __attribute__((aligned(16))) char smem[DqLds<float, DP, BN>::BYTES];
    const int i = blockIdx.x;
    const int yb = a.Hq * a.B;
    const int ti = i / yb, rest = i - ti * yb;
    dq_body<float, DP, 4, BN, CAUSAL, MASK>(a, smem, a.n_qtiles - 1 - ti, rest % a.Hq, rest / a.Hq);
}


constexpr int f32_dkdv_warps(int DP) { return DP >= 256 ? 1 : DP >= 128 ? 2 : 4; }
constexpr int f32_dq_bn(int DP) { return DP >= 256 ? 32 : 64; }

template <typename T, int DP>
hipError_t launch_bwd_t(const AttnShape& s, BwdArgs a, int stages, hipStream_t st) {
    constexpr bool BF = sizeof(T) == 2;
    if (stages & BWD_STAGE_DELTA) {
        constexpr int TPR = DP / Elt<T>::VEC;
        constexpr int RPB = 256 / TPR;
        const int64_t blocks = (a.total_rows + RPB - 1) / RPB;
        hipLaunchKernelGGL((attn_bwd_delta_kernel<T, DP>), dim3((unsigned)blocks), dim3(256), 0, st, a);
    }
    if (stages & (BWD_STAGE_DKDV | BWD_STAGE_DQ)) {
        constexpr int NW = BF ? 4 : f32_dkdv_warps(DP), BN = BF ? 64 : f32_dq_bn(DP);
        const bool kv = stages & BWD_STAGE_DKDV, q = stages & BWD_STAGE_DQ;
        // (causal, mask mode) -> instantiation; mask mode applies the causal
        // flag per element (mask_score) and visits every key
#define MFT_BWD_ROLES(C, M)                                                                                     \
    do {                                                                                                        \
        if constexpr (BF) {                                                                                     \
            if (kv) hipLaunchKernelGGL((attn_bwd_dkdv_bf16<DP, C, M>), dim3(a.n_kv_blocks), dim3(256), 0, st, a); \
            if (q) hipLaunchKernelGGL((attn_bwd_dq_bf16<DP, C, M>), dim3(a.n_q_blocks), dim3(256), 0, st, a);    \
        } else {                                                                                                \
            if (kv)                                                                                             \
                hipLaunchKernelGGL((attn_bwd_dkdv_f32<DP, NW, C, M>), dim3(a.n_kv_blocks), dim3(NW * 64), 0, st, a); \
            if (q) hipLaunchKernelGGL((attn_bwd_dq_f32<DP, BN, C, M>), dim3(a.n_q_blocks), dim3(256), 0, st, a); \
        }                                                                                                       \
    } while (0)
        if (s.masked)
            MFT_BWD_ROLES(false, true);
        else if (s.causal)
            MFT_BWD_ROLES(true, false);
        else
            MFT_BWD_ROLES(false, false);
#undef MFT_BWD_ROLES
    }
    if ((stages & BWD_STAGE_REDUCE) && a.splits > 1) {
        int64_t blocks = (a.part_stride + 255) / 256;
        if (blocks > 4096) blocks = 4096;
        hipLaunchKernelGGL(attn_bwd_reduce_kernel, dim3((unsigned)blocks), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

template <typename T>
hipError_t launch_bwd_dispatch(const AttnShape& s, const BwdArgs& a, int stages, hipStream_t st) {
    if (bwd_fast_path(s)) {
        if (!s.bf16) return f32::launch_bwd_fast(s, a, stages, st);
        if (s.D <= 64) return launch_bwd_fast_64(s, a, stages, st);
        if (s.D <= 128) return launch_bwd_fast_128(s, a, stages, st);
        return launch_bwd_fast_256(s, a, stages, st);
    }
    if (s.D <= 32) return launch_bwd_t<T, 32>(s, a, stages, st);
    if (s.D <= 64) return launch_bwd_t<T, 64>(s, a, stages, st);
    if (s.D <= 128) return launch_bwd_t<T, 128>(s, a, stages, st);
    return launch_bwd_t<T, 256>(s, a, stages, st);
}

int padded_d(int64_t D) { return D <= 32 ? 32 : D <= 64 ? 64 : D <= 128 ? 128 : 256; }

}  // namespace

// The fast kernels: bf16 (they take K and V with one sequence stride, true
// of contiguous operands, [B, S, Hkv, D] views and fused-QKV slices; other
// layouts run the general kernels) and fp32 (any layout).
bool bwd_fast_path(const AttnShape& s) {
    if (s.masked) return false;  // mask mode: the general kernels
    return (s.bf16 && s.D % 8 == 0 && s.D > 32 && s.k.s == s.v.s) || f32::fast_path(s);
}

// Compute units of the current device (256 on MI355X), cached per device.
int device_cus() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

BwdPlan plan_bwd_fast(const AttnShape& s) {
    BwdPlan p{};
    p.fast = bwd_fast_path(s);
    if (!p.fast) return p;
    const int S = (int)s.S, causal = s.causal ? 1 : 0, group = (int)(s.Hq / s.Hkv), W = s.window;
    const FastTiles gkv{S, causal, W, group, 1}, gq{S, causal, W, group, 0};
    const int64_t pairs_kv = s.B * s.Hkv, pairs_q = s.B * s.Hq;
    const int64_t cus = bwd_unit_slots(s);  // units resident at once
    // Both roles share one launch of about one workgroup per CU, with units
    // of about equal cost (the iteration and tile costs price the two roles'
    // work on one scale).  The unit cost T is the smallest
    // at which every unit fits in one round; fewer, longer units than one
    // launch per role would take also mean fewer fp32 partial tiles for
    // REDUCE.
    const int kvi = kv_iter_cost(s), qi = q_iter_cost(s), kvc = kv_tile_cost(s), qc = q_tile_cost(s);
    const int64_t c_kv = make_unit_split(gkv, 1, kvi, kvc).ctot;  // one (batch, kv head)
    const int64_t c_q = make_unit_split(gq, 1, qi, qc).ctot;  // one (batch, query head)
    const int64_t work = c_kv * pairs_kv + c_q * pairs_q;
    auto units = [&](int64_t T) { return pairs_kv * ((c_kv + T - 1) / T) + pairs_q * ((c_q + T - 1) / T); };
    int64_t T = std::max<int64_t>(1, (work + cus - 1) / cus);
    // Longer units than both whole ranges change nothing; stop there.
    const int64_t T_max = std::max(c_kv, c_q);
    while (T < T_max && units(T) > cus) T += std::max<int64_t>(1, T / 64);
    // Units no shorter than kMinUnitIters iterations, and no tile over
    // kSplitMaxSlots units (REDUCE keeps a tile's slot list in LDS).
    p.kv = fit_unit_split(gkv, (c_kv + T - 1) / T, kvi, kvc, kMinUnitIters, kSplitMaxSlots, &p.kv_parts_max);
    p.q = fit_unit_split(gq, (c_q + T - 1) / T, qi, qc, kMinUnitIters, kSplitMaxSlots, &p.q_parts_max);
    return p;
}

BwdLayout bwd_layout(const AttnShape& s, const BwdPlan& p) {
    auto up = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
    const size_t rows = static_cast<size_t>(s.B * s.Hq);
    const size_t stat_floats = rows * static_cast<size_t>((s.S + 31) / 32) * 64;
    const size_t delta_floats = rows * static_cast<size_t>(s.S);
    const size_t kv_elems = static_cast<size_t>(s.B * s.Hkv * s.S * s.D);
    const size_t q_elems = static_cast<size_t>(s.B * s.Hq * s.S * s.D);
    BwdLayout l;
    l.stats = up(sizeof(float) * std::max(stat_floats, delta_floats));
    if (p.fast) {
        // two slots per unit (split_slot), each one 128-row tile: dK and dV
        // tiles for the dK/dV role, a dQ tile for the dQ role
        const size_t tile = static_cast<size_t>(128 * s.D);
        l.kv_part = p.kv_parts_max > 1 ? up(sizeof(float) * 2 * tile * 2 * p.kv.units * s.B * s.Hkv) : 0;
        l.q_part = p.q_parts_max > 1 ? up(sizeof(float) * tile * 2 * p.q.units * s.B * s.Hq) : 0;
    } else {
        const int splits = dkdv_splits(s);
        l.kv_part = splits > 1 ? up(sizeof(float) * 2 * splits * kv_elems) : 0;
        l.q_part = 0;
    }
    l.masked = masked_rows_workspace_bytes(s);
    l.total = l.stats + l.kv_part + l.q_part + l.masked;
    return l;
}

int dkdv_keys_per_block(const AttnShape& s) {
    if (s.bf16) return 128;
    return 32 * (padded_d(s.D) >= 256 ? 1 : padded_d(s.D) >= 128 ? 2 : 4);
}

int dkdv_splits(const AttnShape& s) {
    // Split the query heads of a group across workgroups until the whole
    // MAIN grid (dK/dV blocks + dQ blocks) has about one workgroup per CU;
    // splits must divide the group size.
    const int64_t group = s.Hq / s.Hkv;
    const int64_t kb = dkdv_keys_per_block(s);
    const int64_t kv_base = ((s.S + kb - 1) / kb) * s.Hkv * s.B;
    const int64_t q_blocks = s.bf16 ? ((s.S + 127) / 128) * s.Hq * s.B : 0;
    int64_t best = 1;
    for (int64_t d = 1; d <= group; ++d) {
        if (group % d) continue;
        best = d;
        if (kv_base * d + q_blocks >= 256) break;
    }
    return (int)best;
}

hipError_t launch_attn_bwd(const AttnShape& s, const BwdPlan& p, const void* q, const void* k, const void* v,
                           const void* o, const void* dO, const float* lse, float* dq, float* dk,
                           float* dv, void* workspace, int stages, hipStream_t st) {
    const BwdLayout lay = bwd_layout(s, p);
    char* ws = static_cast<char*>(workspace);
    float* delta = reinterpret_cast<float*>(ws);
    float* part = lay.kv_part ? reinterpret_cast<float*>(ws + lay.stats) : nullptr;
    BwdArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = o;
    a.dO = dO;
    a.lse = lse;
    a.dq = dq;
    a.dk = dk;
    a.dv = dv;
    a.delta = delta;
    a.stats = delta;  // the fast path lays the same workspace out as row-stat blocks
    a.nqb_total = (int)((s.S + 31) / 32);
    a.part = part;
    a.part_stride = s.B * s.Hkv * s.S * s.D;
    a.total_rows = s.B * s.Hq * s.S;
    a.S = (int)s.S;
    a.D = (int)s.D;
    a.Hq = (int)s.Hq;
    a.Hkv = (int)s.Hkv;
    a.B = (int)s.B;
    a.group = (int)(s.Hq / s.Hkv);
    a.splits = dkdv_splits(s);
    a.heads_per_split = a.group / a.splits;
    const int kb = dkdv_keys_per_block(s);
    a.n_ktiles = (int)((s.S + kb - 1) / kb);
    a.n_qtiles = (int)((s.S + 127) / 128);
    a.n_kv_blocks = a.n_ktiles * a.Hkv * a.splits * a.B;
    a.n_q_blocks = a.n_qtiles * a.Hq * a.B;
    a.scale = s.scale;
    a.scale_log2 = s.scale * kLog2e;
    a.vec_ok = (s.D % (s.bf16 ? 8 : 4)) == 0;
    a.vec4_ok = (s.D % 4) == 0;
    a.causal = s.causal ? 1 : 0;
    a.window = s.window;
    a.kv_len = s.kv_len;
    a.m0 = s.m0;
    a.m1 = s.m1;
    a.mask_causal = s.causal ? 1 : 0;
    a.sq = s.q;
    a.sk = s.k;
    a.sv = s.v;
    a.so = s.o;
    a.sdo = s.dO;
    a.sdq = s.dq;
    a.sdk = s.dk;
    a.sdv = s.dv;
    a.kv_part = part;
    a.q_part = lay.q_part ? reinterpret_cast<float*>(ws + lay.stats + lay.kv_part) : nullptr;
    a.q_part_stride = s.B * s.Hq * s.S * s.D;
    a.kv_us = p.kv;
    a.q_us = p.q;
    a.kv_parts_max = p.kv_parts_max;
    a.q_parts_max = p.q_parts_max;
    const hipError_t e =
        s.bf16 ? launch_bwd_dispatch<bf16>(s, a, stages, st) : launch_bwd_dispatch<float>(s, a, stages, st);
    if (e != hipSuccess || !(stages & BWD_STAGE_REDUCE)) return e;
    return launch_bwd_masked_rows(s, q, k, v, o, dO, dq, dk, dv, ws + lay.stats + lay.kv_part + lay.q_part, st);
}

}  // namespace mft
