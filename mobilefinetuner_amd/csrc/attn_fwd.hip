// Fused causal GQA attention forward for gfx950.
//
// Replaces the reference composite forward (repeat_kv_heads -> transpose ->
// matmul -> mul(scale) -> add(-1e10 causal mask) -> softmax -> matmul;
// core/memory_efficient_attention.cpp:23-43, core/ops.cpp:2260-2335) with one
// kernel that never materialises the S x S scores: an online softmax over key
// tiles, keeping per row the running max and sum, and writing O plus the row
// log-sum-exp that the backward recomputes P from.
//
// Work decomposition: one workgroup = NW waves = 32*NW consecutive query rows
// of one query head; wave w owns rows m0+32w .. m0+32w+31, one row per lane
// column n.  GQA: the workgroup reads kv head h / group directly (no
// repeat_kv copy).  Key tiles of BN rows are staged in LDS by all waves:
//   K  row-major [BN][DP+pad]         (A operand of S^T = K Q^T)
//   V  bf16: transposed [DP][BN+4]    (A operand of O^T += V^T P^T)
//      fp32: row-major [BN][DP+4]
// Q lives in registers as the B operand.  Because S^T is computed (keys along
// the accumulator's rows), each lane holds 16 scores of ONE query row: the
// row max and sum are lane-local plus one swap with the other half-wave, and
// the exp'd scores are the B operand of the P.V MFMA without any shuffle (the
// key order inside a 32-key block is permuted identically in V^T).
// Causal: key tiles beyond the workgroup's last row are never visited and
// query tiles run longest-first.
#include <algorithm>

#include "attn_common.h"
#include "attn_geometry.h"
#include "attn_fwd_fast.h"
#include "attn_kernels.h"

namespace mft {
using fwd::FwdArgs;
using fwd::kFwdBM;
using fwd::kFwdBN;
using fwd::kCombBatch;
using fwd::kCombMaxSlots;
using fwd::launch_fwd_fast64;
using fwd::launch_fwd_fast128;
using fwd::launch_fwd_fast256;
namespace {


template <typename T, int DP, int BN> struct FwdLds {
    static constexpr bool VT = sizeof(T) == 2;  // V staged transposed (bf16)
    static constexpr int KSTR = DP + Elt<T>::VEC;
    static constexpr int VSTR = VT ? BN + 4 : DP + 4;
    static constexpr int K_ELEMS = BN * KSTR;
    static constexpr int V_ELEMS = VT ? DP * VSTR : BN * VSTR;
};

// MASK: mask mode (AttnShape::masked, CAUSAL false): every key, scores from
// mask_score, the running max in natural units, and lse written as the pair
// (row max, ln sum), which keeps the row's sum exact when its scores are
// huge (a row masked by -1e10 everywhere is a uniform softmax).
template <typename T, int DP, int NW, int BN, bool CAUSAL, bool MASK = false>
__global__ __launch_bounds__(NW * 64) void attn_fwd_kernel(FwdArgs a) {
    static_assert(!(MASK && CAUSAL), "mask mode visits every key");
    typedef typename Elt<T>::vec V;
    typedef FwdLds<T, DP, BN> L;
    constexpr int VEC = Elt<T>::VEC;
    constexpr int NC = DP / (2 * VEC);  // d-chunks per dot product (2 halves)
    constexpr int NDT = DP / 32;        // 32-wide column blocks of O^T
    constexpr int NKK = BN / 32;        // 32-key blocks per tile
    constexpr int BM = 32 * NW;
    constexpr int NT = NW * 64;

    __shared__ __attribute__((aligned(16))) T Ks[L::K_ELEMS];
    __shared__ __attribute__((aligned(16))) T Vs[L::V_ELEMS];

    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6, n = lane & 31, hh = lane >> 5;
    const int S = a.S, D = a.D;
    const bool vec_ok = a.vec_ok != 0;
    const int qt = a.n_qtiles - 1 - (int)blockIdx.x;  // longest causal rows first
    const int h = blockIdx.y, b = blockIdx.z, hk = h / a.group;
    const int m0 = qt * BM;
    const int wrow0 = m0 + 32 * w;
    const int row = wrow0 + n;
    const int rowc = row < S ? row : S - 1;

    const T* __restrict__ Q = (const T*)a.q + a.sq.at(b, h);
    const T* __restrict__ K = (const T*)a.k + a.sk.at(b, hk);
    const T* __restrict__ Vg = (const T*)a.v + a.sv.at(b, hk);
    const int lq = a.sq.s, lk = a.sk.s, lv = a.sv.s;

    V qf[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c)
        qf[c] = load_chunk<T>(Q + (int64_t)rowc * lq, 2 * VEC * c + VEC * hh, D, row < S, vec_ok);

    f32x16 oacc[NDT];
#pragma unroll
    for (int i = 0; i < NDT; ++i) oacc[i] = zero16();
    float m_run = -INFINITY;  // running row max, log2-scaled units
    float l_run = 0.f;        // running sum over this half-wave's keys

    const KeyVis vis{S, a.window, a.kv_len ? min(max(a.kv_len[b], 0), S) : S, CAUSAL};
    const int kend = CAUSAL ? min(S, m0 + BM) : S;
    const int ntiles = (kend + BN - 1) / BN;
    // The causal window reaches no key before m0 - W + 1.
    const int t0 = (CAUSAL && a.window > 0) ? max(0, m0 - a.window + 1) / BN : 0;

    for (int t = t0; t < ntiles; ++t) {
        const int kbase = t * BN;
        __syncthreads();
        {   // stage K (row-major)
            constexpr int CPR = DP / VEC;
            for (int idx = tid; idx < BN * CPR; idx += NT) {
                const int rr = idx / CPR, c = idx - rr * CPR;
                const int key = kbase + rr;
                const int keyc = key < S ? key : S - 1;
                *reinterpret_cast<V*>(Ks + rr * L::KSTR + c * VEC) =
                    load_chunk<T>(K + (int64_t)keyc * lk, c * VEC, D, key < S, vec_ok);
            }
        }
        if constexpr (L::VT) {  // stage V transposed: 4 keys x 8 columns per item
            constexpr int DG = DP / 8;
            for (int idx = tid; idx < (BN / 4) * DG; idx += NT) {
                const int kg = idx / DG, c = idx - kg * DG;
                bf16x8 x[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int key = kbase + 4 * kg + i;
                    const int keyc = key < S ? key : S - 1;
                    x[i] = load_chunk<bf16>((const bf16*)Vg + (int64_t)keyc * lv, 8 * c, D, key < S, vec_ok);
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    bf16x4 tv = {x[0][j], x[1][j], x[2][j], x[3][j]};
                    *reinterpret_cast<bf16x4*>((bf16*)Vs + (8 * c + j) * L::VSTR + 4 * kg) = tv;
                }
            }
        } else {
            constexpr int CPR = DP / VEC;
            for (int idx = tid; idx < BN * CPR; idx += NT) {
                const int rr = idx / CPR, c = idx - rr * CPR;
                const int key = kbase + rr;
                const int keyc = key < S ? key : S - 1;
                *reinterpret_cast<V*>(Vs + rr * L::VSTR + c * VEC) =
                    load_chunk<T>(Vg + (int64_t)keyc * lv, c * VEC, D, key < S, vec_ok);
            }
        }
        __syncthreads();

        // A wave with no valid rows, or none of whose rows sees a key of this
        // tile, skips it.
        if (wrow0 >= S || !vis.any(wrow0, min(wrow0 + 31, S - 1), kbase, kbase + BN - 1)) continue;

        f32x16 s[NKK];
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const V ka = *reinterpret_cast<const V*>(Ks + (32 * kk + n) * L::KSTR + 2 * VEC * c + VEC * hh);
                if (c == 0)
                    mfma_chunk_first<false>(s[kk], ka, qf[c]);  // VGPR-form translation unit
                else
                    s[kk] = mfma_chunk(ka, qf[c], s[kk]);
            }
        }

        const bool need_mask = !vis.all(wrow0, wrow0 + 31, kbase, kbase + BN - 1);
        float mx = -INFINITY;
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float x = s[kk][r];
                const int key = kbase + 32 * kk + row_of_reg(r, hh);
                if constexpr (MASK)
                    x = key < S ? mask_score(x, a.scale, a.mask_causal, a.m0, a.m1, b, h, rowc, key) : -INFINITY;
                else if (need_mask && !vis.visible(row, key))
                    x = -INFINITY;
                s[kk][r] = x;
                mx = fmaxf(mx, x);
            }
        }
        mx = half_max(mx);
        // log2 units (MASK: natural units, scaled into the exponent below)
        const float m_new = fmaxf(m_run, MASK ? mx : mx * a.scale_log2);
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = MASK ? fast_exp2((m_run - m_use) * kLog2e) : fast_exp2(m_run - m_use);
        float psum = 0.f;
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = MASK ? fast_exp2((s[kk][r] - m_use) * kLog2e)
                                     : fast_exp2(s[kk][r] * a.scale_log2 - m_use);
                s[kk][r] = p;
                psum += p;
            }
        }
        l_run = l_run * alpha + psum;
        m_run = m_new;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;

        // O^T[d][row] += sum_key V^T[d][key] P^T[key][row]
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
            if constexpr (L::VT) {
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    bf16x8 pb;
#pragma unroll
                    for (int j = 0; j < 8; ++j) pb[j] = (bf16)s[kk][8 * e + j];
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt) {
                        const bf16* vp = (const bf16*)Vs + (32 * dt + n) * L::VSTR + 32 * kk + 16 * e + 4 * hh;
                        const bf16x4 lo = *reinterpret_cast<const bf16x4*>(vp);
                        const bf16x4 hi = *reinterpret_cast<const bf16x4*>(vp + 8);
                        const bf16x8 va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                        oacc[dt] = mfma_bf16(va, pb, oacc[dt]);
                    }
                }
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int kl = 32 * kk + row_of_reg(r, hh);
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt)
                        oacc[dt] = mfma_f32((float)Vs[kl * L::VSTR + 32 * dt + n], s[kk][r], oacc[dt]);
                }
            }
        }
    }

    if (wrow0 >= S) return;
    const float l_tot = half_sum(l_run);
    if (row >= S) return;
    // A row that sees no key at all (key padding) gets O = 0 and LSE = +inf
    // here; attn_fwd_masked_rows then writes the reference's output for it.
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    T* O = (T*)a.o + a.so.at(b, h) + (int64_t)row * a.so.s;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g)
            store4<T>(O, 32 * dt + 8 * g + 4 * hh, D, oacc[dt][4 * g] * inv, oacc[dt][4 * g + 1] * inv,
                      oacc[dt][4 * g + 2] * inv, oacc[dt][4 * g + 3] * inv, a.vec4_ok != 0);
    if (a.lse && hh == 0) {
        const int64_t ri = (int64_t)(b * a.Hq + h) * S + row;
        if constexpr (MASK) {
            a.lse[2 * ri] = l_tot > 0.f ? m_run : INFINITY;
            a.lse[2 * ri + 1] = l_tot > 0.f ? logf(l_tot) : 0.f;
        } else {
            a.lse[ri] = l_tot > 0.f ? (m_run + log2f(l_tot)) * kLn2 : INFINITY;
        }
    }
}

// Merge the partial slots of every split query tile, in slot order:
// m = max_i m_i, l = sum_i l_i 2^(m_i - m), O = sum_i O_i 2^(m_i - m) / l,
// LSE = (m + log2 l) ln 2.  One workgroup per (batch, head, query tile,
// group of RW = merge_rows(D) rows); workgroups of tiles that were not split
// return at once.  The per-(slot, row) weights go through LDS (sized by RW),
// then 256 / RW threads share a row: thread t sums its row's 16-byte chunks
// t % (256 / RW) + (256 / RW) j over the slots, kCombBatch slots' loads in
// flight together.
template <bool CAUSAL, typename T, int RW>
__global__ __launch_bounds__(256) void attn_fwd_combine(FwdArgs a) {
    constexpr int BM = kFwdBM, RG = BM / RW, TPR = 256 / RW, MAXJ = 4;
    __shared__ float wgt[kCombMaxSlots][RW];
    __shared__ float2 ml[kCombMaxSlots][RW];
    __shared__ float inv_l[RW];
    __shared__ int64_t slot_of[kCombMaxSlots];
    const int S = a.S, D = a.D;
    const int nqt = (S + BM - 1) / BM;
    const int rg = (int)blockIdx.x % RG, qt = ((int)blockIdx.x / RG) % nqt, bh = (int)blockIdx.x / (RG * nqt);
    const FastTiles tiles{S, CAUSAL, a.window, a.group, 0};
    int u0;
    const int nsl = tile_units(tiles, a.us, qt, &u0);
    const int r0 = qt * BM + rg * RW;
    if (nsl <= 1 || r0 >= S) return;
    const bool starts = unit_first(tiles, a.us, u0) == tiles.start(qt);
    const int64_t head_slots = (int64_t)bh * 2 * a.us.units;
    const int rows = min(RW, S - r0), rit = rg * RW;  // rows, first row inside the tile
    const int tid = threadIdx.x;
    if (tid < nsl) slot_of[tid] = head_slots + split_slot(u0 + tid, u0, starts);
    __syncthreads();
    // (running max, sum) of every (slot, row), loaded in parallel.
    for (int i = tid; i < nsl * rows; i += 256) {
        const int p = i / rows, r = i - p * rows;
        ml[p][r] = *reinterpret_cast<const float2*>(a.part_ml + (slot_of[p] * BM + rit + r) * 2);
    }
    __syncthreads();
    if (tid < rows) {
        float m = -INFINITY;
        for (int p = 0; p < nsl; ++p) m = fmaxf(m, ml[p][tid].x);
        float l = 0.f;
        for (int p = 0; p < nsl; ++p) {
            const float wp = ml[p][tid].x == -INFINITY ? 0.f : fast_exp2(ml[p][tid].x - m);
            l += ml[p][tid].y * wp;
            wgt[p][tid] = wp;
        }
        // l = 0: the row sees no key (see fwd_store_row)
        inv_l[tid] = l > 0.f ? 1.f / l : 0.f;
        if (a.lse) a.lse[(int64_t)bh * S + r0 + tid] = l > 0.f ? (m + log2f(l)) * kLn2 : INFINITY;
    }
    __syncthreads();
    const int r = tid / TPR, cl = tid % TPR, cg = D / 4;  // fast path: D % 4 == 0
    if (r >= rows) return;
    const int64_t rr = rit + r;
    f32x4 acc[MAXJ];
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int p0 = 0; p0 < nsl; p0 += kCombBatch) {
        f32x4 x[kCombBatch][MAXJ];
#pragma unroll
        for (int q = 0; q < kCombBatch; ++q) {
            if (p0 + q >= nsl) break;
            const float* src = a.part_o + (slot_of[p0 + q] * BM + rr) * D;
#pragma unroll
            for (int j = 0; j < MAXJ; ++j) {
                const int c = cl + TPR * j;
                x[q][j] = c < cg ? *reinterpret_cast<const f32x4*>(src + 4 * c) : f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
#pragma unroll
        for (int q = 0; q < kCombBatch; ++q) {
            if (p0 + q >= nsl) break;
            const float wp = wgt[p0 + q][r];
#pragma unroll
            for (int j = 0; j < MAXJ; ++j) acc[j] += x[q][j] * wp;
        }
    }
    const float il = inv_l[r];
    T* O = (T*)a.o + a.so.at(bh / a.Hq, bh % a.Hq) + (int64_t)(r0 + r) * a.so.s;
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) {
        const int c = cl + TPR * j;
        if (c < cg) store4<T>(O, 4 * c, D, acc[j][0] * il, acc[j][1] * il, acc[j][2] * il, acc[j][3] * il, true);
    }
}

template <typename T, int DP, int NW, int BN>
hipError_t launch_fwd_t(const AttnShape& s, FwdArgs a, hipStream_t st) {
    constexpr int BM = 32 * NW;
    a.n_qtiles = (int)((s.S + BM - 1) / BM);
    dim3 grid(a.n_qtiles, (unsigned)s.Hq, (unsigned)s.B);
    if (s.masked)  // causal or not: mask_score applies the flag per element
        hipLaunchKernelGGL((attn_fwd_kernel<T, DP, NW, BN, false, true>), grid, dim3(NW * 64), 0, st, a);
    else if (s.causal)
        hipLaunchKernelGGL((attn_fwd_kernel<T, DP, NW, BN, true>), grid, dim3(NW * 64), 0, st, a);
    else
        hipLaunchKernelGGL((attn_fwd_kernel<T, DP, NW, BN, false>), grid, dim3(NW * 64), 0, st, a);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_fwd_dispatch(const AttnShape& s, FwdArgs a, hipStream_t st) {
    constexpr bool F32 = sizeof(T) == 4;
    if (s.masked) {
        // mask mode: the general kernel only
    } else if constexpr (!F32) {
        if (s.D % 8 == 0 && s.D > 32) {
            if (s.D <= 64) return launch_fwd_fast64(s, a, st);
            if (s.D <= 128) return launch_fwd_fast128(s, a, st);
            return launch_fwd_fast256(s, a, st);
        }
    } else {
        // the fp32 fast kernels run the balanced launch only (with a workspace)
        if (f32::fast_path(s) && a.part_o != nullptr) return f32::launch_fwd_fast(s, a, st);
    }
    if (s.D <= 32) return launch_fwd_t<T, 32, 4, 64>(s, a, st);
    if (s.D <= 64) return launch_fwd_t<T, 64, 4, 64>(s, a, st);
    if (s.D <= 128) return launch_fwd_t<T, 128, 4, 64>(s, a, st);
    return launch_fwd_t<T, 256, 4, F32 ? 32 : 64>(s, a, st);
}

}  // namespace

namespace fwd {
hipError_t launch_fwd_combine(const AttnShape& s, const FwdArgs& a, hipStream_t st) {
    const int rw = merge_rows(s.D);
    const dim3 cgrid((unsigned)(s.B * s.Hq * a.n_qtiles * (kFwdBM / rw)));
#define MFT_COMBINE(T, RW)                                                                      \
    do {                                                                                        \
        if (s.causal)                                                                           \
            hipLaunchKernelGGL((attn_fwd_combine<true, T, RW>), cgrid, dim3(256), 0, st, a);    \
        else                                                                                    \
            hipLaunchKernelGGL((attn_fwd_combine<false, T, RW>), cgrid, dim3(256), 0, st, a);   \
    } while (0)
    if (s.bf16) {
        if (rw == 16) MFT_COMBINE(bf16, 16);
        else if (rw == 32) MFT_COMBINE(bf16, 32);
        else MFT_COMBINE(bf16, 64);
    } else {
        if (rw == 16) MFT_COMBINE(float, 16);
        else if (rw == 32) MFT_COMBINE(float, 32);
        else MFT_COMBINE(float, 64);
    }
#undef MFT_COMBINE
    return hipGetLastError();
}
hipError_t launch_fwd_fast64(const AttnShape& s, FwdArgs a, hipStream_t st) { return launch_fwd_fast_t<64>(s, a, st); }
hipError_t launch_fwd_fast128(const AttnShape& s, FwdArgs a, hipStream_t st) {
    return launch_fwd_fast_t<128>(s, a, st);
}
}  // namespace fwd

int fwd_rows_per_block(const AttnShape&) { return 128; }

FwdPlan plan_fwd_split(const AttnShape& s) {
    FwdPlan p{};
    p.balanced = !s.masked && ((s.bf16 && s.D % 8 == 0 && s.D > 32) || f32::fast_path(s));
    // bf16 shapes whose query tiles alone fill half the launch's slots or
    // more, and whose longest tile is at most 16 key tiles (causal S <= 1024,
    // or a sliding window up to ~900 keys), run one workgroup per query tile:
    // the split's partial stores and combine launch cost more than its
    // shorter units save.  Measured: C4 forward 32.5 against 34.5 us, C5 with
    // a 512-key window 25.4 against 37.4 us; C3 at S = 2048 (32 key tiles)
    // 50.2 against 41.3, and the fp32 fast path at C2 63.5 against 41.0, so
    // those stay split.
    if (p.balanced && s.bf16) {
        const int nqt = (int)((s.S + kFwdBM - 1) / kFwdBM);
        const int64_t tiles = s.B * s.Hq * nqt, slots = fwd_unit_slots(s);
        // the last query tile sees the most key tiles (causal or windowed)
        const int longest = fast_q_n((int)s.S, s.causal ? 1 : 0, s.window, nqt - 1);
        if (longest <= 16 && 2 * tiles >= slots && tiles <= slots) p.balanced = false;
    }
    if (!p.balanced) return p;
    const int S = (int)s.S, causal = s.causal ? 1 : 0, W = s.window;
    const int64_t pairs = s.B * s.Hq;
    const int64_t u = balanced_units(pairs, fwd_unit_slots(s));
    // Units of about equal cost, no shorter than kMinFwdUnitIters key tiles
    // (a split costs one fp32 partial tile), no query tile over kCombMaxSlots.
    const FastTiles g{S, causal, W, (int)(s.Hq / s.Hkv), 0};
    p.us = fit_unit_split(g, u, kFwdIterCost, fwd_tile_cost(s), kMinFwdUnitIters, kCombMaxSlots,
                          &p.parts_max);
    p.any_split = p.parts_max > 1;
    return p;
}

size_t fwd_workspace_bytes(const AttnShape& s, const FwdPlan& p) {
    if (!p.balanced) return 0;
    const size_t rows = p.any_split ? static_cast<size_t>(s.B * s.Hq) * 2 * p.us.units * kFwdBM : 0;
    auto up = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
    // Always non-zero for this path, so that a caller that passes the queried
    // workspace gets the balanced launch.
    return up(rows * static_cast<size_t>(s.D) * 4) + up(rows * 2 * 4) + 256;
}

hipError_t launch_attn_fwd(const AttnShape& s, const FwdPlan& p, const void* q, const void* k, const void* v, void* o,
                           float* lse, void* workspace, hipStream_t st) {
    FwdArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = o;
    a.lse = lse;
    a.B = (int)s.B;
    a.S = (int)s.S;
    a.D = (int)s.D;
    a.Hq = (int)s.Hq;
    a.Hkv = (int)s.Hkv;
    a.group = (int)(s.Hq / s.Hkv);
    a.n_qtiles = 0;
    a.scale_log2 = s.scale * kLog2e;
    a.vec_ok = (s.D % (s.bf16 ? 8 : 4)) == 0;
    a.vec4_ok = (s.D % 4) == 0;
    a.window = s.window;
    a.kv_len = s.kv_len;
    a.sq = s.q;
    a.sk = s.k;
    a.sv = s.v;
    a.so = s.o;
    a.us = UnitSplit{0, 0, 0, 0};
    a.any_split = 0;
    a.part_o = nullptr;
    a.part_ml = nullptr;
    a.m0 = s.m0;
    a.m1 = s.m1;
    a.mask_causal = s.causal ? 1 : 0;
    a.scale = s.scale;
    if (workspace && p.balanced) {
        a.us = p.us;
        a.any_split = p.any_split ? 1 : 0;
        const size_t rows = p.any_split ? static_cast<size_t>(s.B * s.Hq) * 2 * p.us.units * kFwdBM : 0;
        const size_t ob = (rows * static_cast<size_t>(s.D) * 4 + 255) & ~static_cast<size_t>(255);
        a.part_o = static_cast<float*>(workspace);
        a.part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + ob);
    }
    const hipError_t e = s.bf16 ? launch_fwd_dispatch<bf16>(s, a, st) : launch_fwd_dispatch<float>(s, a, st);
    if (e != hipSuccess) return e;
    return launch_fwd_masked_rows(s, v, o, st);
}

}  // namespace mft
