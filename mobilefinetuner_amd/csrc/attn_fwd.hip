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
#include "attn_kernels.h"

namespace mft {
namespace {

struct FwdArgs {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* lse;
    int B, S, D, Hq, Hkv, group, n_qtiles;
    float scale_log2;  // softmax scale * log2(e)
    int vec_ok;        // D % (16 bytes / element size) == 0
    int vec4_ok;       // D % 4 == 0
    int window;              // causal sliding window, 0 = none
    const int* kv_len;       // [B] valid keys per batch, or null
    Strides sq, sk, sv, so;  // layouts of q, k, v, o
    // balanced launch (bf16 fast path with a workspace; see FwdPlan)
    int chunk;               // iterations per unit
    int units;               // units per (batch, head)
    float* part_o;           // [B*Hq][2*units][128][D] unnormalised O (split_slot)
    float* part_ml;          // [B*Hq][2*units][128][2] running max (log2 units), sum
};

template <typename T, int DP, int BN> struct FwdLds {
    static constexpr bool VT = sizeof(T) == 2;  // V staged transposed (bf16)
    static constexpr int KSTR = DP + Elt<T>::VEC;
    static constexpr int VSTR = VT ? BN + 4 : DP + 4;
    static constexpr int K_ELEMS = BN * KSTR;
    static constexpr int V_ELEMS = VT ? DP * VSTR : BN * VSTR;
};

template <typename T, int DP, int NW, int BN, bool CAUSAL>
__global__ __launch_bounds__(NW * 64) void attn_fwd_kernel(FwdArgs a) {
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
            s[kk] = zero16();
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const V ka = *reinterpret_cast<const V*>(Ks + (32 * kk + n) * L::KSTR + 2 * VEC * c + VEC * hh);
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
                if (need_mask) {
                    const int key = kbase + 32 * kk + row_of_reg(r, hh);
                    if (!vis.visible(row, key)) x = -INFINITY;
                }
                s[kk][r] = x;
                mx = fmaxf(mx, x);
            }
        }
        mx = fmaxf(mx, other_half(mx));
        const float m_new = fmaxf(m_run, mx * a.scale_log2);
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = fast_exp2(m_run - m_use);
        float psum = 0.f;
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = fast_exp2(s[kk][r] * a.scale_log2 - m_use);
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
    const float l_tot = l_run + other_half(l_run);
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
    if (a.lse && hh == 0)
        a.lse[(int64_t)(b * a.Hq + h) * S + row] = l_tot > 0.f ? (m_run + log2f(l_tot)) * kLn2 : INFINITY;
}

// ---------------------------------------------------------------------------
// bf16 fast path (D % 8 == 0, 32 < D <= 256).
//
// Same decomposition and math as attn_fwd_kernel, but K/V tiles move
// HBM -> LDS with global_load_lds_dwordx4 (no VGPR round trip), double
// buffered so the next tile streams in while the current one is computed.
// LDS rows are unpadded and XOR-swizzled in 16-byte chunks:
//   K: swz_row (row reads of the S^T A operand), V: swz_tr (transposing
//      reads of the O^T A operand); see attn_common.h.
// V stays row-major; the transposing LDS read delivers V^T to the MFMA A
// operand directly (see ds_read_tr4).
//
// Two launch shapes share the per-tile step:
//   attn_fwd_bf16_fast  one workgroup per 128-row query tile (longest first);
//   attn_fwd_bf16_split the (query tile, 64-key tile) iterations of each
//                       (batch, head) flattened and cut into equal units, about
//                       one per CU; a query tile spread over several units
//                       leaves unnormalised fp32 partials (O, running max, sum)
//                       that attn_fwd_combine merges by log-sum-exp in slot order.

constexpr int kFwdBM = 128, kFwdBN = 64;

// Direct loads per thread of one K (or V) tile, and of both.
template <int DP> struct FwdLoads {
    static constexpr int PER = kFwdBN * (DP / 8) / 256, NPARTS = 2 * PER;
};

// One 64-key tile for this wave's 32 rows: S^T = K Q^T, online softmax with
// lazy rescale, O^T += V^T P^T.  Kb/Vb: the tile in LDS.  issue_part(j),
// j < FwdLoads<DP>::NPARTS, issues the next tile's loads; they are spread
// over the S^T steps.  need_mask (wave-uniform): some key of the tile is
// hidden from some row; this lane's row sees keys [vlo, vhi].
template <int DP, class IssuePart>
__device__ __forceinline__ void fwd_fast_tile(const FwdArgs& a, const bf16* Kb, const bf16* Vb, int kbase,
                                              bool need_mask, int vlo, int vhi, const bf16x8 (&qf)[DP / 16],
                                              f32x16 (&oacc)[DP / 32], float& m_run, float& l_run,
                                              const IssuePart& issue_part) {
    constexpr int NPARTS = FwdLoads<DP>::NPARTS;
    constexpr int BN = kFwdBN, CPR = DP / 8, NC = DP / 16, NDT = DP / 32, NKK = BN / 32;
    constexpr int PF = 4;  // LDS operand prefetch depth
    const int lane = threadIdx.x & 63, n = lane & 31, hh = lane >> 5;
    const int i16 = lane & 15, nh = (lane >> 4) & 1;

    // S^T = K Q^T: the NKK independent accumulator chains are interleaved
    // and the K operands stream through a PF-deep register ring, so LDS
    // latency overlaps the MFMAs instead of stalling each one.
    f32x16 s[NKK];
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) s[kk] = zero16();
    {
        constexpr int NI = NKK * NC;
        auto kread = [&](int it) {
            return *reinterpret_cast<const bf16x8*>(
                Kb + tile_off<CPR, SWZ_ROW>(32 * (it % NKK) + n, 16 * (it / NKK) + 8 * hh));
        };
        bf16x8 ring[PF];
#pragma unroll
        for (int it = 0; it < PF; ++it) ring[it] = kread(it);
#pragma unroll
        for (int it = 0; it < NI; ++it) {
            const bf16x8 ka = ring[it % PF];
            if (it + PF < NI) ring[it % PF] = kread(it + PF);
            s[it % NKK] = mfma_bf16(ka, qf[it / NKK], s[it % NKK]);
            if ((it & 1) && (it >> 1) < NPARTS) issue_part(it >> 1);
        }
#pragma unroll
        for (int j = NI / 2; j < NPARTS; ++j) issue_part(j);
    }

    // Keys outside [vlo, vhi] are masked, as selects so the hot loop stays
    // branch-free.
    if (need_mask) {
        const int hi = vhi - kbase, lo = vlo - kbase;
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int kl = 32 * kk + row_of_reg(r, hh);
                s[kk][r] = (kl > hi || kl < lo) ? -INFINITY : s[kk][r];
            }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kk][r]);
    mx = fmaxf(mx, other_half(mx)) * a.scale_log2;
    // Lazy rescaling: the reference point m_run only moves (and O, l are
    // rescaled) when some row of the wave sees a max above m_run + 8, so
    // exp2 arguments stay <= 8 and P <= 256.  Any reference point gives
    // the same O = acc / l and LSE = m_run + log2(l); this one skips the
    // per-tile O multiply, which lives in accumulation registers.
    if (__any(mx > m_run + kLazyRescale)) {
        const float m_new = fmaxf(m_run, mx);
        const float alpha = fast_exp2(m_run - (m_new == -INFINITY ? 0.f : m_new));
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
        m_run = m_new;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    float psum = 0.f;
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float p = fast_exp2(s[kk][r] * a.scale_log2 - m_use);
            s[kk][r] = p;
            psum += p;
        }
    }
    l_run += psum;

    // O^T += V^T P^T, V^T operands through the same kind of register ring.
    {
        bf16x8 pb[2 * NKK];
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk)
#pragma unroll
            for (int e = 0; e < 2; ++e)
#pragma unroll
                for (int j = 0; j < 8; ++j) pb[2 * kk + e][j] = (bf16)s[kk][8 * e + j];
        constexpr int NI = 2 * NKK * NDT;  // iteration = (kk, e) block x dt
        auto vread = [&](int it) {
            const int ke = it / NDT, dt = it % NDT;
            const int r0 = 16 * ke + 4 * hh + (i16 >> 2);
            const int col = 32 * dt + 16 * nh + 4 * (i16 & 3);
            const bf16x4 lo = ds_read_tr4(Vb + tile_off<CPR, SWZ_TR>(r0, col));
            const bf16x4 hi = ds_read_tr4(Vb + tile_off<CPR, SWZ_TR>(r0 + 8, col));
            return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        };
        bf16x8 ring[PF];
#pragma unroll
        for (int it = 0; it < PF; ++it) ring[it] = vread(it);
#pragma unroll
        for (int it = 0; it < NI; ++it) {
            const bf16x8 va = ring[it % PF];
            if (it + PF < NI) ring[it % PF] = vread(it + PF);
            oacc[it % NDT] = mfma_bf16(va, pb[it / NDT], oacc[it % NDT]);
        }
        pin_read_ahead<NI, PF, 2>();
    }
}

// This lane's query row: Q fragments (B operand of S^T).
template <int DP>
__device__ __forceinline__ void fwd_load_q(const bf16* Q, int ld, int row, int S, int D, bf16x8 (&qf)[DP / 16]) {
    const int hh = (threadIdx.x & 63) >> 5;
    const int rowc = row < S ? row : S - 1;
#pragma unroll
    for (int c = 0; c < DP / 16; ++c)
        qf[c] = load_chunk<bf16>(Q + (int64_t)rowc * ld, 16 * c + 8 * hh, D, row < S, true);
}

// Normalised O row and its LSE (rows < S; call with the wave's l_tot).  A
// row that sees no key (key padding) gets O = 0 and LSE = +inf here, and the
// reference's output from attn_fwd_masked_rows.
template <int DP>
__device__ __forceinline__ void fwd_store_row(const FwdArgs& a, int b, int h, int row, const f32x16 (&oacc)[DP / 32],
                                              float m_run, float l_tot) {
    const int hh = (threadIdx.x & 63) >> 5;
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    bf16* O = (bf16*)a.o + a.so.at(b, h) + (int64_t)row * a.so.s;
#pragma unroll
    for (int dt = 0; dt < DP / 32; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g)
            store4<bf16>(O, 32 * dt + 8 * g + 4 * hh, a.D, oacc[dt][4 * g] * inv, oacc[dt][4 * g + 1] * inv,
                         oacc[dt][4 * g + 2] * inv, oacc[dt][4 * g + 3] * inv, true);
    if (a.lse && hh == 0)
        a.lse[(int64_t)(b * a.Hq + h) * a.S + row] = l_tot > 0.f ? (m_run + log2f(l_tot)) * kLn2 : INFINITY;
}

template <int DP, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_fwd_bf16_fast(FwdArgs a) {
    constexpr int BN = kFwdBN, BM = kFwdBM, NT = 256;
    constexpr int CPR = DP / 8, NC = DP / 16, NDT = DP / 32;
    constexpr int TILE = BN * DP;             // elements of one K or V tile
    __shared__ __attribute__((aligned(1024))) bf16 smem[2 * 2 * TILE];

    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6, n = lane & 31;
    const int S = a.S, D = a.D;
    const int qt = a.n_qtiles - 1 - (int)blockIdx.x;
    const int h = blockIdx.y, b = blockIdx.z, hk = h / a.group;
    const int m0 = qt * BM;
    const int wrow0 = m0 + 32 * w;
    const int row = wrow0 + n;

    const bf16* __restrict__ Q = (const bf16*)a.q + a.sq.at(b, h);
    const bf16* __restrict__ K = (const bf16*)a.k + a.sk.at(b, hk);
    const bf16* __restrict__ Vg = (const bf16*)a.v + a.sv.at(b, hk);
    const int lq = a.sq.s, lk = a.sk.s, lv = a.sv.s;

    const KeyVis vis{S, a.window, a.kv_len ? min(max(a.kv_len[b], 0), S) : S, CAUSAL};
    const int vlo = vis.lo(row), vhi = vis.hi(row);
    const int t0 = fast_q_lo(CAUSAL, a.window, qt);
    const int ntiles = t0 + fast_q_n(S, CAUSAL, a.window, qt);
    issue_tile<DP, BN, NT, SWZ_ROW>(K, t0 * BN, S, D, lk, smem);
    issue_tile<DP, BN, NT, SWZ_TR>(Vg, t0 * BN, S, D, lv, smem + TILE);

    bf16x8 qf[NC];
    fwd_load_q<DP>(Q, lq, row, S, D, qf);
    wait_vmcnt<0>();  // Q complete before the loop (direct loads are untracked)
    f32x16 oacc[NDT];
#pragma unroll
    for (int i = 0; i < NDT; ++i) oacc[i] = zero16();
    float m_run = -INFINITY, l_run = 0.f;

    for (int t = t0; t < ntiles; ++t) {
        const bf16* Kb = smem + ((t - t0) & 1) * 2 * TILE;
        const bf16* Vb = Kb + TILE;
        // This wave's loads of tile t (issued one tile ago) have landed; after
        // the barrier every wave's have, and every wave is done with the
        // buffer tile t+1 streams into.
        wait_vmcnt<0>();
        lds_barrier();
        // Next tile's loads, spread over this tile's S^T steps; the last
        // tile re-loads tile 0 into the idle buffer (no branch in the
        // schedule; waited for before the end).
        bf16* const nb = smem + ((t - t0 + 1) & 1) * 2 * TILE;
        const int nrow = t + 1 < ntiles ? (t + 1) * BN : t0 * BN;
        auto issue_part = [&](int j) {
            if (j < FwdLoads<DP>::PER)
                issue_tile_part<DP, BN, NT, SWZ_ROW>(K, nrow, S, D, lk, nb, j);
            else
                issue_tile_part<DP, BN, NT, SWZ_TR>(Vg, nrow, S, D, lv, nb + TILE, j - FwdLoads<DP>::PER);
        };
        const int kbase = t * BN;
        if (wave_uniform(wrow0 < S && vis.any(wrow0, min(wrow0 + 31, S - 1), kbase, kbase + BN - 1))) {
            const bool need_mask = wave_uniform(!vis.all(wrow0, wrow0 + 31, kbase, kbase + BN - 1));
            fwd_fast_tile<DP>(a, Kb, Vb, kbase, need_mask, vlo, vhi, qf, oacc, m_run, l_run, issue_part);
        } else {
#pragma unroll
            for (int j = 0; j < FwdLoads<DP>::NPARTS; ++j) issue_part(j);
        }
    }
    wait_vmcnt<0>();

    if (wrow0 >= S) return;
    const float l_tot = l_run + other_half(l_run);
    if (row >= S) return;
    fwd_store_row<DP>(a, b, h, row, oacc, m_run, l_tot);
}

// Balanced launch: workgroup i = unit i / (B*Hq) of (batch, head) i % (B*Hq).
template <int DP, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_fwd_bf16_split(FwdArgs a) {
    constexpr int BN = kFwdBN, BM = kFwdBM, NT = 256;
    constexpr int CPR = DP / 8, NC = DP / 16, NDT = DP / 32;
    constexpr int TILE = BN * DP;
    __shared__ __attribute__((aligned(1024))) bf16 smem[2 * 2 * TILE];

    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6, n = lane & 31, hh = lane >> 5;
    const int S = a.S, D = a.D;
    const int bh = a.B * a.Hq, blk = (int)blockIdx.x;
    const int unit = blk / bh, b = (blk % bh) / a.Hq, h = (blk % bh) % a.Hq, hk = h / a.group;

    const bf16* __restrict__ Q = (const bf16*)a.q + a.sq.at(b, h);
    const bf16* __restrict__ K = (const bf16*)a.k + a.sk.at(b, hk);
    const bf16* __restrict__ Vg = (const bf16*)a.v + a.sv.at(b, hk);
    const int lq = a.sq.s, lk = a.sk.s, lv = a.sv.s;

    const int W = a.window;
    const KeyVis vis{S, W, a.kv_len ? min(max(a.kv_len[b], 0), S) : S, CAUSAL};
    // This unit's chunk of the flattened (query tile, key tile) iterations.
    const int64_t g0 = (int64_t)unit * a.chunk;
    const int niter = (int)min((int64_t)a.chunk, fast_q_total(S, CAUSAL, W) - g0);
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
        const int t0 = next_key_tile();
        issue_tile<DP, BN, NT, SWZ_ROW>(K, t0 * BN, S, D, lk, smem);
        issue_tile<DP, BN, NT, SWZ_TR>(Vg, t0 * BN, S, D, lv, smem + TILE);
    }

    bf16x8 qf[NC];
    f32x16 oacc[NDT];
    float m_run, l_run;
    int64_t qstart = fast_q_start(S, CAUSAL, W, qt);
    int qn = fast_q_n(S, CAUSAL, W, qt);
    int qlo = fast_q_lo(CAUSAL, W, qt);
    fwd_load_q<DP>(Q, lq, qt * BM + 32 * w + n, S, D, qf);
    wait_vmcnt<0>();  // Q complete before the loop (direct loads are untracked)

    for (int i = 0, first = 1;; first = 0) {
#pragma unroll
        for (int d = 0; d < NDT; ++d) oacc[d] = zero16();
        m_run = -INFINITY;
        l_run = 0.f;
        const int wrow0 = qt * BM + 32 * w, row = wrow0 + n;
        const int vlo = vis.lo(row), vhi = vis.hi(row);
        // Iterations of query tile qt inside this unit, then its output.
        const int seg_end = (int)min((int64_t)niter, qstart + qn - g0);
        for (; i < seg_end; ++i) {
            const bf16* Kb = smem + (i & 1) * 2 * TILE;
            const bf16* Vb = Kb + TILE;
            wait_vmcnt<0>();  // as in attn_fwd_bf16_fast
            lds_barrier();
            bf16* const nb = smem + ((i + 1) & 1) * 2 * TILE;
            const int nrow = i + 1 < niter ? next_key_tile() * BN : 0;
            auto issue_part = [&](int j) {
                if (j < FwdLoads<DP>::PER)
                    issue_tile_part<DP, BN, NT, SWZ_ROW>(K, nrow, S, D, lk, nb, j);
                else
                    issue_tile_part<DP, BN, NT, SWZ_TR>(Vg, nrow, S, D, lv, nb + TILE, j - FwdLoads<DP>::PER);
            };
            const int kbase = (qlo + (int)(g0 + i - qstart)) * BN;
            if (wave_uniform(wrow0 < S && vis.any(wrow0, min(wrow0 + 31, S - 1), kbase, kbase + BN - 1))) {
                const bool need_mask = wave_uniform(!vis.all(wrow0, wrow0 + 31, kbase, kbase + BN - 1));
                fwd_fast_tile<DP>(a, Kb, Vb, kbase, need_mask, vlo, vhi, qf, oacc, m_run, l_run, issue_part);
            } else {
#pragma unroll
                for (int j = 0; j < FwdLoads<DP>::NPARTS; ++j) issue_part(j);
            }
        }
        // End of this unit's part of query tile qt: a tile inside one unit is
        // written normalised; otherwise this unit's slot gets the unnormalised
        // partial (O, running max, sum) for attn_fwd_combine.
        if (wrow0 < S) {
            const float l_tot = l_run + other_half(l_run);
            const int nsl = fast_slots(qstart, qn, a.chunk);
            if (nsl <= 1) {
                if (row < S) fwd_store_row<DP>(a, b, h, row, oacc, m_run, l_tot);
            } else if (row < S) {
                const int64_t slot = (int64_t)(b * a.Hq + h) * 2 * a.units + 2 * unit + (first ? 0 : 1);
                float* po = a.part_o + (slot * BM + 32 * w + n) * D;
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                    for (int g = 0; g < 4; ++g)
                        store4<float>(po, 32 * dt + 8 * g + 4 * hh, D, oacc[dt][4 * g], oacc[dt][4 * g + 1],
                                      oacc[dt][4 * g + 2], oacc[dt][4 * g + 3], true);
                if (hh == 0) {
                    float* pml = a.part_ml + (slot * BM + 32 * w + n) * 2;
                    pml[0] = m_run;
                    pml[1] = l_tot;
                }
            }
        }
        if (i >= niter) {
            wait_vmcnt<0>();  // the last tile's re-load has landed before the unit ends
            break;
        }
        ++qt;
        qstart = fast_q_start(S, CAUSAL, W, qt);
        qn = fast_q_n(S, CAUSAL, W, qt);
        qlo = fast_q_lo(CAUSAL, W, qt);
        fwd_load_q<DP>(Q, lq, qt * BM + 32 * w + n, S, D, qf);
        wait_vmcnt<0>();
    }
}

// Merge the partial slots of every split query tile, in slot order:
// m = max_i m_i, l = sum_i l_i 2^(m_i - m), O = sum_i O_i 2^(m_i - m) / l,
// LSE = (m + log2 l) ln 2.  One workgroup per (batch, head, query tile,
// 16-row group); workgroups of tiles that were not split return at once.
// The per-(slot, row) weights go through LDS, then each thread sums 16-byte
// column chunks over the slots.
constexpr int kCombRows = 16, kCombMaxSlots = 64;

template <bool CAUSAL>
__global__ __launch_bounds__(256) void attn_fwd_combine(FwdArgs a) {
    constexpr int BM = kFwdBM, RG = BM / kCombRows;
    __shared__ float wgt[kCombMaxSlots][kCombRows];
    __shared__ float2 ml[kCombMaxSlots][kCombRows];
    __shared__ float inv_l[kCombRows];
    const int S = a.S, D = a.D;
    const int nqt = (S + BM - 1) / BM;
    const int rg = (int)blockIdx.x % RG, qt = ((int)blockIdx.x / RG) % nqt, bh = (int)blockIdx.x / (RG * nqt);
    const int64_t qstart = fast_q_start(S, CAUSAL, a.window, qt);
    const int nsl = fast_slots(qstart, fast_q_n(S, CAUSAL, a.window, qt), a.chunk);
    const int r0 = qt * BM + rg * kCombRows;
    if (nsl <= 1 || r0 >= S) return;
    const int64_t u0 = qstart / a.chunk, head_slots = (int64_t)bh * 2 * a.units;
    __shared__ int64_t slot_of[kCombMaxSlots];
    const int rows = min(kCombRows, S - r0);
    const int tid = threadIdx.x;
    if (tid < nsl) slot_of[tid] = head_slots + split_slot(qstart, a.chunk, u0 + tid, u0);
    __syncthreads();
    // (running max, sum) of every (slot, row), loaded in parallel.
    for (int i = tid; i < nsl * kCombRows; i += 256) {
        const int p = i / kCombRows, r = i % kCombRows;
        ml[p][r] = *reinterpret_cast<const float2*>(a.part_ml + (slot_of[p] * BM + rg * kCombRows + r) * 2);
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
    // Thread -> row tid / 16, 16-byte column chunks (tid % 16) + 16 j: the
    // chunks' loads of one slot are independent and issued together.
    const int r = tid / 16, cl = tid % 16, cg = D / 4;  // fast path: D % 8 == 0
    if (r >= rows) return;
    constexpr int MAXJ = 256 / 4 / 16;
    const int64_t rr = rg * kCombRows + r;
    f32x4 acc[MAXJ];
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int p = 0; p < nsl; ++p) {
        const float* src = a.part_o + (slot_of[p] * BM + rr) * D;
        const float wp = wgt[p][r];
        f32x4 x[MAXJ];
#pragma unroll
        for (int j = 0; j < MAXJ; ++j) {
            const int c = cl + 16 * j;
            x[j] = c < cg ? *reinterpret_cast<const f32x4*>(src + 4 * c) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int j = 0; j < MAXJ; ++j) acc[j] += x[j] * wp;
    }
    const float il = inv_l[r];
    bf16* O = (bf16*)a.o + a.so.at(bh / a.Hq, bh % a.Hq) + (int64_t)(r0 + r) * a.so.s;
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) {
        const int c = cl + 16 * j;
        if (c < cg) store4<bf16>(O, 4 * c, D, acc[j][0] * il, acc[j][1] * il, acc[j][2] * il, acc[j][3] * il, true);
    }
}

template <int DP>
hipError_t launch_fwd_fast(const AttnShape& s, FwdArgs a, hipStream_t st) {
    a.n_qtiles = (int)((s.S + kFwdBM - 1) / kFwdBM);
    if (a.part_o) {
        const FwdPlan p = plan_fwd_split(s);
        a.chunk = p.chunk;
        a.units = p.units;
        const dim3 grid((unsigned)(p.units * s.B * s.Hq));
        if (s.causal)
            hipLaunchKernelGGL((attn_fwd_bf16_split<DP, true>), grid, dim3(256), 0, st, a);
        else
            hipLaunchKernelGGL((attn_fwd_bf16_split<DP, false>), grid, dim3(256), 0, st, a);
        if (p.any_split) {
            const dim3 cgrid((unsigned)(s.B * s.Hq * a.n_qtiles * (kFwdBM / kCombRows)));
            if (s.causal)
                hipLaunchKernelGGL(attn_fwd_combine<true>, cgrid, dim3(256), 0, st, a);
            else
                hipLaunchKernelGGL(attn_fwd_combine<false>, cgrid, dim3(256), 0, st, a);
        }
        return hipGetLastError();
    }
    dim3 grid(a.n_qtiles, (unsigned)s.Hq, (unsigned)s.B);
    if (s.causal)
        hipLaunchKernelGGL((attn_fwd_bf16_fast<DP, true>), grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((attn_fwd_bf16_fast<DP, false>), grid, dim3(256), 0, st, a);
    return hipGetLastError();
}

template <typename T, int DP, int NW, int BN>
hipError_t launch_fwd_t(const AttnShape& s, FwdArgs a, hipStream_t st) {
    constexpr int BM = 32 * NW;
    a.n_qtiles = (int)((s.S + BM - 1) / BM);
    dim3 grid(a.n_qtiles, (unsigned)s.Hq, (unsigned)s.B);
    if (s.causal)
        hipLaunchKernelGGL((attn_fwd_kernel<T, DP, NW, BN, true>), grid, dim3(NW * 64), 0, st, a);
    else
        hipLaunchKernelGGL((attn_fwd_kernel<T, DP, NW, BN, false>), grid, dim3(NW * 64), 0, st, a);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_fwd_dispatch(const AttnShape& s, FwdArgs a, hipStream_t st) {
    constexpr bool F32 = sizeof(T) == 4;
    if constexpr (!F32) {
        if (s.D % 8 == 0 && s.D > 32) {
            if (s.D <= 64) return launch_fwd_fast<64>(s, a, st);
            if (s.D <= 128) return launch_fwd_fast<128>(s, a, st);
            return launch_fwd_fast<256>(s, a, st);
        }
    }
    if (s.D <= 32) return launch_fwd_t<T, 32, 4, 64>(s, a, st);
    if (s.D <= 64) return launch_fwd_t<T, 64, 4, 64>(s, a, st);
    if (s.D <= 128) return launch_fwd_t<T, 128, 4, 64>(s, a, st);
    return launch_fwd_t<T, 256, 4, F32 ? 32 : 64>(s, a, st);
}

}  // namespace

int fwd_rows_per_block(const AttnShape&) { return 128; }

FwdPlan plan_fwd_split(const AttnShape& s) {
    const int S = (int)s.S, causal = s.causal ? 1 : 0, W = s.window;
    const int nqt = (S + kFwdBM - 1) / kFwdBM;
    const int64_t n = fast_q_total(S, causal, W);  // iterations per (batch, head)
    const int64_t pairs = s.B * s.Hq;
    const int64_t u = balanced_units(pairs, device_cus());
    FwdPlan p;
    // Units no shorter than 4 key tiles: a split costs one fp32 partial tile.
    // A query tile has at most 2*S/64 key tiles; keep its slots <= kCombMaxSlots.
    int64_t max_tile = 0;
    for (int t = 0; t < nqt; ++t) max_tile = std::max<int64_t>(max_tile, fast_q_n(S, causal, W, t));
    const int64_t min_chunk = std::max<int64_t>(4, (max_tile + kCombMaxSlots - 3) / (kCombMaxSlots - 2));
    p.chunk = (int)std::min<int64_t>(n, std::max<int64_t>(min_chunk, (n + u - 1) / u));
    p.units = (int)((n + p.chunk - 1) / p.chunk);
    p.any_split = false;
    for (int t = 0; t < nqt && !p.any_split; ++t)
        p.any_split = fast_slots(fast_q_start(S, causal, W, t), fast_q_n(S, causal, W, t), p.chunk) > 1;
    return p;
}

size_t fwd_workspace_bytes(const AttnShape& s) {
    if (!(s.bf16 && s.D % 8 == 0 && s.D > 32)) return 0;
    const FwdPlan p = plan_fwd_split(s);
    const size_t rows = p.any_split ? static_cast<size_t>(s.B * s.Hq) * 2 * p.units * kFwdBM : 0;
    auto up = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
    // Always non-zero for this path, so that a caller that passes the queried
    // workspace gets the balanced launch.
    return up(rows * static_cast<size_t>(s.D) * 4) + up(rows * 2 * 4) + 256;
}

hipError_t launch_attn_fwd(const AttnShape& s, const void* q, const void* k, const void* v, void* o,
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
    a.chunk = 0;
    a.units = 0;
    a.part_o = nullptr;
    a.part_ml = nullptr;
    if (workspace && fwd_workspace_bytes(s) > 0) {
        const FwdPlan p = plan_fwd_split(s);
        const size_t rows = p.any_split ? static_cast<size_t>(s.B * s.Hq) * 2 * p.units * kFwdBM : 0;
        const size_t ob = (rows * static_cast<size_t>(s.D) * 4 + 255) & ~static_cast<size_t>(255);
        a.part_o = static_cast<float*>(workspace);
        a.part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + ob);
    }
    const hipError_t e = s.bf16 ? launch_fwd_dispatch<bf16>(s, a, st) : launch_fwd_dispatch<float>(s, a, st);
    if (e != hipSuccess) return e;
    return launch_fwd_masked_rows(s, v, o, st);
}

}  // namespace mft
