// bf16 fast path of the attention forward (D % 8 == 0, 32 < D <= 256) for
// gfx950.  Included by attn_fwd.hip (D <= 128 instantiations) and
// attn_fwd_fast256.hip (D = 256), both built with MFMA accumulators in VGPRs.
//
// Work decomposition: a workgroup of 4 waves owns 128 query rows of one query
// head; wave w owns rows 32w .. 32w + 31, one per lane column.  Key tiles of
// 64 keys move HBM -> LDS with global_load_lds_dwordx4 (no VGPR round trip)
// into double buffers, so the next tile streams in while the current one is
// multiplied.  Per tile a wave computes S^T = K Q^T (keys along the
// accumulator rows, so each lane holds 16 scores of ONE query row: row max and
// sum are lane-local plus one swap with the other half-wave), the online
// softmax with a lazy rescale, and O^T += V^T P^T, whose B operand is the
// exp'd S^T registers themselves (no shuffle).  V stays row-major in LDS and
// the transposing LDS read delivers V^T to the MFMA.  GQA: the workgroup
// reads kv head h / group directly (no repeat_kv copy).
//
// Per-tile VALU work is kept to the softmax: every LDS read address is a
// loop-invariant per-lane register plus an immediate, every direct load a
// per-lane offset plus a scalar base (TileDma), and masks are applied only in
// the tiles that need them (a real branch, not selects executed always).  At
// D = 256 the live state (128 O accumulators, 32 scores, 64 Q registers)
// exceeds the 256 VGPRs only by what the compiler parks in AGPRs; the Q
// fragments are read by the MFMAs from there directly.
#pragma once

#include "attn_common.h"
#include "attn_geometry.h"
#include "attn_kernels.h"

namespace mft {
namespace fwd {

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
    UnitSplit us;            // work units per (batch, head)
    int any_split;           // some query tile spans several units (the combine runs)
    float* part_o;           // [B*Hq][2*us.units][128][D] unnormalised O (split_slot)
    float* part_ml;          // [B*Hq][2*units][128][2] running max (log2 units), sum
    // mask mode (AttnShape::masked; general kernel only)
    MaskView m0, m1;
    int mask_causal;
    float scale;
};

constexpr int kFwdBM = 128, kFwdBN = 64;
// Fewest vector stores a wave issues for a segment's output (32 per lane
// for D = 256: the fp32 partial O or the bf16 O); smaller head dims use
// vmcnt(0) (see attn_fwd_bf16_split).
constexpr int kEpilogueStores = 32;
constexpr int kCombMaxSlots = kSplitMaxSlots, kCombBatch = 4;

// The launches of the fast path for one padded head dim (attn_fwd.hip,
// attn_fwd_fast256.hip).
hipError_t launch_fwd_fast64(const AttnShape& s, FwdArgs a, hipStream_t st);
hipError_t launch_fwd_fast128(const AttnShape& s, FwdArgs a, hipStream_t st);
hipError_t launch_fwd_fast256(const AttnShape& s, FwdArgs a, hipStream_t st);
// The split launch's merge of partial query tiles (attn_fwd.hip).
hipError_t launch_fwd_combine(const AttnShape& s, const FwdArgs& a, hipStream_t st);
}  // namespace fwd

namespace f32 {
// The fp32 fast forward (attn_f32_fast.h): the balanced launch (a.part_o set).
hipError_t launch_fwd_fast(const AttnShape& s, const fwd::FwdArgs& a, hipStream_t st);
}  // namespace f32

namespace fwd {

namespace {

// Direct loads per thread of one K (or V) tile, and of both.
template <int DP> struct FwdLoads {
    static constexpr int PER = kFwdBN * (DP / 8) / 256, NPARTS = 2 * PER;
};

// Per-lane, loop-invariant offsets of the fast forward.  LDS layout of the
// workgroup: [K tile 0][K tile 1][V tile 0][V tile 1], TILEB bytes each, so
// that every read's parity and step offsets fit the 16-bit immediate.
//  kr[j]: K row reads (A operand of S^T).  Step (kk, c) reads row 32kk + n,
//         chunk (2c + hh) ^ swz_row(n) = 2c ^ (hh ^ swz_row(n)): byte
//         n*ROWB + (32c ^ 16 (hh ^ swz_row(n))) + kk*32*ROWB; the XOR only
//         reaches bits 4..7, so c and c + 8 differ by 256 bytes: kr[c % 8].
//  vr[j]: transposed V reads (A operand of O^T).  16-key block ke, column
//         block dt, half `hi`: row 16ke + 8hi + 4hh + i16/4, chunk
//         (4dt + W) ^ 4z with W = 2nh + (i16 & 3)/2 and z the row's swizzle
//         bits (independent of ke, hi): 4 (dt ^ z) + W; dt and dt + 4 differ
//         by 256 bytes: vr[dt % 4].
template <int DP> struct FwdLane {
    static constexpr int CPR = DP / 8, ROWB = DP * 2, NC = DP / 16, NDT = DP / 32;
    static constexpr int KC = NC < 8 ? NC : 8;
    static constexpr int VC = NDT < 4 ? NDT : 4;
    uint32_t kr[KC];
    uint32_t vr[VC];
    TileDma<DP, kFwdBN, 256, SWZ_ROW> dk;
    TileDma<DP, kFwdBN, 256, SWZ_TR> dv;

    __host__ __device__ void init(int lane, int w, int lk, int lv) {
        const int n = lane & 31, hh = lane >> 5, i16 = lane & 15, nh = (lane >> 4) & 1;
        const uint32_t y16 = 16u * (uint32_t)(hh ^ swz_row<CPR>(n));
#pragma unroll
        for (int j = 0; j < KC; ++j) kr[j] = (uint32_t)n * ROWB + ((32u * j) ^ y16);
        const int z = CPR >= 16 ? ((i16 >> 2) & 3) : ((i16 >> 3) & 1);
        const int W = 2 * nh + ((i16 & 3) >> 1);
#pragma unroll
        for (int j = 0; j < VC; ++j)
            vr[j] = (uint32_t)(4 * hh + (i16 >> 2)) * ROWB + 64u * (uint32_t)(j ^ z) + 16u * W + 8u * (i16 & 1);
        dk.init(lane, w, lk);
        dv.init(lane, w, lv);
    }
    // Byte offsets (relative to the LDS tile) of step (kk, c)'s K read and of
    // (ke, dt, hi)'s transposed V read.
    __host__ __device__ uint32_t k_off(int kk, int c) const { return kr[c % KC] + kk * 32 * ROWB + (c / KC) * 256; }
    __host__ __device__ uint32_t v_off(int ke, int dt, int hi) const {
        return vr[dt % VC] + (16 * ke + 8 * hi) * ROWB + (dt / VC) * 256;
    }
};

// Keep the O accumulators in VGPRs at this point.  Without it the compiler
// may give their loop-carried value an AGPR home (they do not all fit the
// VGPRs at D = 256) and then copy all of them to VGPRs and back around every
// tile's MFMAs.
template <int N> __device__ __forceinline__ void pin_vgpr(f32x16 (&acc)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("" : "+v"(acc[i]));
}

// One 64-key tile for this wave's 32 rows.  par: the buffer parity of the
// tile; need_mask (wave-uniform): some key of the tile is hidden from some row
// of the wave (this lane's row sees keys [vlo, vhi]).  issue_part(j), j < NPARTS, issues the
// next tile's loads; they are spread over the S^T steps.
template <int DP, class IssuePart>
__device__ __forceinline__ void fwd_tile(const FwdArgs& a, const char* smem, const FwdLane<DP>& ln, int par,
                                         bool need_mask, int kbase, int vlo, int vhi, const bf16x8 (&qf)[DP / 16],
                                         f32x16 (&oacc)[DP / 32], float& m_run, float& l_run,
                                         const IssuePart& issue_part) {
    constexpr int NPARTS = FwdLoads<DP>::NPARTS;
    constexpr int NC = DP / 16, NDT = DP / 32, NKK = kFwdBN / 32;
    constexpr int TILEB = kFwdBN * DP * 2;
    constexpr int PF = 4;  // LDS operand prefetch depth
    const int hh = (threadIdx.x & 63) >> 5;
    const char* kb = smem + par * TILEB;
    const char* vb = smem + (2 + par) * TILEB;

    // S^T = K Q^T.  The NKK accumulator chains are interleaved and the K
    // operands stream through a PF-deep register ring (the direct loads'
    // volatile asm statements are barriers to memory operations, so the LDS
    // reads keep their place between them).
    f32x16 s[NKK];
    {
        constexpr int NI = NKK * NC;
        auto kread = [&](int it) { return *reinterpret_cast<const bf16x8*>(kb + ln.k_off(it % NKK, it / NKK)); };
        bf16x8 ring[PF];
#pragma unroll
        for (int it = 0; it < PF; ++it) ring[it] = kread(it);
#pragma unroll
        for (int it = 0; it < NI; ++it) {
            const bf16x8 ka = ring[it % PF];
            if (it + PF < NI) ring[it % PF] = kread(it + PF);
            if (it < NKK)
                mfma_v_first(s[it], ka, qf[0]);
            else
                s[it % NKK] = mfma_bf16(ka, qf[it / NKK], s[it % NKK]);
            if ((it & 1) && (it >> 1) < NPARTS) issue_part(it >> 1);
        }
#pragma unroll
        for (int j = NI / 2; j < NPARTS; ++j) issue_part(j);
        static_assert(NKK == 2, "two accumulator chains");
    }

    if (need_mask) {  // keys outside [vlo, vhi]
        int hi = vhi - kbase, lo = vlo - kbase;
        // The bounds pass through an asm statement inside the branch, so the
        // compiler cannot hoist the selects out of it: tiles without masked
        // keys skip them.
        asm volatile("" : "+v"(hi), "+v"(lo));
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
    mx = half_max(mx) * a.scale_log2;
    // Lazy rescaling: the reference point m_run only moves (and O, l are
    // rescaled) when some row of the wave sees a max above m_run + 8, so
    // exp2 arguments stay <= 8 and P <= 256.  Any reference point gives
    // the same O = acc / l and LSE = m_run + log2(l); this one skips the
    // per-tile O multiply.
    if (__any(mx > m_run + kLazyRescale)) {
        const float m_new = fmaxf(m_run, mx);
        const float alpha = fast_exp2(m_run - (m_new == -INFINITY ? 0.f : m_new));
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
        pin_vgpr(oacc);
        m_run = m_new;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    float psum = 0.f;
    bf16x8 pb[2 * NKK];
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk)
#pragma unroll
        for (int e = 0; e < 2; ++e)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float p = fast_exp2(s[kk][8 * e + j] * a.scale_log2 - m_use);
                psum += p;
                pb[2 * kk + e][j] = (bf16)p;
            }
    l_run += psum;

    // O^T += V^T P^T, V^T operands through the same kind of register ring.
    {
        constexpr int NI = 2 * NKK * NDT;  // iteration = 16-key block ke x column block dt
        // The two 8-byte halves of each operand stream through rings of their
        // own and are joined at the MFMA: a ring of joined bf16x8 values made
        // the compiler copy every pair into a fresh register quadruple.
        auto vread = [&](int it, int hi) {
            return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(vb + ln.v_off(it / NDT, it % NDT, hi)));
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

// The next tile's loads (K, then V) into the buffer of parity npar; FAST:
// see issue_tile_j.
template <int DP, bool FAST>
struct FwdIssue {
    const FwdArgs& a;
    const FwdLane<DP>& ln;
    const bf16* K;
    const bf16* V;
    bf16* smem;
    uint32_t smem_addr;  // LDS byte address of smem
    int lk, lv, nrow, npar;
    __device__ __forceinline__ void operator()(int j) const {
        constexpr int PER = FwdLoads<DP>::PER, TILE = kFwdBN * DP;
        if (j < PER)
            issue_tile_j<FAST, DP, kFwdBN, 256, SWZ_ROW>(ln.dk, K, nrow, a.S, a.D, lk, smem + npar * TILE,
                                                         smem_addr + 2u * npar * TILE, j);
        else
            issue_tile_j<FAST, DP, kFwdBN, 256, SWZ_TR>(ln.dv, V, nrow, a.S, a.D, lv, smem + (2 + npar) * TILE,
                                                        smem_addr + 2u * (2 + npar) * TILE, j - PER);
    }
};

// One workgroup per 128-row query tile (longest causal rows first).
template <int DP, bool CAUSAL, bool FAST>
__global__ __launch_bounds__(256) void attn_fwd_bf16_fast(FwdArgs a) {
    constexpr int BN = kFwdBN, BM = kFwdBM;
    constexpr int NC = DP / 16, NDT = DP / 32, TILE = BN * DP;
    __shared__ __attribute__((aligned(1024))) bf16 smem[4 * TILE];

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
    FwdLane<DP> ln;
    ln.init(lane, wave_id(), lk, lv);

    const KeyVis vis{S, a.window, a.kv_len ? min(max(a.kv_len[b], 0), S) : S, CAUSAL};
    const int vlo = vis.lo(row), vhi = vis.hi(row);
    const int t0 = fast_q_lo(CAUSAL, a.window, qt);
    const int ntiles = t0 + fast_q_n(S, CAUSAL, a.window, qt);
    {
        const FwdIssue<DP, FAST> first{a, ln, K, Vg, smem, lds_addr(smem), lk, lv, t0 * BN, 0};
#pragma unroll
        for (int j = 0; j < FwdLoads<DP>::NPARTS; ++j) first(j);
    }

    bf16x8 qf[NC];
    fwd_load_q<DP>(Q, lq, row, S, D, qf);
    wait_vmcnt<0>();  // Q complete before the loop (direct loads are untracked)
    f32x16 oacc[NDT];
#pragma unroll
    for (int i = 0; i < NDT; ++i) oacc[i] = zero16();
    pin_vgpr(oacc);
    float m_run = -INFINITY, l_run = 0.f;

    for (int t = t0; t < ntiles; ++t) {
        const int par = (t - t0) & 1;
        // This wave's loads of tile t (issued one tile ago) have landed; after
        // the barrier every wave's have, and every wave is done with the
        // buffer tile t+1 streams into.
        wait_vmcnt<0>();
        lds_barrier();
        // Next tile's loads, spread over this tile's S^T steps; the last
        // tile re-loads tile t0 into the idle buffer (no branch in the
        // schedule; waited for before the end).
        const FwdIssue<DP, FAST> issue{a, ln, K, Vg, smem, lds_addr(smem), lk, lv, t + 1 < ntiles ? (t + 1) * BN : t0 * BN, par ^ 1};
        const int kbase = t * BN;
        if (wave_uniform(wrow0 < S && vis.any(wrow0, min(wrow0 + 31, S - 1), kbase, kbase + BN - 1))) {
            const bool need_mask = wave_uniform(!vis.all(wrow0, wrow0 + 31, kbase, kbase + BN - 1));
            fwd_tile<DP>(a, (const char*)smem, ln, par, need_mask, kbase, vlo, vhi, qf, oacc, m_run, l_run,
                             issue);
        } else {
#pragma unroll
            for (int j = 0; j < FwdLoads<DP>::NPARTS; ++j) issue(j);
        }
    }
    wait_vmcnt<0>();

    if (wrow0 >= S) return;
    const float l_tot = half_sum(l_run);
    if (row >= S) return;
    fwd_store_row<DP>(a, b, h, row, oacc, m_run, l_tot);
}

// Balanced launch: workgroup i = unit i / (B*Hq) of (batch, head) i % (B*Hq).
// Per (batch, head) the (query tile, key tile) iterations are flattened and
// cut into equal units, about one per CU; a query tile spread over several
// units leaves unnormalised fp32 partials (O, running max, sum) that
// attn_fwd_combine merges by log-sum-exp in slot order.
template <int DP, bool CAUSAL, bool FAST>
__global__ __launch_bounds__(256) void attn_fwd_bf16_split(FwdArgs a) {
    constexpr int BN = kFwdBN, BM = kFwdBM;
    constexpr int NC = DP / 16, NDT = DP / 32, TILE = BN * DP;
    __shared__ __attribute__((aligned(1024))) bf16 smem[4 * TILE];

    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6, n = lane & 31, hh = lane >> 5;
    const int S = a.S, D = a.D;
    const int bh = a.B * a.Hq, blk = xcd_block((int)blockIdx.x, (int)gridDim.x);  // XCD-major (see split16)
    const int unit = blk / bh, b = (blk % bh) / a.Hq, h = (blk % bh) % a.Hq, hk = h / a.group;

    const bf16* __restrict__ Q = (const bf16*)a.q + a.sq.at(b, h);
    const bf16* __restrict__ K = (const bf16*)a.k + a.sk.at(b, hk);
    const bf16* __restrict__ Vg = (const bf16*)a.v + a.sv.at(b, hk);
    const int lq = a.sq.s, lk = a.sk.s, lv = a.sv.s;
    FwdLane<DP> ln;
    ln.init(lane, wave_id(), lk, lv);

    const int W = a.window;
    const KeyVis vis{S, W, a.kv_len ? min(max(a.kv_len[b], 0), S) : S, CAUSAL};
    // This unit's range of the flattened (query tile, key tile) iterations.
    const FastTiles tiles{S, CAUSAL, W, a.group, 0};
    const int64_t g0 = unit_first(tiles, a.us, unit);
    const int niter = (int)(unit_first(tiles, a.us, unit + 1) - g0);
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
        const FwdIssue<DP, FAST> first{a, ln, K, Vg, smem, lds_addr(smem), lk, lv, next_key_tile() * BN, 0};
#pragma unroll
        for (int j = 0; j < FwdLoads<DP>::NPARTS; ++j) first(j);
    }

    bf16x8 qf[NC];
    f32x16 oacc[NDT];
    float m_run, l_run;
    int64_t qstart = fast_q_start(S, CAUSAL, W, qt);
    int qn = fast_q_n(S, CAUSAL, W, qt);
    int qlo = fast_q_lo(CAUSAL, W, qt);
    fwd_load_q<DP>(Q, lq, qt * BM + 32 * w + n, S, D, qf);
    wait_vmcnt<0>();  // Q complete before the loop (direct loads are untracked)

    // After a segment whose outputs this wave stored, the first tile's wait
    // leaves those stores in flight (see the end of the segment loop).
    bool stores_in_flight = false;
    for (int i = 0, first = 1;; first = 0) {
#pragma unroll
        for (int d = 0; d < NDT; ++d) oacc[d] = zero16();
        pin_vgpr(oacc);
        m_run = -INFINITY;
        l_run = 0.f;
        const int wrow0 = qt * BM + 32 * w, row = wrow0 + n;
        const int vlo = vis.lo(row), vhi = vis.hi(row);
        // Iterations of query tile qt inside this unit, then its output.
        const int seg_end = (int)min((int64_t)niter, qstart + qn - g0);
        for (; i < seg_end; ++i) {
            const int par = i & 1;
            // This wave's loads of buffer par have landed (as in
            // attn_fwd_bf16_fast).  Vector memory operations complete in
            // issue order, and the previous segment's epilogue issued at
            // least kEpilogueStores stores after this tile's loads and after
            // the Q reload: waiting until at most that many remain leaves the
            // stores draining behind this tile's work.
            if (stores_in_flight)
                wait_vmcnt<kEpilogueStores>();
            else
                wait_vmcnt<0>();
            stores_in_flight = false;
            lds_barrier();
            const FwdIssue<DP, FAST> issue{a, ln, K, Vg, smem, lds_addr(smem), lk, lv, i + 1 < niter ? next_key_tile() * BN : 0, par ^ 1};
            const int kbase = (qlo + (int)(g0 + i - qstart)) * BN;
            if (wave_uniform(wrow0 < S && vis.any(wrow0, min(wrow0 + 31, S - 1), kbase, kbase + BN - 1))) {
                const bool need_mask = wave_uniform(!vis.all(wrow0, wrow0 + 31, kbase, kbase + BN - 1));
                fwd_tile<DP>(a, (const char*)smem, ln, par, need_mask, kbase, vlo, vhi, qf, oacc, m_run, l_run,
                                 issue);
            } else {
#pragma unroll
                for (int j = 0; j < FwdLoads<DP>::NPARTS; ++j) issue(j);
            }
        }
        // The next segment's Q rows load first (qf is dead here), so that
        // they land while this segment's outputs are stored.
        const bool more = i < niter;
        const int nsl = tile_units(tiles, a.us, qt);  // of the segment just finished
        if (more) {
            ++qt;
            qstart = fast_q_start(S, CAUSAL, W, qt);
            qn = fast_q_n(S, CAUSAL, W, qt);
            qlo = fast_q_lo(CAUSAL, W, qt);
            fwd_load_q<DP>(Q, lq, qt * BM + 32 * w + n, S, D, qf);
        }
        // End of this unit's part of the query tile: a tile inside one unit
        // is written normalised; otherwise this unit's slot gets the
        // unnormalised partial (O, running max, sum) for attn_fwd_combine.
        // Every path below issues at least kEpilogueStores vector stores per
        // wave whose first row is in range (rows of a wave are all in range
        // or all out of range when FAST).
        if (wrow0 < S) {
            const float l_tot = half_sum(l_run);
            if (nsl <= 1) {
                if (row < S) fwd_store_row<DP>(a, b, h, row, oacc, m_run, l_tot);
            } else if (row < S) {
                const int64_t slot = (int64_t)(b * a.Hq + h) * 2 * a.us.units + 2 * unit + (first ? 0 : 1);
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
        if (!more) {
            wait_vmcnt<0>();  // the last tile's re-load has landed before the unit ends
            break;
        }
        stores_in_flight = FAST && DP == 256 && wave_uniform(wrow0 < S);
    }
}

// FAST (TileDma loads): every key tile whole (D == DP, S a multiple of 64).
template <int DP>
bool fwd_fast_dma(const AttnShape& s) {
    return s.D == DP && s.S % kFwdBN == 0;
}

template <int DP, bool CAUSAL, bool FAST>
void launch_fwd_fast_k(const AttnShape& s, const FwdArgs& a, bool split, unsigned units, hipStream_t st) {
    if (split)
        hipLaunchKernelGGL((attn_fwd_bf16_split<DP, CAUSAL, FAST>), dim3((unsigned)(units * s.B * s.Hq)), dim3(256), 0,
                           st, a);
    else
        hipLaunchKernelGGL((attn_fwd_bf16_fast<DP, CAUSAL, FAST>), dim3(a.n_qtiles, (unsigned)s.Hq, (unsigned)s.B),
                           dim3(256), 0, st, a);
}

template <int DP>
hipError_t launch_fwd_fast_t(const AttnShape& s, FwdArgs a, hipStream_t st) {
    a.n_qtiles = (int)((s.S + kFwdBM - 1) / kFwdBM);
    const bool split = a.part_o != nullptr;
    const unsigned units = split ? (unsigned)a.us.units : 0u;
    const bool fast = fwd_fast_dma<DP>(s);
    if (s.causal) {
        if (fast)
            launch_fwd_fast_k<DP, true, true>(s, a, split, units, st);
        else
            launch_fwd_fast_k<DP, true, false>(s, a, split, units, st);
    } else {
        if (fast)
            launch_fwd_fast_k<DP, false, true>(s, a, split, units, st);
        else
            launch_fwd_fast_k<DP, false, false>(s, a, split, units, st);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || !(split && a.any_split)) return e;
    return launch_fwd_combine(s, a, st);
}

}  // namespace
}  // namespace fwd
}  // namespace mft
