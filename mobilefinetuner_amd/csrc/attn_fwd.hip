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
#include "attn_common.h"
#include "attn_kernels.h"

namespace mft {
namespace {

struct FwdArgs {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* lse;
    int S, D, Hq, Hkv, group, n_qtiles;
    float scale_log2;  // softmax scale * log2(e)
    int vec_ok;        // D % (16 bytes / element size) == 0
    int vec4_ok;       // D % 4 == 0
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

    const T* __restrict__ Q = (const T*)a.q + (int64_t)(b * a.Hq + h) * S * D;
    const T* __restrict__ K = (const T*)a.k + (int64_t)(b * a.Hkv + hk) * S * D;
    const T* __restrict__ Vg = (const T*)a.v + (int64_t)(b * a.Hkv + hk) * S * D;

    V qf[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c)
        qf[c] = load_chunk<T>(Q + (int64_t)rowc * D, 2 * VEC * c + VEC * hh, D, row < S, vec_ok);

    f32x16 oacc[NDT];
#pragma unroll
    for (int i = 0; i < NDT; ++i) oacc[i] = zero16();
    float m_run = -INFINITY;  // running row max, log2-scaled units
    float l_run = 0.f;        // running sum over this half-wave's keys

    const int kend = CAUSAL ? min(S, m0 + BM) : S;
    const int ntiles = (kend + BN - 1) / BN;

    for (int t = 0; t < ntiles; ++t) {
        const int kbase = t * BN;
        __syncthreads();
        {   // stage K (row-major)
            constexpr int CPR = DP / VEC;
            for (int idx = tid; idx < BN * CPR; idx += NT) {
                const int rr = idx / CPR, c = idx - rr * CPR;
                const int key = kbase + rr;
                const int keyc = key < S ? key : S - 1;
                *reinterpret_cast<V*>(Ks + rr * L::KSTR + c * VEC) =
                    load_chunk<T>(K + (int64_t)keyc * D, c * VEC, D, key < S, vec_ok);
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
                    x[i] = load_chunk<bf16>((const bf16*)Vg + (int64_t)keyc * D, 8 * c, D, key < S, vec_ok);
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
                    load_chunk<T>(Vg + (int64_t)keyc * D, c * VEC, D, key < S, vec_ok);
            }
        }
        __syncthreads();

        // A wave with no valid rows, or whose rows all precede this tile, skips it.
        if (wrow0 >= S || (CAUSAL && kbase > wrow0 + 31)) continue;

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

        const bool need_mask = (CAUSAL && kbase + BN - 1 > wrow0) || (kbase + BN > S);
        float mx = -INFINITY;
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float x = s[kk][r];
                if (need_mask) {
                    const int key = kbase + 32 * kk + row_of_reg(r, hh);
                    if (key >= S || (CAUSAL && key > row)) x = -INFINITY;
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
    const float inv = 1.f / l_tot;
    T* O = (T*)a.o + (int64_t)(b * a.Hq + h) * S * D + (int64_t)row * D;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g)
            store4<T>(O, 32 * dt + 8 * g + 4 * hh, D, oacc[dt][4 * g] * inv, oacc[dt][4 * g + 1] * inv,
                      oacc[dt][4 * g + 2] * inv, oacc[dt][4 * g + 3] * inv, a.vec4_ok != 0);
    if (a.lse && hh == 0) a.lse[(int64_t)(b * a.Hq + h) * S + row] = (m_run + log2f(l_tot)) * kLn2;
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

template <int DP, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_fwd_bf16_fast(FwdArgs a) {
    constexpr int NW = 4, BN = 64, BM = 32 * NW, NT = 256;
    constexpr int CPR = DP / 8, NC = DP / 16, NDT = DP / 32, NKK = BN / 32;
    constexpr int TILE = BN * DP;                       // elements of one K or V tile
    constexpr int LOADS = 2 * BN * CPR / NT;            // direct loads per thread per tile
    constexpr int PF = 4;                               // LDS operand prefetch depth
    __shared__ __attribute__((aligned(1024))) bf16 smem[2 * 2 * TILE];

    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6, n = lane & 31, hh = lane >> 5;
    const int S = a.S, D = a.D;
    const int qt = a.n_qtiles - 1 - (int)blockIdx.x;
    const int h = blockIdx.y, b = blockIdx.z, hk = h / a.group;
    const int m0 = qt * BM;
    const int wrow0 = m0 + 32 * w;
    const int row = wrow0 + n;
    const int rowc = row < S ? row : S - 1;

    const bf16* __restrict__ Q = (const bf16*)a.q + (int64_t)(b * a.Hq + h) * S * D;
    const bf16* __restrict__ K = (const bf16*)a.k + (int64_t)(b * a.Hkv + hk) * S * D;
    const bf16* __restrict__ Vg = (const bf16*)a.v + (int64_t)(b * a.Hkv + hk) * S * D;

    const int kend = CAUSAL ? min(S, m0 + BM) : S;
    const int ntiles = (kend + BN - 1) / BN;
    issue_tile<DP, BN, NT, SWZ_ROW>(K, 0, S, D, smem);
    issue_tile<DP, BN, NT, SWZ_TR>(Vg, 0, S, D, smem + TILE);

    bf16x8 qf[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c)
        qf[c] = load_chunk<bf16>(Q + (int64_t)rowc * D, 16 * c + 8 * hh, D, row < S, true);

    f32x16 oacc[NDT];
#pragma unroll
    for (int i = 0; i < NDT; ++i) oacc[i] = zero16();
    float m_run = -INFINITY, l_run = 0.f;

    const int g16 = lane >> 4, i16 = lane & 15, nh = g16 & 1;
    for (int t = 0; t < ntiles; ++t) {
        const bf16* Kb = smem + (t & 1) * 2 * TILE;
        const bf16* Vb = Kb + TILE;
        if (t + 1 < ntiles) {
            lds_barrier();  // every wave is done with the buffer tile t+1 reuses
            bf16* nb = smem + ((t + 1) & 1) * 2 * TILE;
            issue_tile<DP, BN, NT, SWZ_ROW>(K, (t + 1) * BN, S, D, nb);
            issue_tile<DP, BN, NT, SWZ_TR>(Vg, (t + 1) * BN, S, D, nb + TILE);
            lds_barrier_vm<LOADS>();  // tile t has landed (all waves), tile t+1 in flight
        } else {
            lds_barrier_vm<0>();
        }
        const int kbase = t * BN;
        if (wrow0 >= S || (CAUSAL && kbase > wrow0 + 31)) continue;

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
            }
            pin_read_ahead<NI, PF, 1>();
        }

        // Keys past `lim` (causal: this lane's row; always: S-1) are masked,
        // as selects so the hot loop stays branch-free.
        if ((CAUSAL && kbase + BN - 1 > wrow0) || (kbase + BN > S)) {
            const int lim = (CAUSAL ? min(row, S - 1) : S - 1) - kbase;
#pragma unroll
            for (int kk = 0; kk < NKK; ++kk)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    s[kk][r] = 32 * kk + row_of_reg(r, hh) > lim ? -INFINITY : s[kk][r];
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

    if (wrow0 >= S) return;
    const float l_tot = l_run + other_half(l_run);
    if (row >= S) return;
    const float inv = 1.f / l_tot;
    bf16* O = (bf16*)a.o + (int64_t)(b * a.Hq + h) * S * D + (int64_t)row * D;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g)
            store4<bf16>(O, 32 * dt + 8 * g + 4 * hh, D, oacc[dt][4 * g] * inv, oacc[dt][4 * g + 1] * inv,
                         oacc[dt][4 * g + 2] * inv, oacc[dt][4 * g + 3] * inv, true);
    if (a.lse && hh == 0) a.lse[(int64_t)(b * a.Hq + h) * S + row] = (m_run + log2f(l_tot)) * kLn2;
}

template <int DP>
hipError_t launch_fwd_fast(const AttnShape& s, FwdArgs a, hipStream_t st) {
    a.n_qtiles = (int)((s.S + 127) / 128);
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

hipError_t launch_attn_fwd(const AttnShape& s, const void* q, const void* k, const void* v, void* o,
                           float* lse, hipStream_t st) {
    FwdArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = o;
    a.lse = lse;
    a.S = (int)s.S;
    a.D = (int)s.D;
    a.Hq = (int)s.Hq;
    a.Hkv = (int)s.Hkv;
    a.group = (int)(s.Hq / s.Hkv);
    a.n_qtiles = 0;
    a.scale_log2 = s.scale * kLog2e;
    a.vec_ok = (s.D % (s.bf16 ? 8 : 4)) == 0;
    a.vec4_ok = (s.D % 4) == 0;
    return s.bf16 ? launch_fwd_dispatch<bf16>(s, a, st) : launch_fwd_dispatch<float>(s, a, st);
}

}  // namespace mft
