// Query rows that see no key at all (key padding).
//
// With key padding (valid keys j < len of each batch) a query row can be left
// without a visible key: every row when len = 0, and with a causal sliding
// window of W keys every row i >= len + W - 1.  The reference still gives
// such a row a defined result: its scores are scale q.k plus the -1e10
// entries of the masks (graph/gemma_model.cpp:481-505: add(base mask), then
// add(pad mask)), so a key hidden by exactly one of the two masks scores
// -1e10 and a key hidden by both -2e10; the softmax (core/ops.cpp softmax,
// max-subtracted) is then exactly uniform over the keys hidden once,
//   T_i = [tlo(i), thi(i)] u [0, len),  |T_i| = thi - tlo + 1 + len,
// the keys the base mask lets through (all padded) plus the unpadded keys the
// base mask hides (scale q.k is far below the 1e10 spacing of 1024, so it
// vanishes from the sum).  Its output is the mean of V over T_i, independent
// of q, and its backward is that of P_ij = 1 / |T_i| on T_i:
//   dS_ij = (dO_i . v_j - delta_i) / |T_i|,  delta_i = dO_i . O_i
//   dq_i = scale sum_j dS_ij k_j,  dk_j += scale dS_ij q_i,  dv_j += dO_i / |T_i|.
// The main kernels leave these rows at O = 0, LSE = +inf, P = 0 (no visible
// key); the kernels below write the reference's values afterwards.  They run
// only when the caller passes key lengths, do O(rows x |T_i| x D) work, and
// skip rows whose dO is all zero (training with the padded positions' loss
// masked out: their gradients are exactly zero).
#include "attn_common.h"
#include "attn_kernels.h"

namespace mft {
namespace {

struct MaskedArgs {
    const void* q;
    const void* k;
    const void* v;
    void* o;          // forward output (overwritten on masked rows)
    const void* dO;
    float* dq;
    float* dk;
    float* dv;
    float* row_delta;  // [B*Hq*S] delta of masked rows (backward scratch)
    int* row_active;   // [B*Hq*S] masked row with non-zero dO (backward scratch)
    const int* kv_len;
    int B, Hq, Hkv, S, D, group, window, causal;
    float scale;
    Strides sq, sk, sv, so, sdo, sdq, sdk, sdv;  // operand layouts
};

// Rows [first, S) of a batch see no key; T_i as above.
struct MaskedRows {
    int S, W, len;
    bool causal;
    __device__ int first() const { return len <= 0 ? 0 : (W > 0 ? min(S, len + W - 1) : S); }
    __device__ int tlo(int i) const { return W > 0 ? max(i - W + 1, 0) : 0; }
    __device__ int thi(int i) const { return causal ? i : S - 1; }
    __device__ int count(int i) const { return thi(i) - tlo(i) + 1 + len; }
};

__device__ __forceinline__ MaskedRows masked_rows(const MaskedArgs& a, int b) {
    return MaskedRows{a.S, a.window, min(max(a.kv_len[b], 0), a.S), a.causal != 0};
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
    return x;
}

template <typename T> __device__ __forceinline__ float ld(const T* p) { return (float)*p; }

// Forward: O_i = mean of V over T_i for every masked row, all query heads of
// the kv head.  Workgroup = (64-row chunk, batch x kv head); thread = column.
// The sum over [0, len) is formed once per workgroup, the window part is
// rolled along the rows; both in double.
template <typename T>
__global__ __launch_bounds__(256) void attn_fwd_masked_rows(MaskedArgs a) {
    const int S = a.S, D = a.D, d = threadIdx.x;
    const int bk = blockIdx.y, b = bk / a.Hkv, hk = bk % a.Hkv;
    const MaskedRows mr = masked_rows(a, b);
    const int r0 = max((int)blockIdx.x * 64, mr.first()), r1 = min((int)blockIdx.x * 64 + 64, S);
    if (r0 >= r1 || d >= D) return;
    const T* V = (const T*)a.v + a.sv.at(b, hk) + d;
    const int64_t lv = a.sv.s;
    double pre = 0.0;
    for (int j = 0; j < mr.len; ++j) pre += ld(V + (int64_t)j * lv);
    int lo = mr.tlo(r0), hi = mr.thi(r0);
    double win = 0.0;
    for (int j = lo; j <= hi; ++j) win += ld(V + (int64_t)j * lv);
    for (int i = r0; i < r1; ++i) {
        const int nlo = mr.tlo(i), nhi = mr.thi(i);
        for (; hi < nhi; ++hi) win += ld(V + (int64_t)(hi + 1) * lv);
        for (; lo < nlo; ++lo) win -= ld(V + (int64_t)lo * lv);
        const float o = (float)((pre + win) / (double)mr.count(i));
        for (int h = hk * a.group; h < (hk + 1) * a.group; ++h)
            ((T*)a.o)[a.so.at(b, h) + (int64_t)i * a.so.s + d] = (T)o;
    }
}

// This lane's columns lane + 64 c (c < 4, D <= 256) of a row.
template <typename T>
__device__ __forceinline__ void load_row4(const T* row, int D, float (&x)[4]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int c = 0; c < 4; ++c) x[c] = lane + 64 * c < D ? (float)row[lane + 64 * c] : 0.f;
}
__device__ __forceinline__ float dot4(const float (&x)[4], const float (&y)[4]) {
    return x[0] * y[0] + x[1] * y[1] + x[2] * y[2] + x[3] * y[3];
}

// Backward, dQ of masked rows (and the row terms the dK/dV pass reads): a
// workgroup per (64 rows, batch x query head), each wave 16 rows in turn.
// Workgroups without masked rows return at once (the common case).
template <typename T>
__device__ void masked_dq_row(const MaskedArgs& a, const MaskedRows& mr, int b, int h, int i);

template <typename T>
__global__ __launch_bounds__(256) void attn_bwd_masked_dq(MaskedArgs a) {
    const int bh = blockIdx.y, b = bh / a.Hq, h = bh % a.Hq;
    const MaskedRows mr = masked_rows(a, b);
    const int r0 = max((int)blockIdx.x * 64 + 16 * (int)(threadIdx.x >> 6), mr.first());
    const int r1 = min((int)blockIdx.x * 64 + 16 * (int)(threadIdx.x >> 6) + 16, a.S);
    for (int i = r0; i < r1; ++i) masked_dq_row<T>(a, mr, b, h, i);
}

template <typename T>
__device__ void masked_dq_row(const MaskedArgs& a, const MaskedRows& mr, int b, int h, int i) {
    const int S = a.S, D = a.D, lane = threadIdx.x & 63, hk = h / a.group;
    const int64_t ri = ((int64_t)b * a.Hq + h) * S + i;  // row-term index (contiguous scratch)
    float g[4], o[4];
    load_row4((const T*)a.dO + a.sdo.at(b, h) + (int64_t)i * a.sdo.s, D, g);
    load_row4((const T*)a.o + a.so.at(b, h) + (int64_t)i * a.so.s, D, o);
    const bool nz = __any(g[0] != 0.f || g[1] != 0.f || g[2] != 0.f || g[3] != 0.f);
    const float dl = wave_sum(dot4(g, o));
    if (lane == 0) {
        a.row_active[ri] = nz ? 1 : 0;
        a.row_delta[ri] = dl;
    }
    if (!nz) return;  // dq_i = 0, as the main pass left it
    const T* K = (const T*)a.k + a.sk.at(b, hk);
    const T* V = (const T*)a.v + a.sv.at(b, hk);
    const float inv_c = 1.f / (float)mr.count(i);
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    auto key = [&](int j) {
        float vj[4], kj[4];
        load_row4(V + (int64_t)j * a.sv.s, D, vj);
        load_row4(K + (int64_t)j * a.sk.s, D, kj);
        const float ds = (wave_sum(dot4(g, vj)) - dl) * inv_c;
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] += ds * kj[c];
    };
    for (int j = 0; j < mr.len; ++j) key(j);
    for (int j = mr.tlo(i); j <= mr.thi(i); ++j) key(j);
    float* dq = a.dq + a.sdq.at(b, h) + (int64_t)i * a.sdq.s;
#pragma unroll
    for (int c = 0; c < 4; ++c)
        if (lane + 64 * c < D) dq[lane + 64 * c] = acc[c] * a.scale;
}

// Backward, dK/dV contributions of masked rows, added to what the main pass
// wrote: a workgroup per (64 keys, batch x kv head), each wave 16 keys in
// turn.  The rows that hold key j in T_i: all masked rows for j < len, else
// rows j .. j + W - 1 (causal window) among the masked ones; active rows are
// found 64 at a time by ballot.  Batches without masked rows return at once.
template <typename T>
__device__ void masked_dkdv_key(const MaskedArgs& a, const MaskedRows& mr, int b, int hk, int j);

template <typename T>
__global__ __launch_bounds__(256) void attn_bwd_masked_dkdv(MaskedArgs a) {
    const int bk = blockIdx.y, b = bk / a.Hkv, hk = bk % a.Hkv;
    const MaskedRows mr = masked_rows(a, b);
    if (mr.first() >= a.S) return;
    const int j0 = (int)blockIdx.x * 64 + 16 * (int)(threadIdx.x >> 6);
    for (int j = j0; j < min(j0 + 16, a.S); ++j) masked_dkdv_key<T>(a, mr, b, hk, j);
}

template <typename T>
__device__ void masked_dkdv_key(const MaskedArgs& a, const MaskedRows& mr, int b, int hk, int j) {
    const int S = a.S, D = a.D, lane = threadIdx.x & 63;
    int i_lo = mr.first(), i_hi = S - 1;
    if (j >= mr.len) {
        if (mr.causal) i_lo = max(i_lo, j);
        if (mr.W > 0) i_hi = min(i_hi, j + mr.W - 1);
    }
    if (i_lo > i_hi) return;
    float vj[4];
    load_row4((const T*)a.v + a.sv.at(b, hk) + (int64_t)j * a.sv.s, D, vj);
    float ak[4] = {0.f, 0.f, 0.f, 0.f}, av[4] = {0.f, 0.f, 0.f, 0.f};
    bool any = false;
    for (int h = hk * a.group; h < (hk + 1) * a.group; ++h) {
        const int64_t bh = (int64_t)b * a.Hq + h;
        for (int c0 = i_lo; c0 <= i_hi; c0 += 64) {
            const int ic = c0 + lane;
            unsigned long long m = __ballot(ic <= i_hi && a.row_active[bh * S + ic] != 0);
            while (m) {
                const int i = c0 + __builtin_ctzll(m);
                m &= m - 1;
                any = true;
                const int64_t ri = bh * S + i;
                float g[4], q[4];
                load_row4((const T*)a.dO + a.sdo.at(b, h) + (int64_t)i * a.sdo.s, D, g);
                load_row4((const T*)a.q + a.sq.at(b, h) + (int64_t)i * a.sq.s, D, q);
                const float inv_c = 1.f / (float)mr.count(i);
                const float ds = (wave_sum(dot4(g, vj)) - a.row_delta[ri]) * inv_c;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    av[c] += g[c] * inv_c;
                    ak[c] += ds * q[c];
                }
            }
        }
    }
    if (!any) return;
    float* dk = a.dk + a.sdk.at(b, hk) + (int64_t)j * a.sdk.s;
    float* dv = a.dv + a.sdv.at(b, hk) + (int64_t)j * a.sdv.s;
#pragma unroll
    for (int c = 0; c < 4; ++c)
        if (lane + 64 * c < D) {
            dk[lane + 64 * c] += ak[c] * a.scale;
            dv[lane + 64 * c] += av[c];
        }
}

MaskedArgs masked_args(const AttnShape& s) {
    MaskedArgs a{};
    a.kv_len = s.kv_len;
    a.B = (int)s.B;
    a.Hq = (int)s.Hq;
    a.Hkv = (int)s.Hkv;
    a.S = (int)s.S;
    a.D = (int)s.D;
    a.group = (int)(s.Hq / s.Hkv);
    a.window = s.window;
    a.causal = s.causal ? 1 : 0;
    a.scale = s.scale;
    a.sq = s.q;
    a.sk = s.k;
    a.sv = s.v;
    a.so = s.o;
    a.sdo = s.dO;
    a.sdq = s.dq;
    a.sdk = s.dk;
    a.sdv = s.dv;
    return a;
}

}  // namespace

size_t masked_rows_workspace_bytes(const AttnShape& s) {
    if (!s.kv_len) return 0;
    const size_t rows = static_cast<size_t>(s.B * s.Hq * s.S);
    return ((rows * 4 + 255) & ~static_cast<size_t>(255)) * 2;
}

hipError_t launch_fwd_masked_rows(const AttnShape& s, const void* v, void* o, hipStream_t st) {
    if (!s.kv_len) return hipSuccess;
    MaskedArgs a = masked_args(s);
    a.v = v;
    a.o = o;
    const dim3 grid((unsigned)((s.S + 63) / 64), (unsigned)(s.B * s.Hkv));
    if (s.bf16)
        hipLaunchKernelGGL(attn_fwd_masked_rows<bf16>, grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL(attn_fwd_masked_rows<float>, grid, dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_bwd_masked_rows(const AttnShape& s, const void* q, const void* k, const void* v, const void* o,
                                  const void* dO, float* dq, float* dk, float* dv, void* scratch, hipStream_t st) {
    if (!s.kv_len) return hipSuccess;
    MaskedArgs a = masked_args(s);
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = const_cast<void*>(o);
    a.dO = dO;
    a.dq = dq;
    a.dk = dk;
    a.dv = dv;
    const size_t half = masked_rows_workspace_bytes(s) / 2;
    a.row_delta = static_cast<float*>(scratch);
    a.row_active = reinterpret_cast<int*>(static_cast<char*>(scratch) + half);
    const dim3 gq((unsigned)((s.S + 63) / 64), (unsigned)(s.B * s.Hq));
    const dim3 gk((unsigned)((s.S + 63) / 64), (unsigned)(s.B * s.Hkv));
    if (s.bf16) {
        hipLaunchKernelGGL(attn_bwd_masked_dq<bf16>, gq, dim3(256), 0, st, a);
        hipLaunchKernelGGL(attn_bwd_masked_dkdv<bf16>, gk, dim3(256), 0, st, a);
    } else {
        hipLaunchKernelGGL(attn_bwd_masked_dq<float>, gq, dim3(256), 0, st, a);
        hipLaunchKernelGGL(attn_bwd_masked_dkdv<float>, gk, dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

}  // namespace mft
