// Backward definitions shared by the general (attn_bwd.hip) and bf16 fast
// path (attn_bwd_fast.h) translation units.
#pragma once

#include "attn_common.h"
#include "attn_kernels.h"

namespace mft {
namespace bwd {

struct BwdArgs {
    const void* q;
    const void* k;
    const void* v;
    const void* o;
    const void* dO;
    const float* lse;
    float* dq;
    float* dk;
    float* dv;
    float* delta;
    float* part;
    float* stats;         // fast path: per 32-row block [32 x lse*log2e][32 x delta]
    int nqb_total;        // 32-row blocks per head (ceil(S / 32))
    int64_t part_stride;  // B*Hkv*S*D
    int64_t total_rows;   // B*Hq*S
    int S, D, Hq, Hkv, B, group, splits, heads_per_split;
    int n_ktiles, n_qtiles;   // key tiles of the dK/dV role, query tiles of the dQ role
    int n_kv_blocks, n_q_blocks;
    float scale, scale_log2;
    int vec_ok, vec4_ok;
    // fast path work units (see BwdPlan)
    int causal;
    int kv_chunk, q_chunk, kv_units, q_units;  // iterations per unit, units per (batch, head)
    float* kv_part;   // [kv_parts_max][2][B*Hkv*S*D]: dK then dV partials
    float* q_part;    // [q_parts_max][B*Hq*S*D]
    int64_t q_part_stride;  // B*Hq*S*D
};

// Fast-path work geometry (host and device use the same formulas).
// dK/dV: per (batch, kv head) the iterations (128-key tile kt, query head of
// the group, 32-row query block) are flattened kt-major; tile kt holds
// fast_kv_n(kt) of them starting at fast_kv_start(kt).  dQ: per (batch, query
// head) the iterations (128-row query tile qt, 64-key tile) are flattened
// qt-major.  Work units are equal chunks of these ranges.
__host__ __device__ inline int fast_nb(int S) { return (S + 31) / 32; }
__host__ __device__ inline int fast_kv_n(int S, int causal, int group, int kt) {
    return group * (causal ? fast_nb(S) - 4 * kt : fast_nb(S));
}
__host__ __device__ inline int64_t fast_kv_start(int S, int causal, int group, int kt) {
    const int64_t nb = fast_nb(S);
    return causal ? group * (kt * nb - 2 * (int64_t)kt * (kt - 1)) : (int64_t)group * nb * kt;
}
__host__ __device__ inline int fast_q_n(int S, int causal, int qt) {
    const int kend = causal ? min(S, 128 * (qt + 1)) : S;
    return (kend + 63) / 64;
}
__host__ __device__ inline int64_t fast_q_start(int S, int causal, int qt) {
    return causal ? (int64_t)qt * (qt + 1) : (int64_t)qt * ((S + 63) / 64);
}
// Units [first, last] of chunk size `chunk` that touch the range [start, start + n).
__host__ __device__ inline int fast_slots(int64_t start, int n, int64_t chunk) {
    return (int)((start + n - 1) / chunk - start / chunk + 1);
}

// Output rows of dK / dV for a split.
__device__ __forceinline__ void dkdv_out_rows(const BwdArgs& a, int b, int hk, int split, int key,
                                              float** dkp, float** dvp) {
    const int64_t off = ((int64_t)(b * a.Hkv + hk) * a.S + key) * a.D;
    if (a.splits == 1) {
        *dkp = a.dk + off;
        *dvp = a.dv + off;
    } else {
        *dkp = a.part + (int64_t)split * a.part_stride + off;
        *dvp = a.part + (int64_t)(a.splits + split) * a.part_stride + off;
    }
}

template <int NDT>
__device__ __forceinline__ void store_dkdv(const BwdArgs& a, float* dkp, float* dvp, int hh, const f32x16 (&dk)[NDT],
                                           const f32x16 (&dv)[NDT]) {
    const bool v4 = a.vec4_ok != 0;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d0 = 32 * dt + 8 * g + 4 * hh;
            store4<float>(dkp, d0, a.D, dk[dt][4 * g] * a.scale, dk[dt][4 * g + 1] * a.scale,
                          dk[dt][4 * g + 2] * a.scale, dk[dt][4 * g + 3] * a.scale, v4);
            store4<float>(dvp, d0, a.D, dv[dt][4 * g], dv[dt][4 * g + 1], dv[dt][4 * g + 2], dv[dt][4 * g + 3], v4);
        }
}

// ----------------------------------------------------------------- REDUCE
// dk = sum over splits of the dK partials (split order), same for dv.
static __global__ __launch_bounds__(256) void attn_bwd_reduce_kernel(BwdArgs a) {
    const int64_t n = a.part_stride;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        float sk = 0.f, sv = 0.f;
        for (int s = 0; s < a.splits; ++s) {
            sk += a.part[(int64_t)s * n + i];
            sv += a.part[(int64_t)(a.splits + s) * n + i];
        }
        a.dk[i] = sk;
        a.dv[i] = sv;
    }
}


// Launchers of the bf16 fast path (attn_bwd_fast.h), one per padded head dim.
hipError_t launch_bwd_fast_64(const AttnShape& s, const BwdArgs& a, int stages, hipStream_t st);
hipError_t launch_bwd_fast_128(const AttnShape& s, const BwdArgs& a, int stages, hipStream_t st);
hipError_t launch_bwd_fast_256(const AttnShape& s, const BwdArgs& a, int stages, hipStream_t st);

}  // namespace bwd
}  // namespace mft
