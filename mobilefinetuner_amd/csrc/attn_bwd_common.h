// Backward definitions shared by the general (attn_bwd.hip) and bf16 fast
// path (attn_bwd_fast.h) translation units.
#pragma once

#include "attn_common.h"
#include "attn_geometry.h"
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
    int window;         // causal sliding window, 0 = none
    const int* kv_len;  // [B] valid keys per batch, or null
    Strides sq, sk, sv, so, sdo, sdq, sdk, sdv;  // operand layouts
    // fast path work units (see BwdPlan)
    int causal;
    UnitSplit kv_us, q_us;  // work units per (batch, kv head), per (batch, query head)
    float* kv_part;   // [B*Hkv][2*kv_us.units][dK, dV][128][D] partial tiles (split_slot)
    float* q_part;    // [B*Hq][2*q_us.units][128][D] partial dQ tiles (split_slot)
    int64_t q_part_stride;  // B*Hq*S*D
    int kv_parts_max, q_parts_max;  // most units of one tile (REDUCE runs when either is > 1)
    // mask mode (AttnShape::masked; general kernels only): lse holds (row max,
    // ln sum) pairs
    MaskView m0, m1;
    int mask_causal;
};

// Work geometry of the fast path (attn_geometry.h), shared with the forward.
using ::mft::fast_kv_n;
using ::mft::fast_kv_nqb;
using ::mft::fast_kv_start;
using ::mft::fast_nb;
using ::mft::fast_q_lo;
using ::mft::fast_q_n;
using ::mft::fast_q_start;
using ::mft::fast_q_total;
using ::mft::FastTiles;
using ::mft::split_slot;
using ::mft::tile_units;
using ::mft::unit_first;
using ::mft::UnitSplit;

// Operand addressing of the fast kernels: STRIDED = false is the contiguous
// [B, H, S, D] layout with offsets formed from the shape alone (no stride
// state kept in registers); STRIDED = true follows the operand's Strides.
template <bool STRIDED>
__device__ __forceinline__ int64_t op_base(const Strides& st, int b, int h, int H, int S, int D) {
    if constexpr (STRIDED) return st.at(b, h);
    else return (int64_t)(b * H + h) * S * D;
}
template <bool STRIDED> __device__ __forceinline__ int op_ld(const Strides& st, int D) {
    if constexpr (STRIDED) return st.s;
    else return D;
}

// Key visibility of batch b (see KeyVis).
__device__ __forceinline__ KeyVis key_vis(const BwdArgs& a, int b, bool causal) {
    return KeyVis{a.S, a.window, a.kv_len ? min(max(a.kv_len[b], 0), a.S) : a.S, causal};
}

// Output rows of dK / dV for a split.
__device__ __forceinline__ void dkdv_out_rows(const BwdArgs& a, int b, int hk, int split, int key,
                                              float** dkp, float** dvp) {
    const int64_t off = ((int64_t)(b * a.Hkv + hk) * a.S + key) * a.D;  // split partials: contiguous
    if (a.splits == 1) {
        *dkp = a.dk + a.sdk.at(b, hk) + (int64_t)key * a.sdk.s;
        *dvp = a.dv + a.sdv.at(b, hk) + (int64_t)key * a.sdv.s;
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

// A wave's 32-row fp32 accumulator tile in the 32x32 MFMA layout (lane
// n = l % 32 holds row n; register 4g + i of column tile dt holds column
// 32dt + 8g + 4hh + i, hh = l / 32), stored row-contiguously through a
// per-wave LDS staging area of 32 rows x 32*DTR columns (4 KiB x DTR).
// Stored from the registers directly, each vector store writes 32 rows x 32
// bytes; after the staging each writes 64 / (8 DTR) whole row runs of
// 128 DTR bytes.  Row r goes to dst + r*ld for all 32 rows and 32*NDT
// columns (16-byte aligned rows; callers take another path for partial
// tiles).  The staging area's 16-byte chunks are XOR-swizzled by row, so
// that the 32 rows of one register write reach distinct chunks.
// Wave-local: the caller makes the area free (a barrier, when other waves
// used it) and keeps other waves out of it until the call returns.
template <int NDT, int DTR>
__device__ __forceinline__ void store_acc32_staged(char* stage, float* dst, int64_t ld, const f32x16 (&acc)[NDT],
                                                   float scale) {
    static_assert(NDT % DTR == 0 && (DTR == 1 || DTR == 2 || DTR == 4), "staging rounds");
    constexpr int CPRR = 8 * DTR, RB = 16 * CPRR, RPI = 64 / CPRR;  // chunks, bytes per row; rows per store
    constexpr int NB = 4;                                            // reads in flight before their stores
    // The lane's offsets are formed here: left to itself, the compiler hoists
    // them out of the caller's loops into registers it then has to spill.
    int lane = threadIdx.x & 63;
    asm volatile("" : "+v"(lane));
    const int n = lane & 31, hh = lane >> 5;
    const int rrow = lane / CPRR, c = lane % CPRR;
    char* wr = stage + n * RB;
    const char* rd = stage + rrow * RB;
    float* out = dst + rrow * ld + 4 * c;
#pragma unroll
    for (int r0 = 0; r0 < NDT / DTR; ++r0) {
        asm volatile("" ::: "memory");  // the last round's reads precede these writes
#pragma unroll
        for (int dl = 0; dl < DTR; ++dl)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x16& t = acc[DTR * r0 + dl];
                const f32x4 v = {t[4 * g] * scale, t[4 * g + 1] * scale, t[4 * g + 2] * scale, t[4 * g + 3] * scale};
                *reinterpret_cast<f32x4*>(wr + 16 * ((8 * dl + 2 * g + hh) ^ (n & (CPRR - 1)))) = v;
            }
        asm volatile("" ::: "memory");  // LDS executes a wave's operations in order
#pragma unroll
        for (int k0 = 0; k0 < 32 / RPI; k0 += NB) {
            f32x4 v[NB];
#pragma unroll
            for (int k = 0; k < NB; ++k)
                v[k] = *reinterpret_cast<const f32x4*>(rd + (k0 + k) * RPI * RB +
                                                        16 * (c ^ ((RPI * (k0 + k) + rrow) & (CPRR - 1))));
#pragma unroll
            for (int k = 0; k < NB; ++k) *reinterpret_cast<f32x4*>(out + (k0 + k) * RPI * ld + 32 * DTR * r0) = v[k];
        }
    }
    asm volatile("" ::: "memory");
}

// ----------------------------------------------------------------- REDUCE
// dk = sum over splits of the dK partials (split order), same for dv.  The
// partials are contiguous [B, Hkv, S, D]; dk, dv follow their layouts.
static __global__ __launch_bounds__(256) void attn_bwd_reduce_kernel(BwdArgs a) {
    const int64_t n = a.part_stride;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        float sk = 0.f, sv = 0.f;
        for (int s = 0; s < a.splits; ++s) {
            sk += a.part[(int64_t)s * n + i];
            sv += a.part[(int64_t)(a.splits + s) * n + i];
        }
        const int64_t d = i % a.D, row = (i / a.D) % a.S, bh = i / ((int64_t)a.D * a.S);
        const int bb = (int)(bh / a.Hkv), hk = (int)(bh % a.Hkv);
        a.dk[a.sdk.at(bb, hk) + row * a.sdk.s + d] = sk;
        a.dv[a.sdv.at(bb, hk) + row * a.sdv.s + d] = sv;
    }
}


// Launchers of the bf16 fast path (attn_bwd_fast.h), one per padded head dim.
hipError_t launch_bwd_fast_64(const AttnShape& s, const BwdArgs& a, int stages, hipStream_t st);
hipError_t launch_bwd_fast_128(const AttnShape& s, const BwdArgs& a, int stages, hipStream_t st);
hipError_t launch_bwd_fast_256(const AttnShape& s, const BwdArgs& a, int stages, hipStream_t st);

}  // namespace bwd

namespace f32 {
// The fp32 fast backward (attn_f32_fast.h).
hipError_t launch_bwd_fast(const AttnShape& s, const bwd::BwdArgs& a, int stages, hipStream_t st);
}  // namespace f32

namespace bwd {

}  // namespace bwd
}  // namespace mft
