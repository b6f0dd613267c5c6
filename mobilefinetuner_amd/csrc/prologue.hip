// Fused q/k prologue of the attention: y = rope(norm(x)) per row, and its
// backward (C ABI in include/mft/prologue.h).
//
// Two lane layouts.  Head dims 128, 256 and 512 with 16-byte-aligned rows take
// the 16-byte-lane kernels (prologue_*_vec below): a row spans D*size/16
// lanes, each holding elements of the first half and their rotate-half
// partners.  Other head dims and unaligned rows take one wave per row
// (b, h, s), each wave RPW rows with all loads issued first; lane l owns the
// elements p = (l + 64 j) * V + e (j < NJ, e < V) of each half.  Either way a
// RoPE pair (p, p + D/2) never leaves its lane.  The row's sum of squares is
// a shuffle reduction in the one-wave kernels (wave_sum) and an in-register
// DPP / permlane reduction in the 16-byte-lane kernels (group_sum).
//
// Arithmetic follows the reference operators step for step, without fused
// multiply-adds (fp contract off):
//   rms_norm         core/ops.cpp:1693-1705   double sum of squares, float
//                                             rms, (x / rms) * (1 + w)
//   rms_norm_affine  core/ops.cpp:1739-1744   float inv_rms, x * inv_rms * w
//   apply_rope       core/ops.cpp:2360-2389   angle = float(pos) * freq,
//                                             freq = 1 / theta^(2d/D) (host
//                                             table, the same float powf)
//   ApplyRoPEBackward core/backward_functions.cpp:757-768
//   RMSNorm(Affine)Backward core/backward_functions.cpp:510-528, 548-567,
//                                             in double, as there.
// cosf/sinf are the device library's (the reference calls the host libm's);
// both are faithfully rounded, so y agrees to a few ulp.  The 16-byte-lane
// forward divides by rms as div_by (one correctly rounded reciprocal per row
// and a correction step per element), which gives the IEEE quotient.
//
// dL/dw: each backward workgroup (4 waves) sums its rows' terms (float,
// fixed order) into one [D] partial, and a second kernel adds the partials in
// a fixed order (in double).  The partition depends only on the shape, so dw
// is deterministic.
#include <hip/hip_runtime.h>

#include "attn_common.h"
#include "prologue_kernels.h"

namespace mft {
namespace {

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// V consecutive elements of type T, converted to / from float.
template <typename T, int V> struct Vec {
    typedef T raw __attribute__((ext_vector_type(V)));
    __device__ static void load(const T* p, float* out) {
        if constexpr (V == 1) {
            out[0] = (float)*p;
        } else {
            const raw r = *reinterpret_cast<const raw*>(p);
#pragma unroll
            for (int e = 0; e < V; ++e) out[e] = (float)r[e];
        }
    }
    __device__ static void store(T* p, const float* in) {
        if constexpr (V == 1) {
            *p = (T)in[0];
        } else {
            raw r;
#pragma unroll
            for (int e = 0; e < V; ++e) r[e] = (T)in[e];
            *reinterpret_cast<raw*>(p) = r;
        }
    }
};

struct RowAddr {
    int64_t b, h;
    int s;
};

__device__ __forceinline__ RowAddr row_addr(const PrologueArgs& a, int64_t r) {
    const int s = (int)(r % a.S);
    const int64_t bh = r / a.S;
    return RowAddr{bh / a.H, bh % a.H, s};
}

// First element of chunk j of this lane in a half.
template <int V> __device__ __forceinline__ int elem(int lane, int j) { return (lane + 64 * j) * V; }

constexpr int FWD_RPW = 2;

template <typename T, int NJ, int V>
__global__ __launch_bounds__(256) void prologue_fwd_kernel(PrologueArgs a) {
#pragma clang fp contract(off)
    constexpr int E = NJ * V;  // elements per lane per half
    constexpr int RPW = FWD_RPW;
    const int lane = threadIdx.x & 63;
    const int half = a.D / 2;
    const int64_t r0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW;
    float x1[RPW][E], x2[RPW][E];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const int64_t r = r0 + i;
        const RowAddr ra = row_addr(a, r < a.rows ? r : 0);
        const T* xr = (const T*)a.x + a.sx.at(ra.b, ra.h) + (int64_t)ra.s * a.sx.s;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int p = elem<V>(lane, j);
            if (r < a.rows && p < half) {
                Vec<T, V>::load(xr + p, &x1[i][j * V]);
                Vec<T, V>::load(xr + p + half, &x2[i][j * V]);
            } else {
#pragma unroll
                for (int e = 0; e < V; ++e) x1[i][j * V + e] = x2[i][j * V + e] = 0.f;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const int64_t r = r0 + i;
        if (r >= a.rows) break;  // wave-uniform
        const RowAddr ra = row_addr(a, r);
        T* yr = (T*)a.y + a.sy.at(ra.b, ra.h) + (int64_t)ra.s * a.sy.s;
        if (a.norm != PROLOGUE_NORM_NONE) {
            double ss = 0.0;
#pragma unroll
            for (int k = 0; k < E; ++k) ss += (double)x1[i][k] * (double)x1[i][k] + (double)x2[i][k] * (double)x2[i][k];
            ss = wave_sum(ss);
            if (a.norm == PROLOGUE_NORM_GEMMA) {
                const float rms = (float)sqrt(ss / (double)a.D + (double)a.eps);
#pragma unroll
                for (int j = 0; j < NJ; ++j)
#pragma unroll
                    for (int e = 0; e < V; ++e) {
                        const int p = elem<V>(lane, j) + e, k = j * V + e;
                        if (p < half) {
                            x1[i][k] = (x1[i][k] / rms) * (1.0f + a.w[p]);
                            x2[i][k] = (x2[i][k] / rms) * (1.0f + a.w[p + half]);
                        }
                    }
            } else {
                const float inv = (float)(1.0 / sqrt(ss / (double)a.D + (double)a.eps));
#pragma unroll
                for (int j = 0; j < NJ; ++j)
#pragma unroll
                    for (int e = 0; e < V; ++e) {
                        const int p = elem<V>(lane, j) + e, k = j * V + e;
                        if (p < half) {
                            x1[i][k] = x1[i][k] * inv * a.w[p];
                            x2[i][k] = x2[i][k] * inv * a.w[p + half];
                        }
                    }
            }
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int p0 = elem<V>(lane, j);
            if (p0 >= half) continue;
            float y1[V], y2[V];
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const int k = j * V + e;
                y1[e] = x1[i][k];
                y2[e] = x2[i][k];
                if (a.rope) {
                    const float ang = (float)ra.s * a.inv_freq[p0 + e];
                    float c, sn;
                    sincosf(ang, &sn, &c);
                    y1[e] = x1[i][k] * c - x2[i][k] * sn;
                    y2[e] = x1[i][k] * sn + x2[i][k] * c;
                }
            }
            Vec<T, V>::store(yr + p0, y1);
            Vec<T, V>::store(yr + p0 + half, y2);
        }
    }
}

// Backward: workgroup g (4 waves) owns rows [4 RPW g, 4 RPW (g + 1)), wave w
// the rows 4 RPW g + w + 4 i (i < RPW), all loaded before any is computed.
// The dL/dw terms are summed per wave in row order, then over the 4 waves in
// wave order (LDS), giving one [D] partial per workgroup.
template <typename T, int NJ, int V>
__global__ __launch_bounds__(256) void prologue_bwd_kernel(PrologueArgs a) {
#pragma clang fp contract(off)
    constexpr int E = NJ * V;
    constexpr int RPW = prologue_bwd_rows_per_wave(E);
    __shared__ float red[3][PROLOGUE_MAX_D];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int half = a.D / 2;
    const bool norm = a.norm != PROLOGUE_NORM_NONE;
    const int64_t rbase = (int64_t)blockIdx.x * 4 * RPW + w;
    float gw1[E], gw2[E];
#pragma unroll
    for (int k = 0; k < E; ++k) gw1[k] = gw2[k] = 0.f;
    float g1[RPW][E], g2[RPW][E], x1[RPW][E], x2[RPW][E];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const int64_t r = rbase + 4 * i;
        const bool live = r < a.rows;
        const RowAddr ra = row_addr(a, live ? r : 0);
        const float* gr = a.dy + a.sdy.at(ra.b, ra.h) + (int64_t)ra.s * a.sdy.s;
        const T* xr = norm ? (const T*)a.x + a.sx.at(ra.b, ra.h) + (int64_t)ra.s * a.sx.s : nullptr;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int p = elem<V>(lane, j);
            if (live && p < half) {
                Vec<float, V>::load(gr + p, &g1[i][j * V]);
                Vec<float, V>::load(gr + p + half, &g2[i][j * V]);
            } else {
#pragma unroll
                for (int e = 0; e < V; ++e) g1[i][j * V + e] = g2[i][j * V + e] = 0.f;
            }
            if (norm && live && p < half) {
                Vec<T, V>::load(xr + p, &x1[i][j * V]);
                Vec<T, V>::load(xr + p + half, &x2[i][j * V]);
            } else {
#pragma unroll
                for (int e = 0; e < V; ++e) x1[i][j * V + e] = x2[i][j * V + e] = 0.f;
            }
        }
    }
    // effective weights: 1 + w for Gemma's rms_norm, w for the affine variant
    double we1[E], we2[E];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int e = 0; e < V; ++e) {
            const int p = elem<V>(lane, j) + e, k = j * V + e;
            const bool ok = norm && p < half;
            const double w1 = ok ? (double)a.w[p] : 0.0, w2 = ok ? (double)a.w[p + half] : 0.0;
            we1[k] = a.norm == PROLOGUE_NORM_GEMMA ? 1.0 + w1 : w1;
            we2[k] = a.norm == PROLOGUE_NORM_GEMMA ? 1.0 + w2 : w2;
        }
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const int64_t r = rbase + 4 * i;
        if (r >= a.rows) break;  // wave-uniform
        const RowAddr ra = row_addr(a, r);
        float* dxr = a.dx + a.sdx.at(ra.b, ra.h) + (int64_t)ra.s * a.sdx.s;
        // gradient at the norm's output: R^T dy
        if (a.rope) {
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    const int p = elem<V>(lane, j) + e, k = j * V + e;
                    if (p >= half) continue;
                    const float ang = (float)ra.s * a.inv_freq[p];
                    float c, sn;
                    sincosf(ang, &sn, &c);
                    const float a1 = g1[i][k], a2 = g2[i][k];
                    g1[i][k] = a1 * c + a2 * sn;
                    g2[i][k] = -a1 * sn + a2 * c;
                }
        }
        if (norm) {
            double ss = 0.0, dot = 0.0;
#pragma unroll
            for (int k = 0; k < E; ++k) {
                ss += (double)x1[i][k] * (double)x1[i][k] + (double)x2[i][k] * (double)x2[i][k];
                dot += (double)g1[i][k] * we1[k] * (double)x1[i][k] + (double)g2[i][k] * we2[k] * (double)x2[i][k];
            }
            ss = wave_sum(ss);
            dot = wave_sum(dot);
            const double inv = 1.0 / sqrt(ss / (double)a.D + (double)a.eps);
            const double coeff = (inv * inv * inv) / (double)a.D;
#pragma unroll
            for (int k = 0; k < E; ++k) {
                const float d1 = (float)((double)g1[i][k] * we1[k] * inv - (double)x1[i][k] * coeff * dot);
                const float d2 = (float)((double)g2[i][k] * we2[k] * inv - (double)x2[i][k] * coeff * dot);
                gw1[k] += (float)((double)g1[i][k] * (double)x1[i][k] * inv);
                gw2[k] += (float)((double)g2[i][k] * (double)x2[i][k] * inv);
                g1[i][k] = d1;
                g2[i][k] = d2;
            }
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int p = elem<V>(lane, j);
            if (p < half) {
                Vec<float, V>::store(dxr + p, &g1[i][j * V]);
                Vec<float, V>::store(dxr + p + half, &g2[i][j * V]);
            }
        }
    }
    if (!norm || !a.dw_part) return;
    // the workgroup's partial: waves 1..3 hand theirs to wave 0, which adds
    // them in wave order
    if (w > 0) {
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const int p = elem<V>(lane, j) + e, k = j * V + e;
                if (p < half) {
                    red[w - 1][p] = gw1[k];
                    red[w - 1][p + half] = gw2[k];
                }
            }
    }
    __syncthreads();
    if (w == 0) {
        float* part = a.dw_part + (int64_t)blockIdx.x * a.D;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const int p = elem<V>(lane, j) + e, k = j * V + e;
                if (p >= half) continue;
                float s1 = gw1[k], s2 = gw2[k];
                for (int q = 0; q < 3; ++q) {
                    s1 += red[q][p];
                    s2 += red[q][p + half];
                }
                part[p] = s1;
                part[p + half] = s2;
            }
    }
}

// dw[c] = sum of the workgroup partials, in a fixed order: 64 slices per
// column (slice t adds partials t, t + 64, ... in double, eight loads in
// flight), then the slices in slice order.
struct DwReduce {
    const float* part[kPrologueMaxBatch];
    int64_t nparts[kPrologueMaxBatch];
    float* dw[kPrologueMaxBatch];
};
__device__ __forceinline__ void prologue_dw_reduce(const float* part, int64_t nparts, int D, float* dw);
// One launch for the dw of every tensor of a batch: blockIdx.y = tensor.
__global__ __launch_bounds__(1024) void prologue_dw_reduce_kernel(DwReduce r, int D) {
    if (blockIdx.y == 0)
        prologue_dw_reduce(r.part[0], r.nparts[0], D, r.dw[0]);
    else
        prologue_dw_reduce(r.part[1], r.nparts[1], D, r.dw[1]);
}
__device__ __forceinline__ void prologue_dw_reduce(const float* part, int64_t nparts, int D, float* dw) {
    constexpr int NS = 64;
    __shared__ double acc[NS][16];
    const int cl = threadIdx.x & 15, sl = threadIdx.x >> 4;
    const int c = blockIdx.x * 16 + cl;
    double s = 0.0;
    if (c < D) {
        int64_t k = sl;
        for (; k + 7 * NS < nparts; k += 8 * NS) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = part[(k + NS * u) * D + c];
#pragma unroll
            for (int u = 0; u < 8; ++u) s += (double)v[u];
        }
        for (; k < nparts; k += NS) s += (double)part[k * D + c];
    }
    acc[sl][cl] = s;
    __syncthreads();
    if (sl == 0 && c < D) {
        double t = 0.0;
        for (int k = 0; k < NS; ++k) t += acc[k][cl];
        dw[c] = (float)t;
    }
}

// ---------------------------------------------------------------------------
// 16-byte lanes (head dims 128, 256, 512): a row is LPR consecutive lanes,
// each holding EPL / 2 contiguous elements of each half (a 16-byte vector
// per half in the forward), so every global access is a vector and a RoPE
// pair stays in its lane.  Row sums are reductions inside the row's LPR-lane
// group (group_sum).  Same arithmetic as the kernels above, element by
// element, up to the order of the row sums' additions.

// Row order of the 16-byte-lane kernels: head fastest, r -> (b, s, h) with
// h = r % H, so that a lane's consecutive row groups are heads of one
// position and share its RoPE angles (sincosf once per position and pair).
__device__ __forceinline__ RowAddr row_addr_hf(const PrologueArgs& a, int64_t r) {
    const int h = (int)(r % a.H);
    const int64_t bs = r / a.H;
    return RowAddr{bs / a.S, h, (int)(bs % a.S)};
}
// The row after ra in row_addr_hf order (head, then position, then batch).
__device__ __forceinline__ RowAddr next_row_hf(const PrologueArgs& a, RowAddr ra) {
    if (++ra.h == a.H) {
        ra.h = 0;
        if (++ra.s == a.S) {
            ra.s = 0;
            ++ra.b;
        }
    }
    return ra;
}
// row_addr_hf of rows r0 .. r0 + G - 1 (r0 < rows): one division pair (32-bit
// multiply-shift when rows < 2^31) and G - 1 steps.
template <int G> __device__ __forceinline__ void rows_hf(const PrologueArgs& a, int64_t r0, RowAddr (&ra)[G]) {
    if (a.rows32) {
        const uint32_t r = (uint32_t)r0, bs = a.fh.div(r), b = a.fs.div(bs);
        ra[0] = RowAddr{(int64_t)b, (int64_t)(r - bs * (uint32_t)a.H), (int)(bs - b * (uint32_t)a.S)};
    } else {
        ra[0] = row_addr_hf(a, r0);
    }
#pragma unroll
    for (int g = 1; g < G; ++g) ra[g] = next_row_hf(a, ra[g - 1]);
}

// x / b, correctly rounded, from y = 1 / b (correctly rounded, once per row):
// q = x y, r = x - q b (exact by an FMA), q + r y rounds to x / b
// (Markstein's correction step; a 3 * 10^9-case random check against IEEE
// division, b with all-ones and all-zeros significands included, found no
// difference).
__device__ __forceinline__ float div_by(float x, float b, float y) {
    const float q = x * y;
    return fmaf(fmaf(-q, b, x), y, q);
}

// Row groups per lane of the forward (all loaded before any is computed).
constexpr int kFwdVecGroups = 2;

// Sum of v over each aligned group of LPR lanes (2 .. 64), the same value in
// every lane of the group, by in-register exchanges (no LDS): DPP quad
// permutes for lanes i ^ 1 and i ^ 2, then half-row and row mirrors (the other
// quad of each 8, the other 8 of each 16: once a quad, or an 8, holds one
// value, pairing with the mirror lane sums the same halves as i ^ 4 or i ^ 8),
// and v_permlane16_swap / v_permlane32_swap for the other row of each 32 and
// the other half-wave.  Each step adds two equal-rank partial sums, so every
// lane of the group adds the same two values.
template <int CTRL> __device__ __forceinline__ double dpp_d(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_mov_dpp((int)b, CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_mov_dpp((int)(b >> 32), CTRL, 0xF, 0xF, false);
    return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}
template <int ROWS> __device__ __forceinline__ double swap_sum(double v) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    const unsigned lo = (unsigned)b, hi = (unsigned)(b >> 32);
    // (first, second) after the swap: (x of this row, x of the paired row)
    // in every lane of the pair, so first + second is the same in both
    const auto l = ROWS == 16 ? __builtin_amdgcn_permlane16_swap(lo, lo, false, false)
                              : __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const auto h = ROWS == 16 ? __builtin_amdgcn_permlane16_swap(hi, hi, false, false)
                              : __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    const double a = __longlong_as_double((long long)(((unsigned long long)h[0] << 32) | l[0]));
    const double c = __longlong_as_double((long long)(((unsigned long long)h[1] << 32) | l[1]));
    return a + c;
}
template <int LPR> __device__ __forceinline__ double group_sum(double v) {
    static_assert(LPR >= 2 && LPR <= 64 && (LPR & (LPR - 1)) == 0, "groups of 2 .. 64 lanes");
    v += dpp_d<0xB1>(v);                          // quad_perm [1,0,3,2]: lane i ^ 1
    if constexpr (LPR >= 4) v += dpp_d<0x4E>(v);  // quad_perm [2,3,0,1]: lane i ^ 2
    if constexpr (LPR >= 8) v += dpp_d<0x141>(v);  // row_half_mirror
    if constexpr (LPR >= 16) v += dpp_d<0x140>(v); // row_mirror
    if constexpr (LPR >= 32) v = swap_sum<16>(v);
    if constexpr (LPR >= 64) v = swap_sum<32>(v);
    return v;
}

// Forward, 16 bytes per lane and row: a lane holds EPL / 2 elements of the
// first half (d = q0 .. q0 + EPL/2 - 1) and their rotate-half partners
// (d + D/2), so each RoPE pair is rotated inside one lane and no shuffle;
// only the norm's sum of squares crosses lanes.  A lane takes GROUPS
// consecutive rows (row_addr_hf order) and evaluates sincosf only when a
// row's position differs from the previous row's.
// blk: the workgroup's index within this tensor's launch range.
template <typename T, int D>
__device__ __forceinline__ void prologue_fwd_vec_body(const PrologueArgs& a, int64_t blk) {
#pragma clang fp contract(off)
    constexpr int EPL = 16 / (int)sizeof(T), H2 = EPL / 2, LPR = D / EPL, RPI = 64 / LPR, HALF = D / 2;
    static_assert(LPR >= 2 && LPR <= 64, "a row spans 2..64 lanes");
    constexpr int GROUPS = kFwdVecGroups;
    const int lane = threadIdx.x & 63, gl = lane % LPR;
    const int q0 = gl * H2;  // this lane's first element of the first half
    // the lane's rows: lane_row0 + g, g < GROUPS
    const int64_t lane_row0 = (blk * 4 + (threadIdx.x >> 6)) * (RPI * GROUPS) + (lane / LPR) * GROUPS;
    float v[GROUPS][2][H2];  // [group][half][element]
    RowAddr ra[GROUPS];
    rows_hf(a, lane_row0 < a.rows ? lane_row0 : 0, ra);
#pragma unroll
    for (int g = 0; g < GROUPS; ++g) {
        const int64_t r = lane_row0 + g;
        if (r < a.rows) {
            const T* x = (const T*)a.x + a.sx.at(ra[g].b, ra[g].h) + (int64_t)ra[g].s * a.sx.s + q0;
            Vec<T, H2>::load(x, v[g][0]);
            Vec<T, H2>::load(x + HALF, v[g][1]);
        } else {
#pragma unroll
            for (int e = 0; e < H2; ++e) v[g][0][e] = v[g][1][e] = 0.f;
        }
    }
    float cs[H2], sn[H2];
    int s_cur = -1;  // position whose angles cs, sn hold
#pragma unroll
    for (int g = 0; g < GROUPS; ++g) {
        const int64_t r = lane_row0 + g;
        if (a.norm != PROLOGUE_NORM_NONE) {
            double ss = 0.0;
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                for (int e = 0; e < H2; ++e) ss += (double)v[g][hf][e] * (double)v[g][hf][e];
            ss = group_sum<LPR>(ss);
            if (a.norm == PROLOGUE_NORM_GEMMA) {
                const float rms = (float)sqrt(ss / (double)D + (double)a.eps), rcp = 1.0f / rms;
#pragma unroll
                for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                    for (int e = 0; e < H2; ++e)
                        v[g][hf][e] = div_by(v[g][hf][e], rms, rcp) * (1.0f + a.w[hf * HALF + q0 + e]);
            } else {
                const float inv = (float)(1.0 / sqrt(ss / (double)D + (double)a.eps));
#pragma unroll
                for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                    for (int e = 0; e < H2; ++e) v[g][hf][e] = v[g][hf][e] * inv * a.w[hf * HALF + q0 + e];
            }
        }
        float y[2][H2];
        if (a.rope) {
            if (ra[g].s != s_cur) {
                s_cur = ra[g].s;
#pragma unroll
                for (int e = 0; e < H2; ++e) sincosf((float)s_cur * a.inv_freq[q0 + e], &sn[e], &cs[e]);
            }
#pragma unroll
            for (int e = 0; e < H2; ++e) {
                const float x1 = v[g][0][e], x2 = v[g][1][e];
                // first half: x1 * c - x2 * s; second half: x1 * s + x2 * c
                y[0][e] = x1 * cs[e] - x2 * sn[e];
                y[1][e] = x1 * sn[e] + x2 * cs[e];
            }
        } else {
#pragma unroll
            for (int e = 0; e < H2; ++e) y[0][e] = v[g][0][e], y[1][e] = v[g][1][e];
        }
        if (r < a.rows) {
            T* yp = (T*)a.y + a.sy.at(ra[g].b, ra[g].h) + (int64_t)ra[g].s * a.sy.s + q0;
            Vec<T, H2>::store(yp, y[0]);
            Vec<T, H2>::store(yp + HALF, y[1]);
        }
    }
}

// Backward with fp32 dy/dx rows as the lane grid (EPL = 4 per lane, LPR =
// D / 4): a lane holds 2 elements of the first half and their rotate-half
// partners, so R^T dy is applied inside the lane.  Rows per workgroup as
// prologue_bwd_blocks counts them, GROUPS consecutive rows per lane in
// row_addr_hf order (sincosf once per position, as in the forward); dL/dw is
// summed per lane over its rows, then over the lanes of the wave that share
// its columns and the 4 waves in fixed order.
template <typename T, int D>
__device__ __forceinline__ void prologue_bwd_vec_body(const PrologueArgs& a, int64_t blk) {
#pragma clang fp contract(off)
    constexpr int EPL = 4, H2 = EPL / 2, LPR = D / EPL, RPI = 64 / LPR, HALF = D / 2;
    static_assert(LPR >= 2 && LPR <= 64, "a row spans 2..64 lanes");
    constexpr int ROWS_WG = 4 * prologue_bwd_rows_per_wave(prologue_elems_per_lane(D));
    constexpr int GROUPS = ROWS_WG / 4 / RPI;  // row groups per wave
    static_assert(GROUPS * RPI * 4 == ROWS_WG, "workgroup rows split evenly");
    __shared__ float red[3][D];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, gl = lane % LPR;
    const int q0 = gl * H2;  // this lane's first element of the first half
    const bool norm = a.norm != PROLOGUE_NORM_NONE;
    // the lane's rows: lane_row0 + g, g < GROUPS
    const int64_t lane_row0 = blk * ROWS_WG + w * (RPI * GROUPS) + (lane / LPR) * GROUPS;
    // every row group's loads first; [group][half][element]
    float gv[GROUPS][2][H2], xv[GROUPS][2][H2];
    RowAddr ra[GROUPS];
    rows_hf(a, lane_row0 < a.rows ? lane_row0 : 0, ra);
#pragma unroll
    for (int g = 0; g < GROUPS; ++g) {
        const int64_t r = lane_row0 + g;
        const bool live = r < a.rows;
        if (live) {
            const float* dy = a.dy + a.sdy.at(ra[g].b, ra[g].h) + (int64_t)ra[g].s * a.sdy.s + q0;
            Vec<float, H2>::load(dy, gv[g][0]);
            Vec<float, H2>::load(dy + HALF, gv[g][1]);
        } else {
#pragma unroll
            for (int e = 0; e < H2; ++e) gv[g][0][e] = gv[g][1][e] = 0.f;
        }
        if (norm && live) {
            const T* x = (const T*)a.x + a.sx.at(ra[g].b, ra[g].h) + (int64_t)ra[g].s * a.sx.s + q0;
            Vec<T, H2>::load(x, xv[g][0]);
            Vec<T, H2>::load(x + HALF, xv[g][1]);
        } else {
#pragma unroll
            for (int e = 0; e < H2; ++e) xv[g][0][e] = xv[g][1][e] = 0.f;
        }
    }
    float gw[2][H2];
    double we[2][H2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int e = 0; e < H2; ++e) {
            gw[hf][e] = 0.f;
            const double wv = norm ? (double)a.w[hf * HALF + q0 + e] : 0.0;
            we[hf][e] = a.norm == PROLOGUE_NORM_GEMMA ? 1.0 + wv : wv;
        }
    float cs[H2], sn[H2];
    int s_cur = -1;  // position whose angles cs, sn hold
#pragma unroll
    for (int g = 0; g < GROUPS; ++g) {
        const int64_t r = lane_row0 + g;
        const bool live = r < a.rows;
        // gradient at the norm's output: R^T dy
        if (a.rope) {
            if (ra[g].s != s_cur) {
                s_cur = ra[g].s;
#pragma unroll
                for (int e = 0; e < H2; ++e) sincosf((float)s_cur * a.inv_freq[q0 + e], &sn[e], &cs[e]);
            }
#pragma unroll
            for (int e = 0; e < H2; ++e) {
                const float g1 = gv[g][0][e], g2 = gv[g][1][e];
                // first half: g1 c + g2 s; second half: -g1 s + g2 c
                gv[g][0][e] = g1 * cs[e] + g2 * sn[e];
                gv[g][1][e] = -g1 * sn[e] + g2 * cs[e];
            }
        }
        if (norm) {
            double ss = 0.0, dot = 0.0;
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                for (int e = 0; e < H2; ++e) {
                    ss += (double)xv[g][hf][e] * (double)xv[g][hf][e];
                    dot += (double)gv[g][hf][e] * we[hf][e] * (double)xv[g][hf][e];
                }
            ss = group_sum<LPR>(ss);
            dot = group_sum<LPR>(dot);
            const double inv = 1.0 / sqrt(ss / (double)D + (double)a.eps);
            const double coeff = (inv * inv * inv) / (double)D;
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                for (int e = 0; e < H2; ++e) {
                    const float d =
                        (float)((double)gv[g][hf][e] * we[hf][e] * inv - (double)xv[g][hf][e] * coeff * dot);
                    if (live) gw[hf][e] += (float)((double)gv[g][hf][e] * (double)xv[g][hf][e] * inv);
                    gv[g][hf][e] = d;
                }
        }
        if (live) {
            float* dx = a.dx + a.sdx.at(ra[g].b, ra[g].h) + (int64_t)ra[g].s * a.sdx.s + q0;
            Vec<float, H2>::store(dx, gv[g][0]);
            Vec<float, H2>::store(dx + HALF, gv[g][1]);
        }
    }
    if (!norm || !a.dw_part) return;
    // the wave's row groups, then the workgroup's waves, in fixed order
#pragma unroll
    for (int o = LPR; o < 64; o <<= 1)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int e = 0; e < H2; ++e) gw[hf][e] += __shfl_xor(gw[hf][e], o, 64);
    if (w > 0 && lane < LPR) {
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int e = 0; e < H2; ++e) red[w - 1][hf * HALF + q0 + e] = gw[hf][e];
    }
    __syncthreads();
    if (w == 0 && lane < LPR) {
        float* part = a.dw_part + blk * D;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int e = 0; e < H2; ++e) {
                const int idx = hf * HALF + q0 + e;
                float t = gw[hf][e];
                for (int q = 0; q < 3; ++q) t += red[q][idx];
                part[idx] = t;
            }
    }
}

// The 16-byte-lane kernels over a batch of tensors (PrologueBatch): tensor
// i takes workgroups first_block[i] .. first_block[i + 1] - 1, each the
// workgroup of that index in a launch of its own; the branch picks a
// statically indexed argument set.
template <typename T, int D>
__global__ __launch_bounds__(256) void prologue_fwd_vec(PrologueBatch bb) {
    const int64_t bx = blockIdx.x;
    if (bb.n > 1 && bx >= bb.first_block[1])
        prologue_fwd_vec_body<T, D>(bb.a[1], bx - bb.first_block[1]);
    else
        prologue_fwd_vec_body<T, D>(bb.a[0], bx);
}
template <typename T, int D>
__global__ __launch_bounds__(256) void prologue_bwd_vec(PrologueBatch bb) {
    const int64_t bx = blockIdx.x;
    if (bb.n > 1 && bx >= bb.first_block[1])
        prologue_bwd_vec_body<T, D>(bb.a[1], bx - bb.first_block[1]);
    else
        prologue_bwd_vec_body<T, D>(bb.a[0], bx);
}
static_assert(kPrologueMaxBatch == 2, "the batch kernels pick one of two argument sets");

// Whether every row of a layout starts on a vbytes boundary.
bool rows_aligned(const void* base, const Strides& st, int64_t esz, int vbytes) {
    const int64_t m = vbytes / esz;
    return (reinterpret_cast<uintptr_t>(base) % vbytes) == 0 && st.b % m == 0 && st.h % m == 0 && st.s % m == 0;
}

template <typename T, int NJ, int V>
hipError_t launch_shape(const PrologueArgs& a, bool bwd, hipStream_t st) {
    if (bwd) {
        hipLaunchKernelGGL((prologue_bwd_kernel<T, NJ, V>), dim3((unsigned)prologue_bwd_blocks(a.rows, a.D)),
                           dim3(256), 0, st, a);
    } else {
        const int64_t blocks = (a.rows + 4 * FWD_RPW - 1) / (4 * FWD_RPW);
        hipLaunchKernelGGL((prologue_fwd_kernel<T, NJ, V>), dim3((unsigned)blocks), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

// Whether the 16-byte-lane kernel of head dim D takes tensor a (its head
// dim and every row's alignment allow it).
template <typename T, int D>
bool vec_takes(const PrologueArgs& a, bool bwd) {
    const int64_t esz = sizeof(T);
    if (a.D != D) return false;
    if (bwd) {
        if constexpr (D / 4 > 64) {
            return false;
        } else {
            if (!rows_aligned(a.dy, a.sdy, 4, 16) || !rows_aligned(a.dx, a.sdx, 4, 16)) return false;
            return a.norm == PROLOGUE_NORM_NONE || rows_aligned(a.x, a.sx, esz, 4 * (int)esz);
        }
    } else {
        if constexpr (D * (int)sizeof(T) / 16 > 64) {
            return false;
        } else {
            return rows_aligned(a.x, a.sx, esz, 16) && rows_aligned(a.y, a.sy, esz, 16);
        }
    }
}

// Workgroups of the 16-byte-lane launch for one tensor.
template <typename T, int D>
int64_t vec_blocks(const PrologueArgs& a, bool bwd) {
    if (bwd) return prologue_bwd_blocks(a.rows, D);
    constexpr int LPR = D * (int)sizeof(T) / 16;
    const int64_t per_block = 4 * (64 / (LPR < 64 ? LPR : 64)) * kFwdVecGroups;
    return (a.rows + per_block - 1) / per_block;
}

// One 16-byte-lane launch over n <= kPrologueMaxBatch tensors it takes.
template <typename T, int D>
hipError_t launch_vec(const PrologueArgs* a, int n, bool bwd, hipStream_t st) {
    PrologueBatch bb;
    bb.n = n;
    int64_t blocks = 0;
    for (int i = 0; i < n; ++i) {
        bb.a[i] = a[i];
        bb.first_block[i] = blocks;
        blocks += vec_blocks<T, D>(a[i], bwd);
    }
    for (int i = n; i <= kPrologueMaxBatch; ++i) bb.first_block[i] = blocks;
    if (bwd) {
        if constexpr (D / 4 <= 64)
            hipLaunchKernelGGL((prologue_bwd_vec<T, D>), dim3((unsigned)blocks), dim3(256), 0, st, bb);
    } else {
        if constexpr (D * (int)sizeof(T) / 16 <= 64)
            hipLaunchKernelGGL((prologue_fwd_vec<T, D>), dim3((unsigned)blocks), dim3(256), 0, st, bb);
    }
    return hipGetLastError();
}

template <typename T, int D>
bool all_vec(const PrologueArgs* a, int n, bool bwd) {
    for (int i = 0; i < n; ++i)
        if (!vec_takes<T, D>(a[i], bwd)) return false;
    return true;
}

// One tensor by the one-wave-per-row kernels.
template <typename T>
hipError_t launch_rows(const PrologueArgs& a, bool bwd, hipStream_t st) {
    const int half = a.D / 2;
    const int64_t esz = sizeof(T);
    if (half == 64 || half == 128 || half == 256) {
        const int V = half / 64;  // contiguous elements per lane
        bool ok;
        if (bwd) {
            ok = rows_aligned(a.dy, a.sdy, 4, 4 * V) && rows_aligned(a.dx, a.sdx, 4, 4 * V);
            if (a.norm != PROLOGUE_NORM_NONE) ok = ok && rows_aligned(a.x, a.sx, esz, V * (int)esz);
        } else {
            ok = rows_aligned(a.x, a.sx, esz, V * (int)esz) && rows_aligned(a.y, a.sy, esz, V * (int)esz);
        }
        if (ok) {
            if (V == 1) return launch_shape<T, 1, 1>(a, bwd, st);
            if (V == 2) return launch_shape<T, 1, 2>(a, bwd, st);
            return launch_shape<T, 1, 4>(a, bwd, st);
        }
    }
    if (half <= 64) return launch_shape<T, 1, 1>(a, bwd, st);
    if (half <= 128) return launch_shape<T, 2, 1>(a, bwd, st);
    return launch_shape<T, 4, 1>(a, bwd, st);
}

// n tensors: one launch when the 16-byte-lane kernel of their common head
// dim takes them all, otherwise one launch per tensor.
template <typename T>
hipError_t launch_t(const PrologueArgs* a, int n, bool bwd, hipStream_t st) {
    const int D = a[0].D;
    if (D == 128 && all_vec<T, 128>(a, n, bwd)) return launch_vec<T, 128>(a, n, bwd, st);
    if (D == 256 && all_vec<T, 256>(a, n, bwd)) return launch_vec<T, 256>(a, n, bwd, st);
    if (D == 512 && all_vec<T, 512>(a, n, bwd)) return launch_vec<T, 512>(a, n, bwd, st);
    for (int i = 0; i < n; ++i) {
        hipError_t e;
        if (a[i].D == 128 && vec_takes<T, 128>(a[i], bwd)) e = launch_vec<T, 128>(a + i, 1, bwd, st);
        else if (a[i].D == 256 && vec_takes<T, 256>(a[i], bwd)) e = launch_vec<T, 256>(a + i, 1, bwd, st);
        else if (a[i].D == 512 && vec_takes<T, 512>(a[i], bwd)) e = launch_vec<T, 512>(a + i, 1, bwd, st);
        else e = launch_rows<T>(a[i], bwd, st);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace

int64_t prologue_bwd_blocks(int64_t rows, int D) {
    const int rows_per_wg = 4 * prologue_bwd_rows_per_wave(prologue_elems_per_lane(D));
    return (rows + rows_per_wg - 1) / rows_per_wg;
}

hipError_t launch_prologue_fwd(const PrologueArgs* a, int n, bool is_bf16, hipStream_t st) {
    return is_bf16 ? launch_t<bf16>(a, n, false, st) : launch_t<float>(a, n, false, st);
}

hipError_t launch_prologue_bwd(const PrologueArgs* a, int n, bool is_bf16, float* const* dw, hipStream_t st) {
    const hipError_t e = is_bf16 ? launch_t<bf16>(a, n, true, st) : launch_t<float>(a, n, true, st);
    if (e != hipSuccess) return e;
    // dw of every tensor with a norm and a dw output: one launch per head
    // dim (one in all when they share it, as the q and k heads do)
    bool done[kPrologueMaxBatch] = {};
    for (int i = 0; i < n; ++i) {
        if (done[i] || a[i].norm == PROLOGUE_NORM_NONE || !dw[i] || !a[i].dw_part) continue;
        DwReduce r{};
        int m = 0;
        for (int j = i; j < n; ++j) {
            if (done[j] || a[j].norm == PROLOGUE_NORM_NONE || !dw[j] || !a[j].dw_part || a[j].D != a[i].D) continue;
            r.part[m] = a[j].dw_part;
            r.nparts[m] = prologue_bwd_blocks(a[j].rows, a[j].D);
            r.dw[m] = dw[j];
            done[j] = true;
            ++m;
        }
        hipLaunchKernelGGL(prologue_dw_reduce_kernel, dim3((unsigned)((a[i].D + 15) / 16), (unsigned)m), dim3(1024), 0,
                           st, r, a[i].D);
        const hipError_t e2 = hipGetLastError();
        if (e2 != hipSuccess) return e2;
    }
    return hipSuccess;
}

}  // namespace mft
