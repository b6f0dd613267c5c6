// Element-wise kernels of the LoRA linear layer (C ABI in include/mft/lora.h,
// GEMMs in lora_capi.cpp).
//
//   lora_round_bf16   fp32 -> bf16 operand staging for the bf16 MFMA GEMMs;
//                     HBM-bound, 6 bytes per element, 16-byte vectors.
//   lora_fill_bias    y = broadcast(bias) ahead of a beta = 1 GEMM (the
//                     reference's add(y, b), nn/lora_linear.cpp:349-351).
//   lora_merge        apply_lora_delta_to_base (nn/lora_linear.cpp:108-138):
//                     per element a rank-long double dot product, then one
//                     fp32 multiply and add, element for element as the
//                     reference rounds them (fp contract off).
#include <hip/hip_runtime.h>

#include "lora_kernels.h"

namespace mft {
namespace {

__device__ __forceinline__ uint16_t bf16_bits_rne(float x) {
    uint32_t bits = __float_as_uint(x);
    bits += 0x7FFFu + ((bits >> 16) & 1u);
    return (uint16_t)(bits >> 16);
}

__device__ __forceinline__ float bf16_bits_to_float(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

__global__ __launch_bounds__(256) void lora_round_bf16_vec(const float4* __restrict__ src, uint2* __restrict__ dst,
                                                           int64_t n4) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
        const float4 v = src[i];
        dst[i] = make_uint2((uint32_t)bf16_bits_rne(v.x) | ((uint32_t)bf16_bits_rne(v.y) << 16),
                            (uint32_t)bf16_bits_rne(v.z) | ((uint32_t)bf16_bits_rne(v.w) << 16));
    }
}

__global__ __launch_bounds__(256) void lora_round_bf16_tail(const float* __restrict__ src,
                                                            uint16_t* __restrict__ dst, int64_t i0, int64_t n) {
    const int64_t i = i0 + (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = bf16_bits_rne(src[i]);
}

__global__ __launch_bounds__(256) void lora_fill_bias_kernel(float* __restrict__ y, const float* __restrict__ bias,
                                                             int64_t N, int64_t out) {
    const int64_t total = N * out;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256)
        y[i] = bias[i % out];
}

// One thread per (i, o) element of the slice's [in, cols] block; o runs
// fastest so that B's row and W's row (untransposed layouts) are read in
// consecutive addresses.  Every multiply and add is rounded on its own, as
// the reference's are (fp contract off in this kernel only).
__global__ __launch_bounds__(256) void lora_merge_kernel(LoraMergeArgs a) {
#pragma clang fp contract(off)
    const int64_t total = a.in * a.cols;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
        const int64_t i = e / a.cols, o = e % a.cols;
        double delta = 0.0;
        for (int64_t r = 0; r < a.rank; ++r) {
            const float av = a.a_transposed ? a.A[r * a.in + i] : a.A[i * a.rank + r];
            const float bv = a.b_transposed ? a.B[o * a.rank + r] : a.B[r * a.cols + o];
            delta += (double)av * (double)bv;
        }
        const int64_t c = a.col0 + o;
        const int64_t w = a.w_transposed ? c * a.in + i : i * a.out + c;
        if (a.w_bf16) {
            uint16_t* W = static_cast<uint16_t*>(a.W);
            W[w] = bf16_bits_rne(bf16_bits_to_float(W[w]) + a.sign_scale * (float)delta);
        } else {
            float* W = static_cast<float*>(a.W);
            W[w] = W[w] + a.sign_scale * (float)delta;
        }
    }
}

// ---- rank-r products (r is small, the inner dimension long) ----
//
// lora_rowdot: out[n, j] = alpha sum_k M[n, k] P(k, j).  A workgroup owns
// kRowsPerWg rows; its 256 threads stride jointly over k (thread t: columns
// VEC t + 256 VEC i) and each keeps kRowsPerWg x 8 partial sums (one 8-wide
// block of j at a time), so each P(k, j) it loads serves kRowsPerWg rows.  The
// 256 partials of each (row, j) are summed through LDS in a fixed order
// (deterministic).  M is read once per 8-wide block of j: HBM-bound for r <= 8.
constexpr int kRowsPerWg = 8, kJB = 8;

template <int VEC>
__global__ __launch_bounds__(256) void lora_rowdot_kernel(LoraRowDot a) {
    constexpr int NV = kRowsPerWg * kJB;  // partial sums per thread
    __shared__ float red[NV][257];
    __shared__ float red2[4][NV];
    const int t = threadIdx.x;
    const int64_t n0 = (int64_t)blockIdx.x * kRowsPerWg;
    for (int jb = 0; jb < a.r; jb += kJB) {
        float acc[kRowsPerWg][kJB];
#pragma unroll
        for (int i = 0; i < kRowsPerWg; ++i)
#pragma unroll
            for (int j = 0; j < kJB; ++j) acc[i][j] = 0.f;
        for (int64_t k = (int64_t)VEC * t; k < a.K; k += 256 * VEC) {
            float p[VEC][kJB];
#pragma unroll
            for (int v = 0; v < VEC; ++v)
#pragma unroll
                for (int j = 0; j < kJB; ++j) {
                    // clamped index, so the load needs no branch; the select zeroes j >= r
                    const int jj = jb + j < a.r ? jb + j : a.r - 1;
                    const float pv = a.P[(k + v) * a.pk + (int64_t)jj * a.pj];
                    p[v][j] = jb + j < a.r ? pv : 0.f;
                }
            float mv[kRowsPerWg][VEC];
#pragma unroll
            for (int i = 0; i < kRowsPerWg; ++i) {
                const int64_t n = n0 + i < a.rows ? n0 + i : a.rows - 1;
                const float* m = a.M + n * a.ldm + k;
                if (VEC == 4) {
                    const float4 q = *reinterpret_cast<const float4*>(m);
                    mv[i][0] = q.x, mv[i][1 % VEC] = q.y, mv[i][2 % VEC] = q.z, mv[i][3 % VEC] = q.w;
                } else {
                    mv[i][0] = m[0];
                }
            }
            if (a.mb && jb == 0) {  // the bf16 copy of M, from the first j-block's loads
#pragma unroll
                for (int i = 0; i < kRowsPerWg; ++i) {
                    if (n0 + i >= a.rows) continue;
                    uint16_t* d = a.mb + (n0 + i) * a.ldb + k;
                    if (VEC == 4)
                        *reinterpret_cast<uint2*>(d) =
                            make_uint2((uint32_t)bf16_bits_rne(mv[i][0]) | ((uint32_t)bf16_bits_rne(mv[i][1 % VEC]) << 16),
                                       (uint32_t)bf16_bits_rne(mv[i][2 % VEC]) |
                                           ((uint32_t)bf16_bits_rne(mv[i][3 % VEC]) << 16));
                    else
                        d[0] = bf16_bits_rne(mv[i][0]);
                }
            }
#pragma unroll
            for (int i = 0; i < kRowsPerWg; ++i)
#pragma unroll
                for (int v = 0; v < VEC; ++v)
#pragma unroll
                    for (int j = 0; j < kJB; ++j) acc[i][j] += mv[i][v] * p[v][j];
        }
#pragma unroll
        for (int i = 0; i < kRowsPerWg; ++i)
#pragma unroll
            for (int j = 0; j < kJB; ++j) red[i * kJB + j][t] = acc[i][j];
        __syncthreads();
        {
            // quarter q of the 256 partials of value e, then the 4 quarters
            const int e = t % NV, q = t / NV;
            float s = 0.f;
            for (int l = 0; l < 64; ++l) s += red[e][64 * q + l];
            red2[q][e] = s;
        }
        __syncthreads();
        if (t < NV) {
            const int i = t / kJB, j = t % kJB;
            const float s = (red2[0][t] + red2[1][t]) + (red2[2][t] + red2[3][t]);
            const int64_t n = n0 + i;
            if (n < a.rows && jb + j < a.r) a.out[n * a.ldo + jb + j] = a.alpha * s;
        }
        __syncthreads();
    }
}

// lora_coldot: per chunk c of rows and column k, partial[c][k][j] = sum over
// the chunk's rows of M[n, k] V[n, j]; one wave per (64 VEC columns, chunk),
// the row of V is the same for the whole wave.  The chunk height is chosen so
// that about 2048 waves run (lora_coldot_chunk, lora_kernels.h).  Then
// lora_coldot_reduce sums the chunks in a fixed order.

template <int VEC>
__global__ __launch_bounds__(64) void lora_coldot_kernel(LoraColDot a, int64_t chunk) {
    const int64_t k = ((int64_t)blockIdx.x * 64 + threadIdx.x) * VEC;
    const int64_t c = blockIdx.y;
    const int64_t r0 = c * chunk, r1 = r0 + chunk < a.rows ? r0 + chunk : a.rows;
    const bool live = k < a.K;
    for (int jb = 0; jb < a.r; jb += kJB) {
        float acc[VEC][kJB];
#pragma unroll
        for (int v = 0; v < VEC; ++v)
#pragma unroll
            for (int j = 0; j < kJB; ++j) acc[v][j] = 0.f;
#pragma unroll 8
        for (int64_t n = r0; n < r1; ++n) {
            float vv[kJB];
#pragma unroll
            for (int j = 0; j < kJB; ++j) {
                const int jj = jb + j < a.r ? jb + j : a.r - 1;
                const float x = a.V[n * a.ldv + jj];
                vv[j] = jb + j < a.r ? x : 0.f;
            }
            float mv[VEC];
            if (live) {
                const float* m = a.M + n * a.ldm + k;
                if (VEC == 4) {
                    const float4 q = *reinterpret_cast<const float4*>(m);
                    mv[0] = q.x, mv[1 % VEC] = q.y, mv[2 % VEC] = q.z, mv[3 % VEC] = q.w;
                } else {
                    mv[0] = m[0];
                }
            } else {
#pragma unroll
                for (int v = 0; v < VEC; ++v) mv[v] = 0.f;
            }
#pragma unroll
            for (int v = 0; v < VEC; ++v)
#pragma unroll
                for (int j = 0; j < kJB; ++j) acc[v][j] += mv[v] * vv[j];
        }
        if (live) {
            float* part = a.partial + (c * a.K + k) * a.r + jb;
#pragma unroll
            for (int v = 0; v < VEC; ++v)
#pragma unroll
                for (int j = 0; j < kJB; ++j)
                    if (jb + j < a.r) part[v * a.r + j] = acc[v][j];
        }
    }
}

// Sixteen lanes per output value: lane l sums chunks l, l + 16, ... in order,
// then the sixteen sums combine in a fixed butterfly (deterministic).
__global__ __launch_bounds__(256) void lora_coldot_reduce(LoraColDot a, int64_t chunks) {
    const int64_t e = ((int64_t)blockIdx.x * 256 + threadIdx.x) / 16;
    const int l = threadIdx.x % 16;
    const int64_t total = a.K * a.r;
    float s = 0.f;
    if (e < total)
        for (int64_t c = l; c < chunks; c += 16) s += a.partial[c * total + e];
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) s += __shfl_xor(s, o, 16);
    if (e < total && l == 0) {
        const int64_t k = e / a.r, j = e % a.r;
        a.out[k * a.ok + j * a.oj] = a.alpha * s;
    }
}

__global__ __launch_bounds__(256) void lora_pack_kmajor_kernel(const float* __restrict__ P, int64_t pk, int64_t pj,
                                                               int64_t K, int r, float* __restrict__ dst) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= K * r) return;
    const int64_t j = e / K, k = e % K;
    dst[e] = P[k * pk + j * pj];
}

unsigned grid_for(int64_t work) {
    const int64_t g = (work + 255) / 256;
    return (unsigned)(g < 1 ? 1 : g > 8192 ? 8192 : g);
}

}  // namespace

hipError_t launch_lora_round_bf16(const float* src, uint16_t* dst, int64_t n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const bool vec = ((uintptr_t)src % 16 == 0) && ((uintptr_t)dst % 8 == 0);
    const int64_t n4 = vec ? n / 4 : 0;
    if (n4 > 0)
        hipLaunchKernelGGL(lora_round_bf16_vec, dim3(grid_for(n4)), dim3(256), 0, st,
                           reinterpret_cast<const float4*>(src), reinterpret_cast<uint2*>(dst), n4);
    const int64_t rest = n - 4 * n4;
    if (rest > 0)
        hipLaunchKernelGGL(lora_round_bf16_tail, dim3((unsigned)((rest + 255) / 256)), dim3(256), 0, st, src, dst,
                           4 * n4, n);
    return hipGetLastError();
}

hipError_t launch_lora_fill_bias(float* y, const float* bias, int64_t N, int64_t out, hipStream_t st) {
    if (N <= 0 || out <= 0) return hipSuccess;
    hipLaunchKernelGGL(lora_fill_bias_kernel, dim3(grid_for(N * out)), dim3(256), 0, st, y, bias, N, out);
    return hipGetLastError();
}

hipError_t launch_lora_rowdot(const LoraRowDot& a, hipStream_t st) {
    if (a.rows <= 0 || a.r <= 0) return hipSuccess;
    const dim3 grid((unsigned)((a.rows + kRowsPerWg - 1) / kRowsPerWg));
    const bool vec = a.K % 4 == 0 && a.ldm % 4 == 0 && (uintptr_t)a.M % 16 == 0 &&
                     (!a.mb || (a.ldb % 4 == 0 && (uintptr_t)a.mb % 8 == 0));
    if (vec)
        hipLaunchKernelGGL(lora_rowdot_kernel<4>, grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL(lora_rowdot_kernel<1>, grid, dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_lora_pack_kmajor(const float* P, int64_t pk, int64_t pj, int64_t K, int r, float* dst,
                                   hipStream_t st) {
    if (K <= 0 || r <= 0) return hipSuccess;
    hipLaunchKernelGGL(lora_pack_kmajor_kernel, dim3((unsigned)((K * r + 255) / 256)), dim3(256), 0, st, P, pk, pj,
                       K, r, dst);
    return hipGetLastError();
}

int64_t lora_coldot_partial_floats(int64_t rows, int64_t K, int r) {
    const int64_t chunk = lora_coldot_chunk(rows, K);
    return (rows + chunk - 1) / chunk * K * r;
}

hipError_t launch_lora_coldot(const LoraColDot& a, hipStream_t st) {
    if (a.K <= 0 || a.r <= 0) return hipSuccess;
    const int64_t chunk = lora_coldot_chunk(a.rows, a.K);
    const int64_t chunks = (a.rows + chunk - 1) / chunk;
    const bool vec = a.K % 4 == 0 && a.ldm % 4 == 0 && (uintptr_t)a.M % 16 == 0;
    const int VEC = vec ? 4 : 1;
    const dim3 grid((unsigned)((a.K + 64 * VEC - 1) / (64 * VEC)), (unsigned)chunks);
    if (vec)
        hipLaunchKernelGGL(lora_coldot_kernel<4>, grid, dim3(64), 0, st, a, chunk);
    else
        hipLaunchKernelGGL(lora_coldot_kernel<1>, grid, dim3(64), 0, st, a, chunk);
    hipLaunchKernelGGL(lora_coldot_reduce, dim3((unsigned)((a.K * a.r * 16 + 255) / 256)), dim3(256), 0, st, a,
                       chunks);
    return hipGetLastError();
}

hipError_t launch_lora_merge(const LoraMergeArgs& a, hipStream_t st) {
    if (a.in <= 0 || a.cols <= 0) return hipSuccess;
    hipLaunchKernelGGL(lora_merge_kernel, dim3(grid_for(a.in * a.cols)), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace mft
