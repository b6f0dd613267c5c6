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
// consecutive addresses.
#pragma clang fp contract(off)
__global__ __launch_bounds__(256) void lora_merge_kernel(LoraMergeArgs a) {
    const int64_t total = a.in * a.cols;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
        const int64_t i = e / a.cols, o = e % a.cols;
        double delta = 0.0;
        for (int64_t r = 0; r < a.rank; ++r) {
            const float av = a.a_transposed ? a.A[r * a.in + i] : a.A[i * a.rank + r];
            const float bv = a.b_transposed ? a.B[o * a.rank + r] : a.B[r * a.cols + o];
            delta = __dadd_rn(delta, __dmul_rn((double)av, (double)bv));
        }
        const int64_t c = a.col0 + o;
        const int64_t w = a.w_transposed ? c * a.in + i : i * a.out + c;
        if (a.w_bf16) {
            uint16_t* W = static_cast<uint16_t*>(a.W);
            W[w] = bf16_bits_rne(__fadd_rn(bf16_bits_to_float(W[w]), __fmul_rn(a.sign_scale, (float)delta)));
        } else {
            float* W = static_cast<float*>(a.W);
            W[w] = __fadd_rn(W[w], __fmul_rn(a.sign_scale, (float)delta));
        }
    }
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

hipError_t launch_lora_merge(const LoraMergeArgs& a, hipStream_t st) {
    if (a.in <= 0 || a.cols <= 0) return hipSuccess;
    hipLaunchKernelGGL(lora_merge_kernel, dim3(grid_for(a.in * a.cols)), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace mft
