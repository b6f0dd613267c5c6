// Element conversions on the device for the drop-in adapters' host tensors
// (mft_convert in include/mft/attention.h): bf16 -> fp32 exactly, fp32 ->
// bf16 with the reference's rounding (core/dtype.h:114-121,
// float32_to_bf16_bits: bits += 0x7FFF + lsb, then the high half; NaN
// payloads and overflow to infinity follow from the same integer add).
// HBM-bound: 16-byte vector loads and stores, a grid-stride loop.
#include <algorithm>
#include <string>

#include "attn_common.h"
#include "capi_util.h"
#include "mft/attention.h"

namespace mft {
namespace {

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float x) {
    uint32_t bits = __builtin_bit_cast(uint32_t, x);
    bits += 0x7FFFu + ((bits >> 16) & 1u);
    return (uint16_t)(bits >> 16);
}

// 8 elements per thread step: 32 bytes of fp32 in, 16 bytes of bf16 out.
__global__ __launch_bounds__(256) void convert_f32_bf16(const float* __restrict__ src, uint16_t* __restrict__ dst,
                                                        int64_t n) {
    const int64_t n8 = n / 8, stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += stride) {
        const f32x4 a = reinterpret_cast<const f32x4*>(src)[2 * i];
        const f32x4 b = reinterpret_cast<const f32x4*>(src)[2 * i + 1];
        typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
        const u16x8 o = {f32_to_bf16_rne(a[0]), f32_to_bf16_rne(a[1]), f32_to_bf16_rne(a[2]), f32_to_bf16_rne(a[3]),
                         f32_to_bf16_rne(b[0]), f32_to_bf16_rne(b[1]), f32_to_bf16_rne(b[2]), f32_to_bf16_rne(b[3])};
        reinterpret_cast<u16x8*>(dst)[i] = o;
    }
    for (int64_t i = 8 * n8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = f32_to_bf16_rne(src[i]);
}

__global__ __launch_bounds__(256) void convert_bf16_f32(const uint16_t* __restrict__ src, float* __restrict__ dst,
                                                        int64_t n) {
    const int64_t n8 = n / 8, stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += stride) {
        typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
        const u16x8 x = reinterpret_cast<const u16x8*>(src)[i];
        f32x4 a, b;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            a[j] = __builtin_bit_cast(float, (uint32_t)x[j] << 16);
            b[j] = __builtin_bit_cast(float, (uint32_t)x[j + 4] << 16);
        }
        reinterpret_cast<f32x4*>(dst)[2 * i] = a;
        reinterpret_cast<f32x4*>(dst)[2 * i + 1] = b;
    }
    for (int64_t i = 8 * n8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = __builtin_bit_cast(float, (uint32_t)src[i] << 16);
}

}  // namespace
}  // namespace mft

extern "C" mft_status mft_convert(const void* src, mft_dtype src_dtype, void* dst, mft_dtype dst_dtype, int64_t n,
                                  hipStream_t stream) {
    using mft::capi::fail;
    if (n < 0) return fail(MFT_ERR_INVALID_ARG, "mft_convert: n must be >= 0");
    if (n == 0) return MFT_OK;
    if (!src || !dst) return fail(MFT_ERR_INVALID_ARG, "mft_convert: src and dst must be non-NULL");
    if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15u)
        return fail(MFT_ERR_INVALID_ARG, "mft_convert: buffers must be 16-byte aligned");
    const int64_t blocks = std::min<int64_t>((n / 8 + 255) / 256 + 1, 4096);
    if (src_dtype == MFT_F32 && dst_dtype == MFT_BF16)
        hipLaunchKernelGGL(mft::convert_f32_bf16, dim3((unsigned)blocks), dim3(256), 0, stream,
                           static_cast<const float*>(src), static_cast<uint16_t*>(dst), n);
    else if (src_dtype == MFT_BF16 && dst_dtype == MFT_F32)
        hipLaunchKernelGGL(mft::convert_bf16_f32, dim3((unsigned)blocks), dim3(256), 0, stream,
                           static_cast<const uint16_t*>(src), static_cast<float*>(dst), n);
    else
        return fail(MFT_ERR_INVALID_ARG, "mft_convert: only MFT_F32 -> MFT_BF16 and MFT_BF16 -> MFT_F32");
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? MFT_OK : fail(MFT_ERR_HIP, std::string("mft_convert launch: ") + hipGetErrorString(e));
}
