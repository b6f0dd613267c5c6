// Launchers of the LoRA linear's element-wise kernels (lora.hip; called by
// lora_capi.cpp).  The GEMMs themselves are rocBLAS calls in lora_capi.cpp.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mft {

// dst[i] = bf16 bits of src[i], rounded to nearest even the way the
// reference's float32_to_bf16_bits does (core/dtype.h:114-121).
hipError_t launch_lora_round_bf16(const float* src, uint16_t* dst, int64_t n, hipStream_t st);

// y[n, o] = bias[o] for n < N, o < out.
hipError_t launch_lora_fill_bias(float* y, const float* bias, int64_t N, int64_t out, hipStream_t st);

struct LoraMergeArgs {
    void* W;               // fp32 or bf16 bits
    const float* A;
    const float* B;
    float sign_scale;      // sign * scale, as the reference forms it
    int w_bf16, w_transposed, a_transposed, b_transposed;
    int64_t in, out, rank, col0, cols;
};

// W[i, col0 + o] = W + sign_scale * float(sum_r double(A[i, r]) * double(B[r, o])).
hipError_t launch_lora_merge(const LoraMergeArgs& a, hipStream_t st);

}  // namespace mft
