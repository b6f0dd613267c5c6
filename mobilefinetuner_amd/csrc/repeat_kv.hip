// repeat_kv_heads forward and backward for gfx950 (HBM-bound copies/sums).
//
// Forward (core/ops.cpp:2260-2335): out[b, h*r + i] = kv[b, h] — every
// [S, D] head block is contiguous, so this is B*Hkv*r block copies done with
// 16-byte loads/stores when the block size allows.
// Backward (RepeatKVHeadsBackward::apply, core/backward_functions.cpp:693-726):
// dkv[b, h] = ((0 + g[b, h*r]) + g[b, h*r+1]) + ... in fp32, the reference's
// exact accumulation order, so the result is bit-identical to it.
// The fused attention kernels never call these (they index the kv head);
// they exist so that the finetune_ops API keeps repeat_kv_heads on device.
#include "attn_common.h"
#include "attn_kernels.h"

namespace mft {
namespace {

template <typename U>
__global__ __launch_bounds__(256) void repeat_kv_fwd_kernel(const U* __restrict__ kv, U* __restrict__ out,
                                                         int64_t block_units, int64_t n_src_blocks,
                                                         int64_t r) {
    // grid-stride over all output units; unit = element group of sizeof(U) bytes
    const int64_t total = block_units * n_src_blocks * r;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int64_t ob = i / block_units;       // output head block (b*Hkv*r + h*r + rep)
        const int64_t off = i - ob * block_units;
        const int64_t sb = ob / r;                // source head block (b*Hkv + h)
        out[i] = kv[sb * block_units + off];
    }
}

__global__ __launch_bounds__(256) void repeat_kv_bwd_kernel(const float* __restrict__ g, float* __restrict__ dkv,
                                                         int64_t block_elems, int64_t n_dst_blocks,
                                                         int64_t r) {
    const int64_t total = block_elems * n_dst_blocks;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int64_t db = i / block_elems;
        const int64_t off = i - db * block_elems;
        const float* src = g + db * r * block_elems + off;
        float acc = 0.f;
        for (int64_t rep = 0; rep < r; ++rep) acc += src[rep * block_elems];
        dkv[i] = acc;
    }
}

unsigned grid_for(int64_t units) {
    int64_t blocks = (units + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    if (blocks < 1) blocks = 1;
    return (unsigned)blocks;
}

}  // namespace

hipError_t launch_repeat_kv_fwd(const void* kv, void* out, int64_t B, int64_t Hkv, int64_t S,
                                int64_t D, int64_t r, int esize, hipStream_t st) {
    const int64_t bytes = S * D * esize;  // one head block
    const int64_t blocks = B * Hkv;
    const uintptr_t align = (uintptr_t)kv | (uintptr_t)out;
    if (bytes % 16 == 0 && align % 16 == 0) {
        const int64_t units = bytes / 16;
        hipLaunchKernelGGL(repeat_kv_fwd_kernel<f32x4>, dim3(grid_for(units * blocks * r)), dim3(256), 0, st,
                           (const f32x4*)kv, (f32x4*)out, units, blocks, r);
    } else if (bytes % 4 == 0 && align % 4 == 0) {
        const int64_t units = bytes / 4;
        hipLaunchKernelGGL(repeat_kv_fwd_kernel<uint32_t>, dim3(grid_for(units * blocks * r)), dim3(256), 0, st,
                           (const uint32_t*)kv, (uint32_t*)out, units, blocks, r);
    } else {
        const int64_t units = bytes / 2;
        hipLaunchKernelGGL(repeat_kv_fwd_kernel<uint16_t>, dim3(grid_for(units * blocks * r)), dim3(256), 0, st,
                           (const uint16_t*)kv, (uint16_t*)out, units, blocks, r);
    }
    return hipGetLastError();
}

hipError_t launch_repeat_kv_bwd(const float* g, float* dkv, int64_t B, int64_t Hkv, int64_t S, int64_t D,
                                int64_t r, hipStream_t st) {
    const int64_t elems = S * D;
    hipLaunchKernelGGL(repeat_kv_bwd_kernel, dim3(grid_for(elems * B * Hkv)), dim3(256), 0, st, g, dkv, elems,
                       B * Hkv, r);
    return hipGetLastError();
}

}  // namespace mft
