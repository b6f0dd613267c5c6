// Launchers of the fused q/k prologue kernels (prologue.hip; called by
// prologue_capi.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_kernels.h"

namespace mft {

enum { PROLOGUE_NORM_NONE = 0, PROLOGUE_NORM_GEMMA = 1, PROLOGUE_NORM_AFFINE = 2 };
constexpr int PROLOGUE_MAX_D = 512;

struct PrologueArgs {
    int64_t B, H, S, rows;  // rows = B * H * S
    int D;
    int norm;
    float eps;
    int rope;
    const void* x;
    Strides sx;
    const float* w;
    void* y;
    Strides sy;
    const float* dy;
    Strides sdy;
    float* dx;
    Strides sdx;
    float* dw_part;  // [workgroups, D] partials of dL/dw (backward with a norm)
    float inv_freq[PROLOGUE_MAX_D / 2];  // 1 / theta^(2d/D), d < D/2
};

// Elements of each row half a lane owns, and rows per backward wave.
constexpr int prologue_elems_per_lane(int D) { return D / 2 <= 64 ? 1 : D / 2 <= 128 ? 2 : 4; }
constexpr int prologue_bwd_rows_per_wave(int elems) { return elems >= 4 ? 2 : 4; }

// Workgroups (4 waves) of the backward launch; the dw partial buffer holds
// one row of D floats per workgroup.
int64_t prologue_bwd_blocks(int64_t rows, int D);

hipError_t launch_prologue_fwd(const PrologueArgs& a, bool is_bf16, hipStream_t st);
hipError_t launch_prologue_bwd(const PrologueArgs& a, bool is_bf16, float* dw, hipStream_t st);

}  // namespace mft
