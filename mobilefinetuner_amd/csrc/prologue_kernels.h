// Launchers of the fused q/k prologue kernels (prologue.hip; called by
// prologue_capi.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_kernels.h"

namespace mft {

enum { PROLOGUE_NORM_NONE = 0, PROLOGUE_NORM_GEMMA = 1, PROLOGUE_NORM_AFFINE = 2 };
constexpr int PROLOGUE_MAX_D = 512;

// n / d for 0 <= n < 2^31 as one multiply and a shift.  With l = ceil(log2 d)
// and m = ceil(2^(31 + l) / d) (below 2^32), floor(n m / 2^(31 + l)) =
// floor(n / d): n m / 2^(31 + l) = n / d + n e / (d 2^(31 + l)) with
// e = m d - 2^(31 + l) < d <= 2^l, so the excess is below 1 / d and cannot
// carry past the next integer.
struct FastDiv {
    uint32_t d, m;
    int sh;
    static FastDiv make(uint32_t d) {
        int l = 0;
        while ((uint64_t(1) << l) < d) ++l;
        const uint64_t p = uint64_t(1) << (31 + l);
        return FastDiv{d, (uint32_t)((p + d - 1) / d), 31 + l};
    }
    __host__ __device__ uint32_t div(uint32_t n) const { return (uint32_t)(((uint64_t)n * m) >> sh); }
};

struct PrologueArgs {
    int64_t B, H, S, rows;  // rows = B * H * S
    FastDiv fh, fs;         // division by H and by S (rows32)
    int rows32;             // rows < 2^31: 32-bit row addressing
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

// Tensors one launch of the 16-byte-lane kernels takes (the q and the k
// heads of a layer): tensor i runs workgroups first_block[i] ..
// first_block[i + 1] - 1, each computing what the workgroup of that index
// computes in a launch of its own.
constexpr int kPrologueMaxBatch = 2;
struct PrologueBatch {
    PrologueArgs a[kPrologueMaxBatch];
    int64_t first_block[kPrologueMaxBatch + 1];
    int n;
};

// n (1 <= n <= kPrologueMaxBatch) tensors of one dtype: one launch per
// direction when the 16-byte-lane kernel takes them all (same head dim,
// aligned rows), otherwise one per tensor.  dw[i]: tensor i's dL/dw (NULL:
// none), reduced from its a[i].dw_part.
hipError_t launch_prologue_fwd(const PrologueArgs* a, int n, bool is_bf16, hipStream_t st);
hipError_t launch_prologue_bwd(const PrologueArgs* a, int n, bool is_bf16, float* const* dw, hipStream_t st);

}  // namespace mft
