// Shared device definitions for the gfx950 attention kernels.
//
// MFMA shapes used (CDNA4, 64-lane waves):
//   v_mfma_f32_32x32x16_bf16 : A,B = 8 bf16 per lane, C = 16 fp32 per lane
//   v_mfma_f32_32x32x2_f32   : A,B = 1 fp32 per lane,  C = 16 fp32 per lane
// Lane l = 32*hh + n (n = l % 32, hh = l / 32).
//   A operand: lane holds row i = n, reduction slots owned by half hh.
//   B operand: lane holds column n, the same reduction slots (half hh).
//   C (32x32): lane holds column n, rows 8*(r/4) + 4*hh + (r%4), r = 0..15.
// A reduction index only has to be assigned to the same (hh, slot) in A and
// B; the kernels exploit that to feed the C registers of one product
// straight into the B operand of the next (see row_of_reg()).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mft {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef __bf16 bf16x4 __attribute__((__vector_size__(4 * sizeof(__bf16))));
typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));
typedef float f32x4 __attribute__((__vector_size__(4 * sizeof(float))));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Element traits: a "vec" is one 16-byte chunk of a row.
template <typename T> struct Elt;
template <> struct Elt<float> {
    static constexpr int VEC = 4;
    typedef f32x4 vec;
};
template <> struct Elt<bf16> {
    static constexpr int VEC = 8;
    typedef bf16x8 vec;
};

// C-register r of a 32x32 accumulator on lane half hh -> row/column index
// (0..31) along the accumulator's M dimension.
__device__ __forceinline__ constexpr int row_of_reg(int r, int hh) {
    return 8 * (r >> 2) + 4 * hh + (r & 3);
}

__device__ __forceinline__ f32x16 mfma_bf16(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma_f32(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// One 16-byte chunk pair of a dot product: bf16 = one 32x32x16 MFMA over the
// 8 values each half holds; fp32 = four 32x32x2 MFMAs, one per value.
__device__ __forceinline__ f32x16 mfma_chunk(bf16x8 a, bf16x8 b, f32x16 c) {
    return mfma_bf16(a, b, c);
}
__device__ __forceinline__ f32x16 mfma_chunk(f32x4 a, f32x4 b, f32x16 c) {
    c = mfma_f32(a[0], b[0], c);
    c = mfma_f32(a[1], b[1], c);
    c = mfma_f32(a[2], b[2], c);
    c = mfma_f32(a[3], b[3], c);
    return c;
}

__device__ __forceinline__ f32x16 zero16() {
    f32x16 z;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = 0.f;
    return z;
}

template <typename V> __device__ __forceinline__ V zero_vec() {
    V z;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(V) / sizeof(z[0])); ++i) z[i] = 0;
    return z;
}

// Load the 16-byte chunk starting at column d0 of a row of length D.
// vec_ok: D is a multiple of the chunk width and the row base is 16-byte
// aligned, so a whole in-range chunk can be read as one vector.  Columns
// >= D and rows that do not exist read as zero.
template <typename T>
__device__ __forceinline__ typename Elt<T>::vec load_chunk(const T* __restrict__ row, int d0, int D,
                                                          bool row_ok, bool vec_ok) {
    typedef typename Elt<T>::vec V;
    constexpr int W = Elt<T>::VEC;
    V r = zero_vec<V>();
    if (row_ok && d0 < D) {
        if (vec_ok) {
            r = *reinterpret_cast<const V*>(row + d0);
        } else {
#pragma unroll
            for (int i = 0; i < W; ++i)
                if (d0 + i < D) r[i] = row[d0 + i];
        }
    }
    return r;
}

// Store 4 consecutive values (columns d0..d0+3) of an output row.
template <typename T>
__device__ __forceinline__ void store4(T* __restrict__ row, int d0, int D, float a, float b, float c,
                                       float d, bool vec4_ok) {
    if (d0 >= D) return;
    if (vec4_ok) {
        if constexpr (sizeof(T) == 4) {
            f32x4 v = {a, b, c, d};
            *reinterpret_cast<f32x4*>(row + d0) = v;
        } else {
            bf16x4 v = {(bf16)a, (bf16)b, (bf16)c, (bf16)d};
            *reinterpret_cast<bf16x4*>(row + d0) = v;
        }
    } else {
        const float x[4] = {a, b, c, d};
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (d0 + i < D) row[d0 + i] = (T)x[i];
    }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float other_half(float x) { return __shfl_xor(x, 32); }

}  // namespace mft
