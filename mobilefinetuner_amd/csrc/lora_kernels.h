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

// Rank-r products with a long inner dimension, which library GEMMs run on a
// handful of workgroups.  P(k, j) = P[k * pk + j * pj] describes A_eff / B_eff
// in either stored layout.
struct LoraRowDot {
    const float* M;        // [rows, K] with leading dimension ldm
    int64_t ldm, rows, K;
    const float* P;
    int64_t pk, pj;
    float* out;            // [rows, r] with leading dimension ldo
    int64_t ldo;
    int r;
    float alpha;
    uint16_t* mb;          // optional: bf16 (RNE) copy of M[:, :K], leading dimension ldb
    int64_t ldb;
};
// out[n, j] = alpha * sum_k M[n, k] P(k, j); with mb, also mb[n * ldb + k] =
// bf16(M[n, k]) from the same loads (M is read once).
hipError_t launch_lora_rowdot(const LoraRowDot& a, hipStream_t st);
// dst[j * K + k] = P(k, j) for k < K, j < r: the k-contiguous copy rowdot
// reads with coalesced loads when P is not k-contiguous already.
hipError_t launch_lora_pack_kmajor(const float* P, int64_t pk, int64_t pj, int64_t K, int r, float* dst,
                                   hipStream_t st);

constexpr int64_t kLoraMaxGridY = 65535;  // a launch's grid limit in y (and z)

struct LoraColDot {
    const float* M;        // [rows, K] with leading dimension ldm
    int64_t ldm, rows, K;
    const float* V;        // [rows, r] with leading dimension ldv
    int64_t ldv;
    int r;
    float alpha;
    float* partial;        // workspace: lora_coldot_partial_floats(rows, K, r)
    float* out;            // out[k * ok + j * oj]
    int64_t ok, oj;
};
// out(k, j) = alpha * sum_n M[n, k] V[n, j]: per row-chunk partial sums, then
// one fixed-order sum over the chunks (deterministic).
hipError_t launch_lora_coldot(const LoraColDot& a, hipStream_t st);
int64_t lora_coldot_partial_floats(int64_t rows, int64_t K, int r);

// Rows per chunk of lora_coldot (one grid row, blockIdx.y, per chunk): 16 to
// 128, doubled while more than about 2048 waves would run, and never so few
// that the chunk count passes the grid's 65535 limit in y (rows beyond
// 65535 * 128 = ~8.4M take taller chunks).
inline int64_t lora_coldot_chunk(int64_t rows, int64_t K) {
    const int64_t col_waves = (K + 255) / 256;
    int64_t chunk = 16;
    while (chunk < 128 && col_waves * ((rows + chunk - 1) / chunk) > 2048) chunk *= 2;
    const int64_t min_chunk = (rows + kLoraMaxGridY - 1) / kLoraMaxGridY;
    return chunk > min_chunk ? chunk : min_chunk;
}

}  // namespace mft
