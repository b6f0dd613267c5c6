/*
 * mft/lora.h — C ABI of the LoRA-augmented linear layer on gfx950.
 *
 * Replaces, for tensors resident on the GPU:
 *
 *   ops::LoRALinear::forward(x [B,S,in])            nn/lora_linear.cpp:332-444
 *       y = x . W + b + sum_i scale_i * (x . A_i) . B_i
 *     and its Engine backward (the graph of matmul / mul / add it builds:
 *     MatmulBackward core/backward_functions.cpp:94-160; W and b frozen)
 *   ops::LoRALinear::merge_to_base / unmerge_from_base  nn/lora_linear.cpp:446-495
 *       W[:, col0 + o] += sign * scale * sum_r A[:, r] B[r, o]
 *       (apply_lora_delta_to_base, nn/lora_linear.cpp:108-138)
 *
 * Shapes and types follow the reference's matmul, which needs an fp32 left
 * operand (core/ops.cpp:634-636): x, b, y, dy, dx, A, B and their gradients
 * are fp32.  W is fp32 or bf16 (frozen; a low-precision W cannot be trained in
 * the reference either, core/ops.cpp:640-642), stored [in, out], or [out, in]
 * with w_transposed (the reference's matmul transposes such a W on the fly,
 * core/ops.cpp:649-654).  A_i is [in, rank] or, with a_transposed, [rank, in];
 * B_i is [rank, cols] or, with b_transposed, [cols, rank] (the reference
 * infers these from the shapes, nn/lora_linear.cpp:52-88).  Slice i adds its
 * [N, cols] delta into columns col0 .. col0 + cols - 1 of y.
 *
 * Arithmetic.  W fp32: every GEMM is an fp32 rocBLAS GEMM.  W bf16: the
 * products with W run on the bf16 MFMA path (x, resp. dy, rounded to bf16 to
 * nearest even; fp32 accumulation); the LoRA branch stays fp32.
 *
 * Gradients.  The reference tracks a slice's delta through autograd only when
 * it covers all columns (col0 == 0 and cols == out, nn/lora_linear.cpp:417-
 * 434); a slice over a column range is added to y's storage in place and gets
 * no gradient (nor does it add to dx).  grads_for_column_slices = 0 keeps
 * that behaviour; 1 gives every slice its gradient.
 *
 * Conventions are those of mft/attention.h (status codes, mft_last_error,
 * caller-owned device memory, stream ordering).  The GEMMs run through
 * rocBLAS on a per-device handle created on first use, with the GEMM
 * workspace taken from the caller's workspace.
 */
#ifndef MFT_LORA_H
#define MFT_LORA_H

#include "mft/attention.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    const float* A;        /* [in, rank], or [rank, in] with a_transposed            */
    const float* B;        /* [rank, cols], or [cols, rank] with b_transposed        */
    float* grad_A;         /* backward output in A's layout, or NULL                 */
    float* grad_B;         /* backward output in B's layout, or NULL                 */
    float scale;           /* alpha / rank                                           */
    int32_t a_transposed;
    int32_t b_transposed;
    int64_t rank;
    int64_t col0;          /* first column of y the slice adds into                  */
    int64_t cols;          /* columns of the slice (B's output width)                */
} mft_lora_slice;

typedef struct {
    int64_t N;             /* rows of x and y (B * S)                                */
    int64_t in_dim;        /* columns of x                                           */
    int64_t out_dim;       /* columns of y                                           */
    int32_t w_dtype;       /* MFT_F32 or MFT_BF16                                    */
    int32_t w_transposed;  /* W stored [out, in]                                     */
    int32_t n_slices;      /* 0 = plain linear (a merged layer)                      */
    int32_t grads_for_column_slices;
    const mft_lora_slice* slices; /* host array of n_slices                          */
} mft_lora_desc;

/* Workspace bytes of the forward and backward. */
mft_status mft_lora_workspace_size(const mft_lora_desc* desc, size_t* fwd_bytes, size_t* bwd_bytes);

/* Forward.  x [N, in], W per desc, bias [out] or NULL, y [N, out] fp32.
 * u: [N, R] fp32 with R = sum of the ranks, receives x . A_i of slice i in
 * columns (sum of earlier ranks) .. + rank_i for the backward; NULL when no
 * backward follows. */
mft_status mft_lora_fwd(const mft_lora_desc* desc, const float* x, const void* W, const float* bias, float* y,
                        float* u, void* workspace, hipStream_t stream);

/* Backward from dy [N, out] fp32.  dx [N, in] (NULL: x needs no gradient);
 * grad_A / grad_B of each slice through desc->slices (overwritten, not
 * accumulated).  u is the forward's output. */
mft_status mft_lora_bwd(const mft_lora_desc* desc, const float* x, const void* W, const float* dy, const float* u,
                        float* dx, void* workspace, hipStream_t stream);

/* W += sign * scale_i * A_i . B_i over each slice's columns, in W's dtype:
 * the rank sum in double, then one fp32 add, then (bf16 W) rounding to nearest
 * even, element for element as apply_lora_delta_to_base.  sign is +1 (merge)
 * or -1 (the reference's unmerge without a backup). */
mft_status mft_lora_merge(const mft_lora_desc* desc, void* W, float sign, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MFT_LORA_H */
