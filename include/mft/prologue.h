/*
 * mft/prologue.h — C ABI of the fused q/k prologue of the attention (gfx950).
 *
 * One pass over a projection's output produces the attention's input:
 *
 *   y = rope(norm(x))        per row (b, h, s) of D elements
 *
 * replacing, for tensors resident on the GPU, the chain the model graphs run
 * between the q/k projections and the attention:
 *
 *   permute [B,S,H,D] -> [B,H,S,D]      graph/gemma_model.cpp:403-409,
 *                                       graph/qwen_model.cpp:293-299
 *   ops::rms_norm (Gemma: x / rms * (1 + w))
 *       core/ops.cpp:1677-1725, called at graph/gemma_model.cpp:459-460
 *   ops::rms_norm_affine (x / rms * w)  core/ops.cpp:1728-1762
 *   ops::apply_rope (rotate-half pairs (d, d + D/2), theta^(-2d/D))
 *       core/ops.cpp:2337-2414, called at graph/gemma_model.cpp:470-471 and
 *       graph/qwen_model.cpp:308-309
 *
 * and, backward, ApplyRoPEBackward::apply (core/backward_functions.cpp:728-774)
 * followed by RMSNormBackward::apply / RMSNormAffineBackward::apply
 * (core/backward_functions.cpp:492-532, 534-575).
 *
 * Conventions are those of mft/attention.h (status codes, mft_last_error,
 * caller-owned 16-byte aligned device memory, stream ordering, no
 * allocation).  x and y have element type `dtype`; w, dy, dx, dw are fp32.
 * Row (b, h, s) has RoPE position s.  Qwen applies RoPE after repeat_kv_heads;
 * RoPE acts on each row alone, so applying it to the Hkv un-repeated heads
 * gives the same rows.
 */
#ifndef MFT_PROLOGUE_H
#define MFT_PROLOGUE_H

#include "mft/attention.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    MFT_NORM_NONE = 0,   /* y = rope(x)                                   */
    MFT_NORM_GEMMA = 1,  /* ops::rms_norm: x / rms * (1 + w)              */
    MFT_NORM_AFFINE = 2  /* ops::rms_norm_affine: x * (1 / rms) * w       */
} mft_norm;

typedef struct {
    int64_t B, H, S, D;  /* D even, 2 <= D <= 512                          */
    int32_t dtype;       /* mft_dtype of x and y                           */
    int32_t norm;        /* mft_norm                                       */
    float eps;           /* rms = sqrt(mean(x^2) + eps)                    */
    float theta;         /* RoPE base (rope_theta); 0 = no RoPE            */
    /* Layouts, as in mft_attn_desc (all zero = contiguous [B, H, S, D]). */
    mft_strides x, y, dy, dx;
} mft_prologue_desc;

/* Forward: y = rope(norm(x)).  w ([D], fp32) may be NULL only with
 * MFT_NORM_NONE. */
mft_status mft_prologue_fwd(const mft_prologue_desc* desc, const void* x, const float* w, void* y,
                            hipStream_t stream);

/* Bytes of device workspace mft_prologue_bwd needs (0 without a norm). */
mft_status mft_prologue_workspace_size(const mft_prologue_desc* desc, size_t* bytes);

/* Backward: dx = dL/dx from dy = dL/dy, recomputing the row norms from x.
 * With a norm, dw ([D], fp32) receives dL/dw summed over all rows (written,
 * not accumulated; NULL skips it).  dx may not alias x or dy. */
mft_status mft_prologue_bwd(const mft_prologue_desc* desc, const void* x, const float* w, const float* dy,
                            float* dx, float* dw, void* workspace, hipStream_t stream);

/* Batched forms: n (1 or 2) independent prologues in one launch per
 * direction, such as a layer's q heads and k heads (graph/gemma_model.cpp:
 * 459-471 runs rms_norm and apply_rope on each).  Tensor i has descs[i] and
 * the i-th pointer of every array; the results are those of n calls of
 * mft_prologue_fwd / mft_prologue_bwd, bit for bit.  Every tensor of a batch
 * has one dtype; they run as one launch when they share a head dim of 128,
 * 256 or 512 with 16-byte-aligned rows, else one launch each.  The backward
 * workspace (mft_prologue_workspace_size_n) holds every tensor's dw
 * partials; dw[i] may be NULL.  No counterpart in the reference, which runs
 * the two chains one after the other. */
mft_status mft_prologue_fwd_n(int n, const mft_prologue_desc* descs, const void* const* x, const float* const* w,
                              void* const* y, hipStream_t stream);
mft_status mft_prologue_workspace_size_n(int n, const mft_prologue_desc* descs, size_t* bytes);
mft_status mft_prologue_bwd_n(int n, const mft_prologue_desc* descs, const void* const* x, const float* const* w,
                              const float* const* dy, float* const* dx, float* const* dw, void* workspace,
                              hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* MFT_PROLOGUE_H */
