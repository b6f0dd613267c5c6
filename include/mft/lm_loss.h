/*
 * mft/lm_loss.h — C ABI of the language-model cross-entropy on gfx950.
 *
 * Replaces, for tensors resident on the GPU:
 *
 *   ops::lm_cross_entropy(logits [B,S,V], labels [B,S], ignore_index, reduction)
 *       core/lm_loss.h:31-34, core/lm_loss.cpp:268-382, and its backward
 *       LMCrossEntropyBackward (core/lm_loss.cpp:74-163)
 *   ops::selected_token_lm_cross_entropy / ops::streaming_lm_cross_entropy
 *       (hidden [B,S,H], lm_head_weight [V,H], labels) without dense logits
 *       core/lm_loss.h:36-69, core/lm_loss.cpp:384-481, and its backward
 *       SelectedTokenLMCrossEntropyBackward (core/lm_loss.cpp:165-266)
 *
 * Semantics are the reference's: HF-style shift (logits at position s are
 * scored against labels[b, s + 1]; position S - 1 scores nothing), labels
 * equal to ignore_index are skipped, "mean" divides by the number of scored
 * positions (NaN when there are none), "none" returns a per-position [B, S]
 * NLL with 0 at unscored positions (dense variant only, as in the reference).
 *
 * Conventions are those of mft/attention.h (status codes, mft_last_error,
 * caller-owned device memory, stream ordering).  With bf16 hidden and weight
 * and H a multiple of 64 the streaming forward is one fused kernel (the logits
 * GEMM with the online log-sum-exp in its epilogue; no logits are written),
 * and the backward's per-chunk G comes from the same kernel (logits
 * recomputed, G written in bf16).  The backward's two GEMMs per chunk, and the
 * logits GEMMs in the other cases, run on rocBLAS with a per-device handle
 * created on first use; the GEMM workspace comes from the caller's workspace.
 *
 * A label outside [0, V) that is not ignore_index makes the reference throw
 * ("lm_cross_entropy: label out of range").  A device cannot throw: the
 * forward then writes 1 to *status (if status is not NULL) and NaN to the
 * loss; callers raise from that.
 */
#ifndef MFT_LM_LOSS_H
#define MFT_LM_LOSS_H

#include "mft/attention.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum { MFT_REDUCE_MEAN = 0, MFT_REDUCE_SUM = 1, MFT_REDUCE_NONE = 2 } mft_reduction;

typedef struct {
    int64_t B, S, V;       /* labels [B, S]; dense logits [B, S, V]                      */
    int64_t H;             /* streaming: hidden [B, S, H], weight [V, H]; 0 for dense    */
    int32_t dtype;         /* element type of logits (dense) or hidden and weight         */
    int32_t ignore_index;  /* skipped label value (reference default -100)                */
    int32_t reduction;     /* mft_reduction; streaming takes MEAN or SUM                  */
    int32_t chunk;         /* streaming: vocabulary rows per GEMM chunk (0 = 16384)        */
} mft_lm_loss_desc;

/* Workspace bytes of the forward and backward (dense or streaming per desc->H). */
mft_status mft_lm_ce_workspace_size(const mft_lm_loss_desc* desc, size_t* fwd_bytes, size_t* bwd_bytes);

/* Dense forward.  loss: [1] (MEAN, SUM) or [B, S] fp32 (NONE).  lse: [B, S]
 * fp32 row log-sum-exp for the backward (0 at unscored positions). */
mft_status mft_lm_ce_fwd(const mft_lm_loss_desc* desc, const void* logits, const int32_t* labels, float* loss,
                         float* lse, int32_t* status, void* workspace, hipStream_t stream);

/* Dense backward: grad_logits [B, S, V] fp32 = (softmax - onehot) * g, with
 * g = grad_loss[0] (or grad_loss[b, s] for NONE) / count for MEAN; rows that
 * score nothing get 0. */
mft_status mft_lm_ce_bwd(const mft_lm_loss_desc* desc, const void* logits, const int32_t* labels, const float* lse,
                         const float* grad_loss, float* grad_logits, void* workspace, hipStream_t stream);

/* Streaming forward: the same loss from hidden and weight, logits computed
 * chunk by chunk and never stored whole.  loss: [1]; lse: [B, S] as above. */
mft_status mft_lm_ce_streaming_fwd(const mft_lm_loss_desc* desc, const void* hidden, const void* weight,
                                   const int32_t* labels, float* loss, float* lse, int32_t* status, void* workspace,
                                   hipStream_t stream);

/* Streaming backward: grad_hidden [B, S, H] and grad_weight [V, H] (fp32,
 * written; either may be NULL), recomputing each logits chunk. */
mft_status mft_lm_ce_streaming_bwd(const mft_lm_loss_desc* desc, const void* hidden, const void* weight,
                                   const int32_t* labels, const float* lse, const float* grad_loss, float* grad_hidden,
                                   float* grad_weight, void* workspace, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* MFT_LM_LOSS_H */
