/*
 * mft/attention.h — C ABI of the MI355X (gfx950) fused causal GQA attention.
 *
 * This is the drop-in boundary for MobileFineTuner's attention hot path.  It
 * replaces, for tensors resident on the GPU:
 *
 *   ops::memory_efficient_attention(q, k, v, mask, cfg)
 *       operator/finetune_ops/core/memory_efficient_attention.h:49-55
 *       (its grad path is the composite of core/memory_efficient_attention.cpp:23-43)
 *   the composite the model graphs call directly,
 *       repeat_kv_heads -> transpose -> matmul -> mul(scale) -> add(mask)
 *       -> softmax -> matmul
 *       graph/gemma_model.cpp:481-505, graph/qwen_model.cpp:302-318
 *   and its Engine backward (MatmulBackward, SoftmaxBackward, ScaleBackward,
 *   AddBackward, TransposeBackward, RepeatKVHeadsBackward;
 *       core/backward_functions.cpp:36-147, 306-349, 422-426, 693-726, 981-985)
 *   ops::repeat_kv_heads / RepeatKVHeadsBackward
 *       core/ops.h:177, core/ops.cpp:2260-2335, core/backward_functions.cpp:693-726
 *
 * Conventions
 *   - Tensors are [B, H, S, D] in device memory: contiguous row-major (the
 *     reference Tensor is contiguous row-major, core/tensor.h:78-237) unless the
 *     descriptor gives strides (mft_strides), e.g. for [B, S, H, D] views.
 *   - q, o, dO have Hq heads; k, v, dk, dv have Hkv heads; Hq % Hkv == 0 and
 *     q-head h reads kv head h / (Hq / Hkv) (core/ops.cpp:2283-2284).
 *   - Element type of q, k, v, o, dO: MFT_F32 or MFT_BF16.  lse, dq, dk, dv
 *     are always fp32: the reference Engine accumulates gradients as float
 *     only (core/autograd_engine.cpp:135-140).
 *   - lse[b, h, i] = log(sum_j exp(scale * q_i . k_j)) over the visible keys
 *     (natural log, fp32, [B, Hq, S]).  The backward recomputes the softmax
 *     from it; no S x S tensor is ever stored.
 *   - All pointers are caller-owned device memory, 16-byte aligned; no call
 *     allocates device memory.  The workspace of mft_attn_bwd_noalloc, a
 *     fixed 128 MiB __device__ array, sits in a code object of its own (no
 *     kernel shares it), which the HIP runtime loads on a GPU at that entry
 *     point's first call there (deferred code-object loading, the ROCm
 *     default; with HIP_ENABLE_DEFERRED_LOADING=0 every code object loads
 *     with the library).  Work is enqueued on `stream` (NULL = the null
 *     stream) and is ordered there; the calls return before the GPU finishes.
 *   - Errors: a non-zero mft_status, and mft_last_error() returns a
 *     thread-local message.  The C++ adapter rethrows it as the reference's
 *     TensorError / std::runtime_error (core/memory_efficient_attention.cpp:86-99).
 *   - Thread safety: stateless; calls on different streams may overlap.
 */
#ifndef MFT_ATTENTION_H
#define MFT_ATTENTION_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    MFT_OK = 0,
    MFT_ERR_INVALID_ARG = 1, /* null pointer, bad shape, Hq % Hkv != 0 ...          */
    MFT_ERR_UNSUPPORTED = 2, /* valid request the kernels do not cover (D > 256)     */
    MFT_ERR_HIP = 3          /* a HIP runtime call failed (launch error, ...)         */
} mft_status;

/* Values match ops::DType (core/dtype.h:9-18): kFloat32 = 0, kBFloat16 = 2. */
typedef enum { MFT_F32 = 0, MFT_BF16 = 2 } mft_dtype;

/* Element strides of an operand's batch, head and sequence dimensions; its head
 * dim is contiguous, so element (b, h, s, d) lives at b*b + h*h + s*s + d.
 * All zero = contiguous [B, H, S, D].  Strides let callers pass the models'
 * [B, S, H, D] projection layout (graph/gemma_model.cpp:403-409, 506-508 and
 * graph/qwen_model.cpp:290-299 permute it to [B, H, S, D] with a copy) as a view:
 * b = S*H*D, h = D, s = H*D.  Every stride must be a multiple of 16 bytes.
 * The bf16 backward's fast kernels need k and v to share the sequence stride
 * (as contiguous tensors, [B, S, Hkv, D] views and fused-QKV slices do);
 * otherwise the general kernels run, with the same results to the tolerance
 * and at lower speed. */
typedef struct {
    int64_t b, h, s;
} mft_strides;

/* An additive mask (mask mode): element (b, h, i, j) - batch, query head,
 * query row, key - is ptr[b*sb + h*sh + i*si + j*sj], fp32 device memory
 * (4-byte aligned); a zero stride broadcasts that dimension, so an [S, S] mask
 * is (0, 0, S, 1) and a [B, 1, 1, S] padding mask (S, 0, 0, 1).  ptr = NULL:
 * no mask. */
typedef struct {
    const float* ptr;
    int64_t sb, sh, si, sj;
} mft_mask;

typedef struct {
    int64_t B, Hq, Hkv, S, D; /* batch, query heads, kv heads, sequence, head dim     */
    float scale;              /* > 0: softmax scale; <= 0: 1/sqrt(D), as
                                 MemoryEfficientAttentionConfig::scale
                                 (core/memory_efficient_attention.h:26-31, .cpp:103) */
    int32_t causal;           /* 1: key j visible to query i iff j <= i (the -1e10
                                 mask of core/ops.cpp:2167-2180); 0: all visible      */
    mft_dtype dtype;          /* element type of q, k, v, o, dO                        */
    int32_t window;           /* > 0 (needs causal = 1): also i - j < window, the
                                 Gemma sliding mask (graph/gemma_model.cpp:272-285,
                                 config sliding_window); 0: no window.  A window
                                 >= S is the plain causal mask.                       */
    const int32_t* kv_len;    /* NULL, or device int32 [B]: keys j >= kv_len[b] are
                                 hidden in batch b, the padding mask of an
                                 attention_mask that is 1 on the first kv_len[b]
                                 positions (graph/gemma_model.cpp:287-320,
                                 graph/qwen_model.cpp:338-353; the datasets pad on
                                 the right, data/wikitext2_dataset.cpp:461-500).
                                 Values are clamped to [0, S].                        */
    mft_strides q, k, v, o;   /* layouts of q, k, v, o (see mft_strides)              */
    mft_strides dO, dq, dk, dv; /* layouts of dO and the gradients (backward)          */
    mft_mask mask0, mask1;    /* Mask mode (either non-NULL): the scores are
                                 x = (causal && j > i ? -1e10 : scale * q_i.k_j),
                                 then x += mask0, then x += mask1 (float adds, in
                                 that order), and the softmax runs over every key.
                                 causal = 1 is the no-grad operator's rule
                                 (core/memory_efficient_attention.cpp:163-172:
                                 -1e10 above the diagonal, then the mask added);
                                 the grad path's composite (:29-38) ignores the
                                 causal flag when given a mask, i.e. causal = 0
                                 here.  Any mask values are taken (rows masked
                                 everywhere by one value get a uniform softmax, as
                                 in the reference).  window must be 0 and kv_len
                                 NULL (the masks express them).  The general
                                 kernels run (no fast path).  lse then holds two
                                 floats per row: [B, Hq, S, 2] = (max of the row's
                                 scores, ln of the sum of exp(x - max)).          */
} mft_attn_desc;

/* Rows with no visible key.  With kv_len a query row can see no key (every
 * row when kv_len[b] = 0; with a window, rows i >= kv_len[b] + window - 1).
 * The reference's -1e10 masks then leave a uniform softmax over the keys
 * hidden by exactly one of its two masks; o, and the gradients, follow that
 * (see mobilefinetuner_amd/csrc/attn_masked_rows.hip), and lse is +inf for
 * such rows. */

/* Workspace bytes of the calls.
 *   fwd: fp32 partial output tiles of query tiles whose key range is split
 *        across work units (the fast paths: bf16 with D % 8 == 0 and fp32
 *        with D % 4 == 0, 32 < D <= 256; 0 for the others, and for bf16
 *        shapes whose query tiles alone fill half the GPU or more and see at
 *        most 16 key tiles each (causal S <= 1024, or a short sliding
 *        window), which run one workgroup per query tile).  The forward also
 *        accepts workspace = NULL and then runs one workgroup per query tile
 *        (same results within the dtype's tolerance; no cross-unit load
 *        balancing, and for fp32 the general kernels).
 *   bwd: per-row softmax terms and the fp32 partials of split tiles.
 * Replaces: nothing (the reference allocates from its pool implicitly). */
mft_status mft_attn_workspace_size(const mft_attn_desc* desc, size_t* fwd_bytes,
                                   size_t* bwd_bytes);

/* Forward: o = softmax(scale * q k^T [masks]) v, and lse.
 * Replaces the composite forward / memory_efficient_attention
 * (core/memory_efficient_attention.cpp:73-203 and :23-43).
 * lse may be NULL when no backward will follow (no-grad path).
 * workspace: fwd_bytes from mft_attn_workspace_size, or NULL (see there). */
mft_status mft_attn_fwd(const mft_attn_desc* desc, const void* q, const void* k,
                        const void* v, void* o, float* lse, void* workspace,
                        hipStream_t stream);

/* Backward: dq, dk, dv of sum(o * dO), recomputing P from lse.
 * dk, dv are [B, Hkv, S, D]: already summed over the Hq/Hkv query heads that
 * share each kv head (RepeatKVHeadsBackward folded in).
 * Replaces Engine::run_backward over the composite's nodes
 * (core/autograd_engine.cpp:144-273 with the backward functions cited above). */
mft_status mft_attn_bwd(const mft_attn_desc* desc, const void* q, const void* k,
                        const void* v, const void* o, const void* dO, const float* lse,
                        float* dq, float* dk, float* dv, void* workspace,
                        hipStream_t stream);

/* Backward that allocates nothing and takes no workspace: the same kernels as
 * mft_attn_bwd, with the workspace in a library-owned device array of a fixed
 * 128 MiB per GPU, taken at the first call on that GPU and held until the
 * process ends.  Shapes whose backward
 * workspace (mft_attn_workspace_size) exceeds that return MFT_ERR_UNSUPPORTED
 * with a message.  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams, other threads) race.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). */
mft_status mft_attn_bwd_noalloc(const mft_attn_desc* desc, const void* q, const void* k,
                                const void* v, const void* o, const void* dO, const float* lse,
                                float* dq, float* dk, float* dv, hipStream_t stream);

/* The backward's stages, as a bit mask for mft_attn_bwd_stage.
 *   DELTA : per-row softmax terms (delta_i = dO_i . O_i) into the workspace
 *   DKDV  : dK and dV
 *   DQ    : dQ
 *           (asked for together, DKDV and DQ run as one launch whose work
 *           units of both kinds fill the GPU together; alone, each is one
 *           launch of the same units)
 *   REDUCE: sums the fp32 partials of tiles split across work units, and
 *           with kv_len writes the terms of rows with no visible key
 * MAIN = DKDV | DQ.  mft_attn_bwd == mft_attn_bwd_stage(MFT_BWD_ALL).
 * Callers may run the stages separately on one stream, DELTA first and REDUCE
 * last (e.g. to time them, or to start DELTA early); later stages read what
 * earlier ones wrote into the same workspace. */
enum {
    MFT_BWD_DELTA = 1,
    MFT_BWD_DKDV = 2,
    MFT_BWD_REDUCE = 4,
    MFT_BWD_DQ = 8,
    MFT_BWD_MAIN = 10,
    MFT_BWD_ALL = 15
};

/* Backward, selected stages only (same arguments as mft_attn_bwd).
 * Replaces: the same Engine backward as mft_attn_bwd, split into launches. */
mft_status mft_attn_bwd_stage(const mft_attn_desc* desc, int stages, const void* q,
                              const void* k, const void* v, const void* o, const void* dO,
                              const float* lse, float* dq, float* dk, float* dv,
                              void* workspace, hipStream_t stream);

/* repeat_kv_heads forward: out[b, h*r + i] = kv[b, h] for i < r
 * ([B,Hkv,S,D] -> [B,Hkv*r,S,D], element type `dtype`).
 * Replaces ops::repeat_kv_heads (core/ops.cpp:2260-2335). */
mft_status mft_repeat_kv_fwd(const void* kv, void* out, int64_t B, int64_t Hkv, int64_t S,
                             int64_t D, int64_t r, mft_dtype dtype, hipStream_t stream);

/* repeat_kv_heads backward: dkv[b, h] = sum_{i<r} g[b, h*r + i] (fp32,
 * float accumulation in i order).
 * Replaces RepeatKVHeadsBackward::apply (core/backward_functions.cpp:693-726). */
mft_status mft_repeat_kv_bwd(const float* g, float* dkv, int64_t B, int64_t Hkv, int64_t S,
                             int64_t D, int64_t r, hipStream_t stream);

/* Message of the last failing call on this thread ("" if none). */
const char* mft_last_error(void);

/* Element conversion on the device: MFT_BF16 -> MFT_F32 (exact) or MFT_F32 ->
 * MFT_BF16 with the reference's round-to-nearest-even
 * (float32_to_bf16_bits, core/dtype.h:114-121).  n elements; src and dst
 * 16-byte aligned device memory.  No counterpart in the reference, which
 * converts on the host (ops::cast, core/ops.cpp:2894-2952, and the adapters'
 * tensor reads): it lets the drop-in widen the bf16 output and round the fp32
 * incoming gradient on the GPU instead of in host loops. */
mft_status mft_convert(const void* src, mft_dtype src_dtype, void* dst, mft_dtype dst_dtype,
                       int64_t n, hipStream_t stream);

/* Library version, for the bindings' sanity check. */
int mft_version(void);

#ifdef __cplusplus
}
#endif
#endif /* MFT_ATTENTION_H */
