/*
 * refcpu — CPU restatement of MobileFineTuner's causal attention composite.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity oracle for the HIP
 * kernels and the CPU baseline timed by bench.py.  Only tests/, the smoke()
 * entry and bench.py's cpu_baseline leg may load it; the product library
 * (libmft_attn.so) never links or calls it.
 *
 * Every function restates a reference operator on plain float arrays, with
 * the same floating-point operation order, so that on the same compiler the
 * results are bit-identical to the reference build (checked against
 * oracle/_ref and the golden fixtures under tests/golden/).
 *
 * Layout of every tensor: contiguous row-major [B, H, S, D] (fp32).
 */
#ifndef MFT_ORACLE_REFCPU_H
#define MFT_ORACLE_REFCPU_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- deterministic input generator (the reference randn is unseeded) ---- */
/* splitmix64(seed ^ (stream << 32) ^ counter) -> 53-bit uniform in (0,1). */
double orc_uniform(uint64_t seed, uint32_t stream, uint64_t counter);
/* x[i] = sigma * N(0,1) by Box-Muller over consecutive uniform pairs. */
void orc_fill_normal(float* x, int64_t n, uint64_t seed, uint32_t stream, float sigma);
/* Deterministic closed-form fill used by the reference unit tests:
 * x[i] = a * ((i % m) - o)   (e.g. optim/test_qkt_softmax_grad.cpp:41-42). */
void orc_fill_mod(float* x, int64_t n, float a, int m, int o);
/* K-row stress of config C4: per (b, kv) pick `count` distinct rows by a
 * partial Fisher-Yates shuffle on stream 4 and multiply them by `factor`. */
void orc_stress_rows(float* k, int64_t B, int64_t Hkv, int64_t S, int64_t D,
                     int64_t count, float factor, uint64_t seed);

/* ---- bf16 (core/dtype.h:114-128) ---- */
uint16_t orc_f32_to_bf16_bits(float x);
float orc_bf16_bits_to_f32(uint16_t b);
/* Round every value to the nearest bf16 (RNE), keeping it as float. */
void orc_round_bf16(float* x, int64_t n);
void orc_to_bf16_bits(const float* x, uint16_t* out, int64_t n);
void orc_from_bf16_bits(const uint16_t* b, float* out, int64_t n);

/* ---- the reference composite, forward + backward ----
 * Restates, per (b, h):
 *   repeat_kv_heads  (core/ops.cpp:2260-2335)       q-head h uses kv head h / (Hq/Hkv)
 *   transpose+matmul (core/ops.cpp:61-84, 619-822)  S = Q K^T, float, sequential over d
 *   mul(scale)       (core/ops.cpp:550-560)
 *   add(causal mask) (core/ops.cpp:415-442, 2167-2180)  -1e10 above the diagonal
 *   softmax(-1)      (core/ops.cpp:1307-1363)       float max / exp / sum / divide
 *   matmul(P, V)     (core/ops.cpp:61-84)
 * and the Engine backward of that graph (core/autograd_engine.cpp:144-273):
 *   MatmulBackward   (core/backward_functions.cpp:94-147)
 *   SoftmaxBackward  (core/backward_functions.cpp:306-349) double row dot
 *   AddBackward/ScaleBackward (core/backward_functions.cpp:36-72, 981-985)
 *   TransposeBackward, RepeatKVHeadsBackward (core/backward_functions.cpp:422-426, 693-726)
 * Any of o, dO/dq/dk/dv may be NULL to skip that part (dO NULL skips the
 * backward).  dk, dv are [B, Hkv, S, D] (summed over the repeated heads).
 * Returns 0 on success, -1 on bad arguments. */
int orc_attn_composite(const float* q, const float* k, const float* v, const float* dO,
                       int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D,
                       float scale, int causal,
                       float* o, float* lse, float* dq, float* dk, float* dv);

// The same with explicit additive masks (either may be NULL): base_mask
// [S,S] replaces the causal mask, pad_mask [B,S] is added after it
// (graph/gemma_model.cpp:494-499).
int orc_attn_composite_masked(const float* q, const float* k, const float* v, const float* dO,
                              int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D,
                              float scale, int causal, const float* base_mask, const float* pad_mask,
                              float* o, float* lse, float* dq, float* dk, float* dv);

/* The composite with general additive masks (the mask mode of the C ABI):
 *   mode 0: x = s * scale
 *   mode 1: x = j > i ? -1e10 : s * scale   (the no-grad operator's causal rule,
 *           core/memory_efficient_attention.cpp:163-167)
 *   mode 2: x = s * scale + (j > i ? -1e10 : 0)   (create_causal_mask added,
 *           core/ops.cpp:2167-2180)
 * then x = x + m0[b*s0[0] + h*s0[1] + i*s0[2] + j*s0[3]] and the same for m1
 * (each may be NULL; float adds in that order, ops::add's broadcast,
 * core/ops.cpp:299-377), then the composite's softmax, matmul and Engine
 * backward as orc_attn_composite.  lse2, if given, is [B,Hq,S,2]: the row max
 * and ln of the float row sum (not reference outputs: for checking the
 * kernels' row terms). */
int orc_attn_composite_masks(const float* q, const float* k, const float* v, const float* dO,
                             int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D,
                             float scale, int mode, const float* m0, const int64_t* s0,
                             const float* m1, const int64_t* s1,
                             float* o, float* lse, float* lse2, float* dq, float* dk, float* dv);

/* The no-grad streaming path of ops::memory_efficient_attention
 * (core/memory_efficient_attention.cpp:110-200): double sum_exp, float
 * inv_sum, float context accumulation.  MHA only (Hq == Hkv), as there. */
int orc_attn_streaming(const float* q, const float* k, const float* v,
                       int64_t B, int64_t H, int64_t S, int64_t D,
                       float scale, int causal, float* o);
/* The same with the operator's optional [S,S] mask added after the causal
 * replacement (core/memory_efficient_attention.cpp:169-172). */
int orc_attn_streaming_mask(const float* q, const float* k, const float* v,
                            int64_t B, int64_t H, int64_t S, int64_t D,
                            float scale, int causal, const float* mask, float* o);

/* Independent fp64 brute-force attention (textbook formula, no reference
 * op order) used as a third check.  Outputs are double. */
int orc_attn_f64(const float* q, const float* k, const float* v, const float* dO,
                 int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D,
                 double scale, int causal,
                 double* o, double* lse, double* dq, double* dk, double* dv);

/* repeat_kv_heads forward / RepeatKVHeadsBackward on float arrays. */
void orc_repeat_kv(const float* kv, float* out, int64_t B, int64_t Hkv, int64_t S,
                   int64_t D, int64_t r);
void orc_repeat_kv_backward(const float* g, float* dkv, int64_t B, int64_t Hkv,
                            int64_t S, int64_t D, int64_t r);

/* ---- q/k prologue: norm then RoPE, per row of D (layout [B, H, S, D]) ----
 * norm 0: none; 1: ops::rms_norm (core/ops.cpp:1677-1706), y = (x / rms) * (1 + w)
 * with rms = float(sqrt(double sum x^2 / D + eps)); 2: ops::rms_norm_affine
 * (core/ops.cpp:1728-1745), y = x * inv_rms * w.  Then, if theta > 0,
 * ops::apply_rope (core/ops.cpp:2337-2391): pairs (d, d + D/2), freq =
 * 1 / powf(theta, 2d/D), angle = pos * freq, cosf / sinf.  w may be NULL for
 * norm 0. */
void orc_prologue_fwd(const float* x, const float* w, int64_t B, int64_t H, int64_t S, int64_t D,
                      int norm, float eps, float theta, float* y);
/* Backward of the same chain, as the Engine runs it: ApplyRoPEBackward
 * (core/backward_functions.cpp:728-774) gives g = R^T dy, then
 * RMSNormBackward / RMSNormAffineBackward (core/backward_functions.cpp:492-575)
 * in double; dw (may be NULL) = the float sum over rows in row order. */
void orc_prologue_bwd(const float* x, const float* w, const float* dy, int64_t B, int64_t H, int64_t S,
                      int64_t D, int norm, float eps, float theta, float* dx, float* dw);

/* ---- LM cross-entropy (core/lm_loss.cpp) ----
 * Dense ops::lm_cross_entropy (:268-382) and LMCrossEntropyBackward
 * (:85-158): position (b, s) is scored against labels[b, s + 1] unless that
 * is ignore_index; reduction 0 mean, 1 sum, 2 none ([B, S] losses).
 * grad_out: [1] (mean, sum) or [B, S] (none); NULL skips the backward.
 * Returns -1 on a label outside [0, V) (the reference throws). */
int orc_lm_ce(const float* logits, const int32_t* labels, int64_t B, int64_t S, int64_t V, int ignore_index,
              int reduction, const float* grad_out, float* loss, float* grad_logits);
/* ops::selected_token_lm_cross_entropy (:384-472) and its backward
 * (:165-266) on fp32 hidden [B, S, H] and weight [V, H]: logits are dot
 * products in float, h order; reduction 0 mean, 1 sum.  grad_hidden and
 * grad_weight may be NULL. */
int orc_selected_ce(const float* hidden, const float* weight, const int32_t* labels, int64_t B, int64_t S,
                    int64_t H, int64_t V, int ignore_index, int reduction, float grad_out, float* loss,
                    float* grad_hidden, float* grad_weight);

/* ---- LoRA linear (nn/lora_linear.cpp) ----
 * n slices; meta holds 5 int64 per slice: rank, col0, cols, a_transposed,
 * b_transposed; A_all / B_all hold the slices' A ([in, rank] or [rank, in])
 * and B ([rank, cols] or [cols, rank]) back to back.  W holds the weight's
 * values ([in, out], or [out, in] with w_transposed; bf16 weights as their
 * exact fp32 values).
 * Forward (:332-444): y = matmul(x, W) (+ bias) and per slice
 * y[:, col0 ..] += mul(matmul(matmul(x, A), B), scale), each matmul with
 * the arithmetic of matmul_fallback_nn.
 * Backward (dy != NULL), the Engine's graph: g = matmul(mul(dy_slice,
 * scale), B^T), grad_B = xA^T . (scale dy_slice), grad_A = x^T . g,
 * dx = dy . W^T + sum g . A^T over the slices that have a gradient (full
 * slices, or all with all_grads); has_grad[i] says which.  dx may be NULL.
 * w_lowp: W is bf16 in the reference, whose dy . W^T then sums in 64-wide
 * blocks of k (matmul_fallback_nt_mixed_b). */
void orc_lora(const float* x, const float* W, const float* bias, int64_t N, int64_t in, int64_t out, int w_transposed,
              int w_lowp, int n, const int64_t* meta, const float* scale, const float* A_all, const float* B_all,
              int all_grads, const float* dy, float* y, float* dx, float* dA_all, float* dB_all, int32_t* has_grad);
/* apply_lora_delta_to_base (:108-138) of every slice in order, W [in, out]:
 * W[i, col0 + o] = W + (sign * scale) * float(sum_r double(A) * double(B)),
 * rounded to bf16 (core/dtype.h:114-121) after each slice when w_bf16. */
void orc_lora_merge(float* W, int w_bf16, int64_t in, int64_t out, int n, const int64_t* meta, const float* scale,
                    const float* A_all, const float* B_all, float sign);

#ifdef __cplusplus
}
#endif
#endif
