// Launchers of the cross-entropy kernels (lm_loss.hip; called by
// lm_loss_capi.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mft {

enum { CE_MEAN = 0, CE_SUM = 1, CE_NONE = 2 };

struct CeArgs {
    int64_t B, S, V, N;     // N = B * S positions
    int ignore, reduction;
    const int32_t* labels;  // [B, S]
    // per-row state (workspace)
    float* run_m;           // running max of the row's logits
    double* run_s;          // running sum of exp(z - run_m)
    float* tgt;             // the row's target logit
    double* nll;            // per-row NLL (0 when unscored)
    long long* count;       // scored rows
    // outputs / inputs
    float* lse;             // [N] written by the forward (may be null)
    const float* lse_in;    // [N] read by the backward
    float* loss;            // [1] or [N] (NONE)
    const float* grad_loss; // [1] or [N] (NONE); null = 1
    int32_t* status;        // set to 1 on an out-of-range label (may be null)
};

// Row statistics of a [N, ncols] block of logits (row stride ld) holding
// vocabulary columns [v0, v0 + ncols); first = start the running pair.
hipError_t launch_ce_stats(const CeArgs& a, const void* z, bool z_bf16, int64_t ld, int64_t ncols, int64_t v0,
                           bool first, hipStream_t st);
// lse, per-row nll, count and the loss.
hipError_t launch_ce_finalize(const CeArgs& a, hipStream_t st);
// count of scored rows only (backward).
hipError_t launch_ce_count(const CeArgs& a, hipStream_t st);
// g[n, v] = (exp(z - lse) - onehot) * coeff for a block of columns.
hipError_t launch_ce_grad(const CeArgs& a, const void* z, bool z_bf16, int64_t ld, int64_t ncols, int64_t v0, void* g,
                          bool g_bf16, int64_t ldg, hipStream_t st);

// Fused streaming forward (lm_loss_fused.hip): the logits GEMM and the row
// statistics in one kernel, for bf16 hidden and weight with H a multiple of
// 64.  Workgroups cover 256 positions x a range of 256-row vocabulary tiles;
// part[n * nparts + 2 * range + half] holds each range's (max, sum) pair per
// position and vocabulary half, folded by a second kernel into run_m / run_s
// (the same state the chunked path leaves for launch_ce_finalize).
constexpr int kCeFusedMaxRanges = 64;
struct CeFusedArgs {
    const void* hidden;  // [N, H] bf16
    const void* weight;  // [V, H] bf16
    const int32_t* labels;
    float* tgt;
    float2* part;
    int64_t N, V, S;
    int H, ignore;
    int nb_pos, ntiles_v, tiles_per_range, ranges, nparts;
    int xbr, xbp;  // XCD rectangle: ranges x position blocks per XCD run (0: range-major)
    // backward (launch_ce_fused_grad): V above is the chunk's row count
    __bf16* g;              // [N, ldg] bf16 gradient of the chunk's logits
    int64_t ldg, v0, vall;  // row stride of g, chunk start, full vocabulary size
    const float* lse_in;
    const long long* count;
    const float* grad_loss;
    int reduction;
    // LoRA forward (launch_lora_fused_fwd): weight = W [out, in] (V = out,
    // H = in), hidden = x in bf16 [N, in]; y[n, o] = (x W^T)[n, o] +
    // scale * sum_k u[n, k] B(o, k) (+ bias[o]), B(o, k) = lb[o * lb_so + k * lb_sk]
    float* y;
    int64_t ldy, ldu, lb_so, lb_sk;
    const float* bias;
    const float* u;
    const float* lb;
    int rank;
    float scale;
};
bool ce_fused_supported(int64_t H, bool bf16);
CeFusedArgs ce_fused_plan(int64_t N, int64_t V, int64_t H);  // the launch geometry (nparts: pairs per position)
hipError_t launch_ce_fused_fwd(const CeArgs& a, const CeFusedArgs& plan, const void* hidden, const void* weight,
                               float2* part, hipStream_t st);
// The backward's logits recompute for vocabulary rows [v0, v0 + plan.V) with
// G = (exp(z - lse) - onehot) * coeff written in bf16 to g (row stride ldg, a
// multiple of 8) instead of the logits; plan = ce_fused_plan(N, chunk rows, H),
// weight_chunk = the chunk's first weight row.  Needs the scored count.
hipError_t launch_ce_fused_grad(const CeArgs& a, const CeFusedArgs& plan, const void* hidden, const void* weight_chunk,
                                int64_t v0, void* g, int64_t ldg, hipStream_t st);

// The same GEMM as the LoRA layer's forward (bf16 x and W [out, in], in a
// multiple of 64) with the rank-r update and the bias in its epilogue: one
// pass writes y.  plan = ce_fused_plan(N, out, in) with the LoRA fields set;
// rank <= kLoraFusedMaxRank.
constexpr int kLoraFusedMaxRank = 32;
hipError_t launch_lora_fused_fwd(const CeFusedArgs& plan, hipStream_t st);

}  // namespace mft
