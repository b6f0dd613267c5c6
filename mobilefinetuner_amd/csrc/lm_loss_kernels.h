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

}  // namespace mft
