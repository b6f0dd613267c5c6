// C ABI of the language-model cross-entropy (declared in include/mft/lm_loss.h).
//
// Validation mirrors the reference's checks (core/lm_loss.cpp:273-286 for the
// dense variant, :389-414 for the selected-token / streaming variant).  The
// streaming variant cuts the vocabulary into chunks of `chunk` rows of the
// LM-head weight; per chunk, with rocBLAS column-major GEMMs over the
// row-major tensors:
//   forward   Z = hidden . W_c^T          (fp32 [N, chunk], workspace)
//             row statistics of Z merged into the running (max, sum)
//   backward  Z recomputed, G = (exp(Z - lse) - onehot) * coeff  (input dtype)
//             grad_hidden += G . W_c,  grad_weight[c] = G^T . hidden
// so the [N, V] logits never exist at once.  With bf16 operands and H a
// multiple of 64 the fused kernels of lm_loss_fused.hip replace the logits
// GEMM and the passes over it: the forward computes the row statistics in
// one pass with no logits at all, and the backward writes each chunk's G
// straight from the recomputed logits (no fp32 chunk).
#include "mft/lm_loss.h"

#include <string>

#include "blas_util.h"
#include "capi_util.h"
#include "lm_loss_kernels.h"

namespace {

using namespace mft::capi;

constexpr int64_t kDefaultChunk = 16384;
constexpr size_t kBlasWorkspace = size_t(64) << 20;

size_t up(size_t x) { return (x + 255) & ~size_t(255); }

struct Layout {
    size_t m, s, tgt, nll, count, z, g, blas, part, total;
};

int64_t chunk_of(const mft_lm_loss_desc* d) {
    const int64_t c = d->chunk > 0 ? d->chunk : kDefaultChunk;
    return c < d->V ? c : d->V;
}

Layout layout(const mft_lm_loss_desc* d, bool streaming) {
    const size_t N = (size_t)(d->B * d->S);
    Layout l{};
    size_t o = 0;
    l.m = o, o += up(N * 4);
    l.s = o, o += up(N * 8);
    l.tgt = o, o += up(N * 4);
    l.nll = o, o += up(N * 8);
    l.count = o, o += up(8);
    if (streaming) {
        const size_t c = (size_t)chunk_of(d);
        const size_t esz = d->dtype == MFT_BF16 ? 2 : 4;
        // the fused kernels need no fp32 logits chunk; their G rows are
        // padded to a multiple of 8 elements (8-byte stores)
        const bool fused = mft::ce_fused_supported(d->H, d->dtype == MFT_BF16);
        l.z = o, o += fused ? 0 : up(N * c * 4);
        l.g = o, o += up(N * (fused ? (c + 7) / 8 * 8 : c) * esz);
        l.blas = o, o += kBlasWorkspace;
        // fused forward: (max, sum) pairs per position and vocabulary part
        l.part = o, o += up(N * 2 * mft::kCeFusedMaxRanges * sizeof(float2));
    }
    l.total = o;
    return l;
}

mft_status check(const mft_lm_loss_desc* d, const char* who, bool streaming) {
    if (!d) return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": desc is NULL");
    if (d->B <= 0 || d->S <= 0 || d->V <= 0)
        return fail(MFT_ERR_INVALID_ARG, "lm_cross_entropy: logits must be [B,S,V] and labels [B,S] (positive sizes)");
    if (d->dtype != MFT_F32 && d->dtype != MFT_BF16)
        return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": dtype must be MFT_F32 or MFT_BF16");
    if (d->reduction != MFT_REDUCE_MEAN && d->reduction != MFT_REDUCE_SUM && d->reduction != MFT_REDUCE_NONE)
        return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": reduction must be MEAN, SUM or NONE");
    if (d->chunk < 0) return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": chunk must be >= 0");
    if (d->B * d->S > (int64_t(1) << 31) - 1 || d->V > (int64_t(1) << 31) - 1)
        return fail(MFT_ERR_UNSUPPORTED, std::string(who) + ": B*S and V must be below 2^31");
    if (streaming) {
        if (d->H <= 0) return fail(MFT_ERR_INVALID_ARG, "selected_token_lm_cross_entropy: hidden must be [B,S,H]");
        if (d->H > (int64_t(1) << 31) - 1) return fail(MFT_ERR_UNSUPPORTED, std::string(who) + ": H >= 2^31");
        if (d->reduction == MFT_REDUCE_NONE)
            return fail(MFT_ERR_INVALID_ARG,
                        "selected_token_lm_cross_entropy: only mean and sum reductions are supported");
    }
    return MFT_OK;
}

mft::CeArgs args(const mft_lm_loss_desc* d, const Layout& l, void* ws, const int32_t* labels) {
    mft::CeArgs a{};
    char* w = static_cast<char*>(ws);
    a.B = d->B;
    a.S = d->S;
    a.V = d->V;
    a.N = d->B * d->S;
    a.ignore = d->ignore_index;
    a.reduction = d->reduction;
    a.labels = labels;
    a.run_m = reinterpret_cast<float*>(w + l.m);
    a.run_s = reinterpret_cast<double*>(w + l.s);
    a.tgt = reinterpret_cast<float*>(w + l.tgt);
    a.nll = reinterpret_cast<double*>(w + l.nll);
    a.count = reinterpret_cast<long long*>(w + l.count);
    return a;
}

// Z[N, nc] (row-major, fp32) = hidden[N, H] . W[v0 : v0 + nc, :]^T
mft_status logits_chunk(rocblas_handle h, const mft_lm_loss_desc* d, const void* hidden, const void* weight,
                        int64_t v0, int64_t nc, float* Z) {
    const bool bf = d->dtype == MFT_BF16;
    const char* W = static_cast<const char*>(weight) + v0 * d->H * (bf ? 2 : 4);
    return mft::blas::gemm_rm("mft_lm_ce", h, d->B * d->S, nc, d->H, 1.f, hidden, d->H, false, W, d->H, true, 0.f, Z,
                              nc, bf);
}

}  // namespace

extern "C" {

mft_status mft_lm_ce_workspace_size(const mft_lm_loss_desc* desc, size_t* fwd_bytes, size_t* bwd_bytes) {
    const bool streaming = desc && desc->H > 0;
    mft_status r = check(desc, "mft_lm_ce_workspace_size", streaming);
    if (r != MFT_OK) return r;
    const size_t t = layout(desc, streaming).total;
    if (fwd_bytes) *fwd_bytes = t;
    if (bwd_bytes) *bwd_bytes = t;
    return MFT_OK;
}

mft_status mft_lm_ce_fwd(const mft_lm_loss_desc* desc, const void* logits, const int32_t* labels, float* loss,
                         float* lse, int32_t* status, void* workspace, hipStream_t stream) {
    mft_status r = check(desc, "mft_lm_ce_fwd", false);
    if (r != MFT_OK) return r;
    if (!logits || !labels || !loss || !workspace)
        return fail(MFT_ERR_INVALID_ARG, "mft_lm_ce_fwd: logits, labels, loss and workspace must be non-NULL");
    const Layout l = layout(desc, false);
    mft::CeArgs a = args(desc, l, workspace, labels);
    a.lse = lse;
    a.loss = loss;
    a.status = status;
    hipError_t e = mft::launch_ce_stats(a, logits, desc->dtype == MFT_BF16, desc->V, desc->V, 0, true, stream);
    if (e == hipSuccess) e = mft::launch_ce_finalize(a, stream);
    return hip_status(e, "mft_lm_ce_fwd launch");
}

mft_status mft_lm_ce_bwd(const mft_lm_loss_desc* desc, const void* logits, const int32_t* labels, const float* lse,
                         const float* grad_loss, float* grad_logits, void* workspace, hipStream_t stream) {
    mft_status r = check(desc, "mft_lm_ce_bwd", false);
    if (r != MFT_OK) return r;
    if (!logits || !labels || !lse || !grad_logits || !workspace)
        return fail(MFT_ERR_INVALID_ARG,
                    "mft_lm_ce_bwd: logits, labels, lse, grad_logits and workspace must be non-NULL");
    const Layout l = layout(desc, false);
    mft::CeArgs a = args(desc, l, workspace, labels);
    a.lse_in = lse;
    a.grad_loss = grad_loss;
    hipError_t e = mft::launch_ce_count(a, stream);
    if (e == hipSuccess)
        e = mft::launch_ce_grad(a, logits, desc->dtype == MFT_BF16, desc->V, desc->V, 0, grad_logits, false, desc->V,
                                stream);
    return hip_status(e, "mft_lm_ce_bwd launch");
}

mft_status mft_lm_ce_streaming_fwd(const mft_lm_loss_desc* desc, const void* hidden, const void* weight,
                                   const int32_t* labels, float* loss, float* lse, int32_t* status, void* workspace,
                                   hipStream_t stream) {
    mft_status r = check(desc, "mft_lm_ce_streaming_fwd", true);
    if (r != MFT_OK) return r;
    if (!hidden || !weight || !labels || !loss || !workspace)
        return fail(MFT_ERR_INVALID_ARG,
                    "mft_lm_ce_streaming_fwd: hidden, weight, labels, loss and workspace must be non-NULL");
    const Layout l = layout(desc, true);
    mft::CeArgs a = args(desc, l, workspace, labels);
    a.lse = lse;
    a.loss = loss;
    a.status = status;
    char* w = static_cast<char*>(workspace);
    if (mft::ce_fused_supported(desc->H, desc->dtype == MFT_BF16)) {
        const mft::CeFusedArgs plan = mft::ce_fused_plan(a.N, desc->V, desc->H);
        hipError_t e = mft::launch_ce_fused_fwd(a, plan, hidden, weight, reinterpret_cast<float2*>(w + l.part), stream);
        if (e == hipSuccess) e = mft::launch_ce_finalize(a, stream);
        return hip_status(e, "mft_lm_ce_streaming_fwd launch");
    }
    float* Z = reinterpret_cast<float*>(w + l.z);
    const int64_t chunk = chunk_of(desc);
    auto lock = mft::blas::lock();
    rocblas_handle h;
    if ((r = mft::blas::bind("mft_lm_ce_streaming_fwd", stream, w + l.blas, kBlasWorkspace, &h)) != MFT_OK) return r;
    for (int64_t v0 = 0; v0 < desc->V; v0 += chunk) {
        const int64_t nc = desc->V - v0 < chunk ? desc->V - v0 : chunk;
        if ((r = logits_chunk(h, desc, hidden, weight, v0, nc, Z)) != MFT_OK) return r;
        const hipError_t e = mft::launch_ce_stats(a, Z, false, nc, nc, v0, v0 == 0, stream);
        if (e != hipSuccess) return hip_status(e, "mft_lm_ce_streaming_fwd launch");
    }
    return hip_status(mft::launch_ce_finalize(a, stream), "mft_lm_ce_streaming_fwd launch");
}

mft_status mft_lm_ce_streaming_bwd(const mft_lm_loss_desc* desc, const void* hidden, const void* weight,
                                   const int32_t* labels, const float* lse, const float* grad_loss, float* grad_hidden,
                                   float* grad_weight, void* workspace, hipStream_t stream) {
    mft_status r = check(desc, "mft_lm_ce_streaming_bwd", true);
    if (r != MFT_OK) return r;
    if (!hidden || !weight || !labels || !lse || !workspace)
        return fail(MFT_ERR_INVALID_ARG,
                    "mft_lm_ce_streaming_bwd: hidden, weight, labels, lse and workspace must be non-NULL");
    if (!grad_hidden && !grad_weight) return MFT_OK;
    const Layout l = layout(desc, true);
    mft::CeArgs a = args(desc, l, workspace, labels);
    a.lse_in = lse;
    a.grad_loss = grad_loss;
    char* w = static_cast<char*>(workspace);
    float* Z = reinterpret_cast<float*>(w + l.z);
    void* G = w + l.g;
    const bool bf = desc->dtype == MFT_BF16;
    const int64_t chunk = chunk_of(desc), N = desc->B * desc->S, H = desc->H;
    hipError_t e = mft::launch_ce_count(a, stream);
    if (e != hipSuccess) return hip_status(e, "mft_lm_ce_streaming_bwd launch");
    auto lock = mft::blas::lock();
    rocblas_handle h;
    if ((r = mft::blas::bind("mft_lm_ce_streaming_bwd", stream, w + l.blas, kBlasWorkspace, &h)) != MFT_OK) return r;
    const bool fused = mft::ce_fused_supported(H, bf);
    const int64_t ldg = fused ? (chunk + 7) / 8 * 8 : chunk;
    mft::CeFusedArgs plan{};
    for (int64_t v0 = 0; v0 < desc->V; v0 += chunk) {
        const int64_t nc = desc->V - v0 < chunk ? desc->V - v0 : chunk;
        const char* Wc = static_cast<const char*>(weight) + v0 * H * (bf ? 2 : 4);
        if (fused) {  // G straight from the recomputed logits, no fp32 chunk
            if (v0 == 0 || nc != chunk) plan = mft::ce_fused_plan(N, nc, H);
            e = mft::launch_ce_fused_grad(a, plan, hidden, Wc, v0, G, ldg, stream);
        } else {
            if ((r = logits_chunk(h, desc, hidden, weight, v0, nc, Z)) != MFT_OK) return r;
            e = mft::launch_ce_grad(a, Z, false, nc, nc, v0, G, bf, ldg, stream);
        }
        if (e != hipSuccess) return hip_status(e, "mft_lm_ce_streaming_bwd launch");
        // grad_hidden[N, H] (+)= G[N, nc] . W_c[nc, H]
        if (grad_hidden && (r = mft::blas::gemm_rm("mft_lm_ce_streaming_bwd", h, N, H, nc, 1.f, G, ldg, false, Wc, H,
                                                   false, v0 > 0 ? 1.f : 0.f, grad_hidden, H, bf)) != MFT_OK)
            return r;
        // grad_weight[v0 : v0 + nc, :] = G^T . hidden
        if (grad_weight && (r = mft::blas::gemm_rm("mft_lm_ce_streaming_bwd", h, nc, H, N, 1.f, G, ldg, true, hidden,
                                                   H, false, 0.f, grad_weight + v0 * H, H, bf)) != MFT_OK)
            return r;
    }
    return MFT_OK;
}

}  // extern "C"
