// C ABI of the fused q/k prologue (declared in include/mft/prologue.h).
//
// Validation mirrors the reference operators' checks: apply_rope requires a
// 4-D [B, H, S, D] input (core/ops.cpp:2341-2354), ApplyRoPEBackward an even
// head dim (core/backward_functions.cpp:742-744).  The RoPE frequency table is
// computed here, on the host, with the reference's own float expression
// 1.0f / std::pow(theta, 2.0f * d / D) (core/ops.cpp:2368-2370), and passed
// to the kernels by value.
#include "mft/prologue.h"

#include <cmath>
#include <string>

#include "capi_util.h"
#include "prologue_kernels.h"

namespace {

using namespace mft::capi;

mft_status check(const mft_prologue_desc* d, const char* who, mft::PrologueArgs* a) {
    if (!d) return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": desc is NULL");
    if (d->B <= 0 || d->H <= 0 || d->S <= 0 || d->D <= 0)
        return fail(MFT_ERR_INVALID_ARG, "apply_rope expects 4D tensor: [batch, heads, seq_len, head_dim]");
    if (d->D % 2 != 0) return fail(MFT_ERR_INVALID_ARG, "ApplyRoPEBackward requires even head_dim");
    if (d->D > mft::PROLOGUE_MAX_D) return fail(MFT_ERR_UNSUPPORTED, std::string(who) + ": head_dim > 512");
    if (d->S > (int64_t(1) << 24)) return fail(MFT_ERR_UNSUPPORTED, std::string(who) + ": sequence length > 2^24");
    if (d->dtype != MFT_F32 && d->dtype != MFT_BF16)
        return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": dtype must be MFT_F32 or MFT_BF16");
    if (d->norm != MFT_NORM_NONE && d->norm != MFT_NORM_GEMMA && d->norm != MFT_NORM_AFFINE)
        return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": norm must be MFT_NORM_NONE, _GEMMA or _AFFINE");
    if (!std::isfinite(d->eps) || d->eps < 0.f)
        return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": eps must be finite and >= 0");
    if (!std::isfinite(d->theta) || d->theta < 0.f)
        return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": theta must be finite and >= 0 (0 = no RoPE)");
    const int64_t esz = d->dtype == MFT_BF16 ? 2 : 4;
    bool dense = true;
    mft_status r;
    if ((r = resolve_layout(d->x, d->H, d->S, d->D, esz, who, "x", &a->sx, &dense)) != MFT_OK) return r;
    if ((r = resolve_layout(d->y, d->H, d->S, d->D, esz, who, "y", &a->sy, &dense)) != MFT_OK) return r;
    if ((r = resolve_layout(d->dy, d->H, d->S, d->D, 4, who, "dy", &a->sdy, &dense)) != MFT_OK) return r;
    if ((r = resolve_layout(d->dx, d->H, d->S, d->D, 4, who, "dx", &a->sdx, &dense)) != MFT_OK) return r;
    a->B = d->B;
    a->H = d->H;
    a->S = d->S;
    a->rows = d->B * d->H * d->S;
    a->rows32 = a->rows < (int64_t(1) << 31);
    if (a->rows32) {
        a->fh = mft::FastDiv::make((uint32_t)d->H);
        a->fs = mft::FastDiv::make((uint32_t)d->S);
    }
    a->D = (int)d->D;
    a->norm = d->norm;
    a->eps = d->eps;
    a->rope = d->theta > 0.f;
    a->x = nullptr;
    a->w = nullptr;
    a->y = nullptr;
    a->dy = nullptr;
    a->dx = nullptr;
    a->dw_part = nullptr;
    const int64_t half = d->D / 2;
    for (int64_t i = 0; i < mft::PROLOGUE_MAX_D / 2; ++i) a->inv_freq[i] = 0.f;
    if (a->rope)
        for (int64_t i = 0; i < half; ++i)
            a->inv_freq[i] = 1.0f / std::pow(d->theta, 2.0f * i / d->D);
    return MFT_OK;
}

bool elem_aligned(const void* p, int64_t esz) { return (reinterpret_cast<uintptr_t>(p) % esz) == 0; }

// Bytes of one tensor's dw partials, and of a batch's (each 256-byte aligned).
size_t part_bytes(const mft_prologue_desc* d, const mft::PrologueArgs& a) {
    return d->norm == MFT_NORM_NONE ? 0 : (size_t)(mft::prologue_bwd_blocks(a.rows, a.D) * a.D) * sizeof(float);
}
size_t up256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

mft_status check_n(int n, const mft_prologue_desc* descs, const char* who, mft::PrologueArgs* a) {
    if (n < 1 || n > mft::kPrologueMaxBatch)
        return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": n must be 1 or 2");
    if (!descs) return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": descs is NULL");
    for (int i = 0; i < n; ++i) {
        const mft_status r = check(&descs[i], who, &a[i]);
        if (r != MFT_OK) return r;
        if (descs[i].dtype != descs[0].dtype)
            return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": every tensor of a batch has one dtype");
    }
    return MFT_OK;
}

mft_status fwd_n(int n, const mft_prologue_desc* descs, const void* const* x, const float* const* w, void* const* y,
                 hipStream_t stream, const char* who) {
    mft::PrologueArgs a[mft::kPrologueMaxBatch];
    mft_status r = check_n(n, descs, who, a);
    if (r != MFT_OK) return r;
    if (!x || !w || !y) return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": x, w and y must be non-NULL arrays");
    for (int i = 0; i < n; ++i) {
        if (!x[i] || !y[i]) return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": x and y must be non-NULL");
        if (descs[i].norm != MFT_NORM_NONE && !w[i])
            return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": a norm needs its weight w");
        const int64_t esz = descs[i].dtype == MFT_BF16 ? 2 : 4;
        if (!elem_aligned(x[i], esz) || !elem_aligned(y[i], esz) || (w[i] && !elem_aligned(w[i], 4)))
            return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": pointers must be element-aligned");
        a[i].x = x[i];
        a[i].w = w[i];
        a[i].y = y[i];
    }
    return hip_status(mft::launch_prologue_fwd(a, n, descs[0].dtype == MFT_BF16, stream),
                      (std::string(who) + " launch").c_str());
}

mft_status bwd_n(int n, const mft_prologue_desc* descs, const void* const* x, const float* const* w,
                 const float* const* dy, float* const* dx, float* const* dw, void* workspace, hipStream_t stream,
                 const char* who) {
    mft::PrologueArgs a[mft::kPrologueMaxBatch];
    mft_status r = check_n(n, descs, who, a);
    if (r != MFT_OK) return r;
    if (!x || !w || !dy || !dx || !dw)
        return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": x, w, dy, dx and dw must be non-NULL arrays");
    size_t off = 0;
    for (int i = 0; i < n; ++i) {
        if (!dy[i] || !dx[i]) return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": dy and dx must be non-NULL");
        const bool norm = descs[i].norm != MFT_NORM_NONE;
        if (norm && (!x[i] || !w[i]))
            return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": a norm needs x and its weight w");
        if (norm && dw[i] && !workspace)
            return fail(MFT_ERR_INVALID_ARG,
                        std::string(who) + ": dw needs the workspace (mft_prologue_workspace_size)");
        if (static_cast<const void*>(dx[i]) == x[i] || static_cast<const void*>(dx[i]) == static_cast<const void*>(dy[i]))
            return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": dx may not alias x or dy");
        const int64_t esz = descs[i].dtype == MFT_BF16 ? 2 : 4;
        if ((x[i] && !elem_aligned(x[i], esz)) || !elem_aligned(dy[i], 4) || !elem_aligned(dx[i], 4) ||
            (w[i] && !elem_aligned(w[i], 4)) || (dw[i] && !elem_aligned(dw[i], 4)) ||
            (workspace && !elem_aligned(workspace, 4)))
            return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": pointers must be element-aligned");
        a[i].x = x[i];
        a[i].w = w[i];
        a[i].dy = dy[i];
        a[i].dx = dx[i];
        a[i].dw_part = norm && dw[i] ? reinterpret_cast<float*>(static_cast<char*>(workspace) + off) : nullptr;
        off += up256(part_bytes(&descs[i], a[i]));
    }
    return hip_status(mft::launch_prologue_bwd(a, n, descs[0].dtype == MFT_BF16, dw, stream),
                      (std::string(who) + " launch").c_str());
}

}  // namespace

extern "C" {

mft_status mft_prologue_fwd(const mft_prologue_desc* desc, const void* x, const float* w, void* y,
                            hipStream_t stream) {
    return fwd_n(1, desc, &x, &w, &y, stream, "mft_prologue_fwd");
}

mft_status mft_prologue_workspace_size(const mft_prologue_desc* desc, size_t* bytes) {
    mft::PrologueArgs a;
    mft_status r = check(desc, "mft_prologue_workspace_size", &a);
    if (r != MFT_OK) return r;
    if (!bytes) return fail(MFT_ERR_INVALID_ARG, "mft_prologue_workspace_size: bytes is NULL");
    *bytes = part_bytes(desc, a);
    return MFT_OK;
}

mft_status mft_prologue_bwd(const mft_prologue_desc* desc, const void* x, const float* w, const float* dy,
                            float* dx, float* dw, void* workspace, hipStream_t stream) {
    return bwd_n(1, desc, &x, &w, &dy, &dx, &dw, workspace, stream, "mft_prologue_bwd");
}

mft_status mft_prologue_fwd_n(int n, const mft_prologue_desc* descs, const void* const* x, const float* const* w,
                              void* const* y, hipStream_t stream) {
    return fwd_n(n, descs, x, w, y, stream, "mft_prologue_fwd_n");
}

mft_status mft_prologue_workspace_size_n(int n, const mft_prologue_desc* descs, size_t* bytes) {
    mft::PrologueArgs a[mft::kPrologueMaxBatch];
    mft_status r = check_n(n, descs, "mft_prologue_workspace_size_n", a);
    if (r != MFT_OK) return r;
    if (!bytes) return fail(MFT_ERR_INVALID_ARG, "mft_prologue_workspace_size_n: bytes is NULL");
    size_t total = 0;
    for (int i = 0; i < n; ++i) total += up256(part_bytes(&descs[i], a[i]));
    *bytes = total;
    return MFT_OK;
}

mft_status mft_prologue_bwd_n(int n, const mft_prologue_desc* descs, const void* const* x, const float* const* w,
                              const float* const* dy, float* const* dx, float* const* dw, void* workspace,
                              hipStream_t stream) {
    return bwd_n(n, descs, x, w, dy, dx, dw, workspace, stream, "mft_prologue_bwd_n");
}

}  // extern "C"
