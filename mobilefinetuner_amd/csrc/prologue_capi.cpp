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

}  // namespace

extern "C" {

mft_status mft_prologue_fwd(const mft_prologue_desc* desc, const void* x, const float* w, void* y,
                            hipStream_t stream) {
    mft::PrologueArgs a;
    mft_status r = check(desc, "mft_prologue_fwd", &a);
    if (r != MFT_OK) return r;
    if (!x || !y) return fail(MFT_ERR_INVALID_ARG, "mft_prologue_fwd: x and y must be non-NULL");
    if (desc->norm != MFT_NORM_NONE && !w)
        return fail(MFT_ERR_INVALID_ARG, "mft_prologue_fwd: a norm needs its weight w");
    const int64_t esz = desc->dtype == MFT_BF16 ? 2 : 4;
    if (!elem_aligned(x, esz) || !elem_aligned(y, esz) || (w && !elem_aligned(w, 4)))
        return fail(MFT_ERR_INVALID_ARG, "mft_prologue_fwd: pointers must be element-aligned");
    a.x = x;
    a.w = w;
    a.y = y;
    return hip_status(mft::launch_prologue_fwd(a, desc->dtype == MFT_BF16, stream), "mft_prologue_fwd launch");
}

mft_status mft_prologue_workspace_size(const mft_prologue_desc* desc, size_t* bytes) {
    mft::PrologueArgs a;
    mft_status r = check(desc, "mft_prologue_workspace_size", &a);
    if (r != MFT_OK) return r;
    if (!bytes) return fail(MFT_ERR_INVALID_ARG, "mft_prologue_workspace_size: bytes is NULL");
    *bytes = desc->norm == MFT_NORM_NONE ? 0 : (size_t)(mft::prologue_bwd_blocks(a.rows, a.D) * a.D) * sizeof(float);
    return MFT_OK;
}

mft_status mft_prologue_bwd(const mft_prologue_desc* desc, const void* x, const float* w, const float* dy,
                            float* dx, float* dw, void* workspace, hipStream_t stream) {
    mft::PrologueArgs a;
    mft_status r = check(desc, "mft_prologue_bwd", &a);
    if (r != MFT_OK) return r;
    if (!dy || !dx) return fail(MFT_ERR_INVALID_ARG, "mft_prologue_bwd: dy and dx must be non-NULL");
    const bool norm = desc->norm != MFT_NORM_NONE;
    if (norm && (!x || !w)) return fail(MFT_ERR_INVALID_ARG, "mft_prologue_bwd: a norm needs x and its weight w");
    if (norm && dw && !workspace)
        return fail(MFT_ERR_INVALID_ARG, "mft_prologue_bwd: dw needs the workspace (mft_prologue_workspace_size)");
    if (static_cast<const void*>(dx) == x || static_cast<const void*>(dx) == static_cast<const void*>(dy))
        return fail(MFT_ERR_INVALID_ARG, "mft_prologue_bwd: dx may not alias x or dy");
    const int64_t esz = desc->dtype == MFT_BF16 ? 2 : 4;
    if ((x && !elem_aligned(x, esz)) || !elem_aligned(dy, 4) || !elem_aligned(dx, 4) || (w && !elem_aligned(w, 4)) ||
        (dw && !elem_aligned(dw, 4)) || (workspace && !elem_aligned(workspace, 4)))
        return fail(MFT_ERR_INVALID_ARG, "mft_prologue_bwd: pointers must be element-aligned");
    a.x = x;
    a.w = w;
    a.dy = dy;
    a.dx = dx;
    a.dw_part = norm && dw ? static_cast<float*>(workspace) : nullptr;
    return hip_status(mft::launch_prologue_bwd(a, desc->dtype == MFT_BF16, dw, stream), "mft_prologue_bwd launch");
}

}  // extern "C"
