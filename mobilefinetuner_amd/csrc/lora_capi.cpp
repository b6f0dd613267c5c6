// C ABI of the LoRA linear layer (declared in include/mft/lora.h).
//
// The layer is GEMMs plus element-wise staging.  Row-major throughout, R =
// sum of the slices' ranks, s_i = scale_i:
//   forward   y  = x . W (+ bias)                 rocBLAS; bf16 W: x staged
//                                                  to bf16 by the first rowdot
//                                                  (bf16 W [out, in] with one
//                                                  full-width slice and a large
//                                                  output: one fused kernel for
//                                                  this line and the s_i u_i B_i
//                                                  line, lora_fused_fwd_ok)
//             u_i = x . A_i                        lora_rowdot, into u[:, ro_i ..]
//             y[:, col0_i ..] += s_i u_i . B_i     rocBLAS fp32, beta = 1
//   backward  g_i = s_i dy[:, col0_i ..] . B_i^T   lora_rowdot (workspace [N, R])
//             grad_B_i = s_i u_i^T . dy[:, col0_i ..]   lora_coldot
//             grad_A_i = x^T . g_i                      lora_coldot
//             dx = dy . W^T + sum_i g_i . A_i^T     rocBLAS; bf16 W: dy staged to bf16
//                                                  by a full-width slice's rowdot
// which is the reference's autograd graph of matmul / mul / add
// (nn/lora_linear.cpp:384-434 with MatmulBackward,
// core/backward_functions.cpp:94-160).  The rank-r products with a long inner
// dimension (u, g, grad_A, grad_B) are this library's own HBM-bound kernels:
// rocBLAS runs those shapes on a few workgroups.  Validation messages follow
// the reference's (nn/lora_linear.cpp:52-88, 118-128, 397-404).
#include "mft/lora.h"

#include <algorithm>
#include <cmath>
#include <string>

#include "attn_kernels.h"
#include "blas_util.h"
#include "capi_util.h"
#include "lm_loss_kernels.h"
#include "lora_kernels.h"

namespace {

using namespace mft::capi;

constexpr size_t kBlasWorkspace = size_t(32) << 20;
constexpr int64_t kMaxInt = (int64_t(1) << 31) - 1;

size_t up(size_t x) { return (x + 255) & ~size_t(255); }

int64_t total_rank(const mft_lora_desc* d) {
    int64_t r = 0;
    for (int i = 0; i < d->n_slices; ++i) r += d->slices[i].rank;
    return r;
}

mft_status check(const mft_lora_desc* d, const char* who) {
    if (!d) return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": desc is NULL");
    if (d->N <= 0 || d->in_dim <= 0 || d->out_dim <= 0)
        return fail(MFT_ERR_INVALID_ARG, "LoRALinear: x must be [N, in] and W [in, out] with positive sizes");
    if (d->w_dtype != MFT_F32 && d->w_dtype != MFT_BF16)
        return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": w_dtype must be MFT_F32 or MFT_BF16");
    if (d->n_slices < 0 || (d->n_slices > 0 && !d->slices))
        return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": n_slices > 0 needs a slices array");
    if (d->N > kMaxInt || d->in_dim > kMaxInt || d->out_dim > kMaxInt)
        return fail(MFT_ERR_UNSUPPORTED, std::string(who) + ": N, in and out must be below 2^31");
    for (int i = 0; i < d->n_slices; ++i) {
        const mft_lora_slice& s = d->slices[i];
        if (!s.A || !s.B) return fail(MFT_ERR_INVALID_ARG, "LoRALinear::attach_lora: A and B must not be null");
        if (s.rank <= 0) return fail(MFT_ERR_INVALID_ARG, "LoRALinear: LoRA rank must be positive");
        if (s.cols <= 0) return fail(MFT_ERR_INVALID_ARG, "LoRALinear: LoRA slice cols must be positive");
        if (s.col0 < 0 || s.col0 + s.cols > d->out_dim)
            return fail(MFT_ERR_INVALID_ARG, "LoRALinear: LoRA slice range exceeds base weight width");
        if (s.rank > kMaxInt) return fail(MFT_ERR_UNSUPPORTED, std::string(who) + ": rank must be below 2^31");
    }
    if (total_rank(d) > kMaxInt) return fail(MFT_ERR_UNSUPPORTED, std::string(who) + ": total rank too large");
    return MFT_OK;
}

// A slice whose delta is part of the autograd graph (see mft/lora.h).
bool has_grad(const mft_lora_desc* d, const mft_lora_slice& s) {
    return d->grads_for_column_slices || (s.col0 == 0 && s.cols == d->out_dim);
}

struct FwdLayout {
    size_t xb, u, pt, blas, total;
};
struct BwdLayout {
    size_t dyb, g, part, pt, blas, total;
};

// k-contiguous copy of a rank-r operand (see rowdot): the largest slice's.
size_t pack_bytes(const mft_lora_desc* d) {
    size_t m = 0;
    for (int i = 0; i < d->n_slices; ++i) {
        const mft_lora_slice& s = d->slices[i];
        const size_t k = (size_t)(s.cols > d->in_dim ? s.cols : d->in_dim);
        m = std::max(m, k * (size_t)s.rank * 4);
    }
    return up(m);
}

FwdLayout fwd_layout(const mft_lora_desc* d) {
    FwdLayout l{};
    size_t o = 0;
    l.xb = o, o += d->w_dtype == MFT_BF16 ? up((size_t)d->N * d->in_dim * 2) : 0;
    l.u = o, o += up((size_t)d->N * total_rank(d) * 4);
    l.pt = o, o += pack_bytes(d);
    l.blas = o, o += kBlasWorkspace;
    l.total = o;
    return l;
}

BwdLayout bwd_layout(const mft_lora_desc* d) {
    BwdLayout l{};
    size_t o = 0;
    l.dyb = o, o += d->w_dtype == MFT_BF16 ? up((size_t)d->N * d->out_dim * 2) : 0;
    l.g = o, o += up((size_t)d->N * total_rank(d) * 4);
    int64_t part = 0;
    for (int i = 0; i < d->n_slices; ++i) {
        const mft_lora_slice& s = d->slices[i];
        // grad_B's reduction runs over cols columns, grad_A's over in (the chunk
        // height depends on the width, so take both)
        for (const int64_t k : {s.cols, d->in_dim}) {
            const int64_t p = mft::lora_coldot_partial_floats(d->N, k, (int)s.rank);
            part = p > part ? p : part;
        }
    }
    l.part = o, o += up((size_t)part * 4);
    l.pt = o, o += pack_bytes(d);
    l.blas = o, o += kBlasWorkspace;
    l.total = o;
    return l;
}

// u_i = x . A_eff, or g_i = scale * dy_slice . B_eff^T: rank-r products over a
// long inner dimension (lora_rowdot).
// A P that is not k-contiguous (pk != 1) is first copied k-major into
// `pack` (K x r floats of workspace): rowdot's lanes stride over k, and a
// j-contiguous P would put every lane of a load on its own cache line.
// With mb, the same pass also writes the bf16 copy of M[:, :K] (row stride
// K) that the MFMA GEMM reads, so M is read from HBM once.
mft_status rowdot(const float* M, int64_t ldm, int64_t rows, int64_t K, const float* P, int64_t pk, int64_t pj,
                  float* out, int64_t ldo, int64_t r, float alpha, float* pack, hipStream_t stream, const char* who,
                  uint16_t* mb = nullptr) {
    if (pk != 1) {
        const hipError_t e = mft::launch_lora_pack_kmajor(P, pk, pj, K, (int)r, pack, stream);
        if (e != hipSuccess) return hip_status(e, who);
        P = pack, pk = 1, pj = K;
    }
    mft::LoraRowDot a{M, ldm, rows, K, P, pk, pj, out, ldo, (int)r, alpha, mb, K};
    return hip_status(mft::launch_lora_rowdot(a, stream), who);
}

// out(k, j) = alpha * M^T V over the N rows (lora_coldot), for grad_A / grad_B.
mft_status coldot(const float* M, int64_t ldm, int64_t rows, int64_t K, const float* V, int64_t ldv, int64_t r,
                  float alpha, float* partial, float* out, int64_t ok, int64_t oj, hipStream_t stream,
                  const char* who) {
    mft::LoraColDot a{M, ldm, rows, K, V, ldv, (int)r, alpha, partial, out, ok, oj};
    return hip_status(mft::launch_lora_coldot(a, stream), who);
}

// op(W) as the right operand of x . W ([in, out]) or of dy . W^T ([out, in]).
struct WOperand {
    int64_t ld;
    bool t;
};
WOperand w_for_forward(const mft_lora_desc* d) {
    return d->w_transposed ? WOperand{d->in_dim, true} : WOperand{d->out_dim, false};
}
WOperand w_for_backward(const mft_lora_desc* d) {
    return d->w_transposed ? WOperand{d->in_dim, false} : WOperand{d->out_dim, true};
}

// The forward as one fused kernel (launch_lora_fused_fwd: the bf16 GEMM with
// the rank-r update and the bias in its epilogue) when W is bf16 [out, in]
// with in a multiple of 64, there is at most one slice and it spans every
// column with rank <= kLoraFusedMaxRank, and the 256 x 256 output tiles fill
// the GPU (smaller outputs stay on the library GEMM, which splits K).
bool lora_fused_fwd_ok(const mft_lora_desc* d, mft::CeFusedArgs* plan) {
    if (d->w_dtype != MFT_BF16 || !d->w_transposed || !mft::ce_fused_supported(d->in_dim, true)) return false;
    if (d->n_slices > 1) return false;
    if (d->n_slices == 1) {
        const mft_lora_slice& s = d->slices[0];
        if (s.col0 != 0 || s.cols != d->out_dim || s.rank > mft::kLoraFusedMaxRank) return false;
    }
    *plan = mft::ce_fused_plan(d->N, d->out_dim, d->in_dim);
    return (int64_t)plan->nb_pos * plan->ntiles_v >= mft::device_cus();
}

}  // namespace

extern "C" {

mft_status mft_lora_workspace_size(const mft_lora_desc* desc, size_t* fwd_bytes, size_t* bwd_bytes) {
    mft_status r = check(desc, "mft_lora_workspace_size");
    if (r != MFT_OK) return r;
    if (fwd_bytes) *fwd_bytes = fwd_layout(desc).total;
    if (bwd_bytes) *bwd_bytes = bwd_layout(desc).total;
    return MFT_OK;
}

mft_status mft_lora_fwd(const mft_lora_desc* desc, const float* x, const void* W, const float* bias, float* y,
                        float* u, void* workspace, hipStream_t stream) {
    static const char* who = "mft_lora_fwd";
    mft_status r = check(desc, who);
    if (r != MFT_OK) return r;
    if (!x || !W || !y || !workspace)
        return fail(MFT_ERR_INVALID_ARG, "mft_lora_fwd: x, W, y and workspace must be non-NULL");
    const FwdLayout l = fwd_layout(desc);
    char* ws = static_cast<char*>(workspace);
    const int64_t N = desc->N, in = desc->in_dim, out = desc->out_dim, R = total_rank(desc);
    const bool bf = desc->w_dtype == MFT_BF16;
    if (!u) u = reinterpret_cast<float*>(ws + l.u);

    mft::CeFusedArgs plan{};
    const bool fused = lora_fused_fwd_ok(desc, &plan);
    hipError_t e = hipSuccess;
    if (bias && !fused) e = mft::launch_lora_fill_bias(y, bias, N, out, stream);
    // bf16 W: the GEMM reads x rounded to bf16, written by the first slice's
    // rowdot (one read of x) or, without slices, by lora_round_bf16.
    uint16_t* xb = bf ? reinterpret_cast<uint16_t*>(ws + l.xb) : nullptr;
    if (e == hipSuccess && bf && desc->n_slices == 0) e = mft::launch_lora_round_bf16(x, xb, N * in, stream);
    if (e != hipSuccess) return hip_status(e, "mft_lora_fwd launch");
    int64_t ro = 0;
    for (int i = 0; i < desc->n_slices; ++i) {
        const mft_lora_slice& s = desc->slices[i];
        // u_i[N, r] = x . A_eff, A_eff(k, j) = A[k, j] or A[j, k]
        if ((r = rowdot(x, in, N, in, s.A, s.a_transposed ? 1 : s.rank, s.a_transposed ? in : 1, u + ro, R, s.rank,
                        1.f, reinterpret_cast<float*>(ws + l.pt), stream, "mft_lora_fwd launch",
                        i == 0 ? xb : nullptr)) != MFT_OK)
            return r;
        ro += s.rank;
    }

    if (fused) {
        plan.hidden = xb;
        plan.weight = W;
        plan.S = 1;
        plan.y = y;
        plan.ldy = out;
        plan.bias = bias;
        plan.u = u;
        plan.ldu = R;
        if (desc->n_slices == 1) {
            const mft_lora_slice& s = desc->slices[0];
            plan.lb = s.B;  // B(o, k): [rank, cols] or, transposed, [cols, rank]
            plan.lb_so = s.b_transposed ? s.rank : 1;
            plan.lb_sk = s.b_transposed ? 1 : s.cols;
            plan.rank = (int)s.rank;
            plan.scale = s.scale;
        }
        return hip_status(mft::launch_lora_fused_fwd(plan, stream), "mft_lora_fwd launch");
    }

    auto lock = mft::blas::lock();
    rocblas_handle h;
    if ((r = mft::blas::bind(who, stream, ws + l.blas, kBlasWorkspace, &h)) != MFT_OK) return r;
    const WOperand wo = w_for_forward(desc);
    if ((r = mft::blas::gemm_rm(who, h, N, out, in, 1.f, bf ? static_cast<const void*>(xb) : x, in, false, W, wo.ld,
                                wo.t, bias ? 1.f : 0.f, y, out, bf)) != MFT_OK)
        return r;
    ro = 0;
    for (int i = 0; i < desc->n_slices; ++i) {
        const mft_lora_slice& s = desc->slices[i];
        // y[:, col0 .. col0 + cols] += scale * u_i . B_i
        if ((r = mft::blas::gemm_rm(who, h, N, s.cols, s.rank, s.scale, u + ro, R, false, s.B,
                                    s.b_transposed ? s.rank : s.cols, s.b_transposed != 0, 1.f, y + s.col0, out,
                                    false)) != MFT_OK)
            return r;
        ro += s.rank;
    }
    return MFT_OK;
}

mft_status mft_lora_bwd(const mft_lora_desc* desc, const float* x, const void* W, const float* dy, const float* u,
                        float* dx, void* workspace, hipStream_t stream) {
    static const char* who = "mft_lora_bwd";
    mft_status r = check(desc, who);
    if (r != MFT_OK) return r;
    if (!x || !W || !dy || !workspace || (desc->n_slices > 0 && !u))
        return fail(MFT_ERR_INVALID_ARG, "mft_lora_bwd: x, W, dy, u (with slices) and workspace must be non-NULL");
    const BwdLayout l = bwd_layout(desc);
    char* ws = static_cast<char*>(workspace);
    const int64_t N = desc->N, in = desc->in_dim, out = desc->out_dim, R = total_rank(desc);
    const bool bf = desc->w_dtype == MFT_BF16;
    float* g = reinterpret_cast<float*>(ws + l.g);
    float* part = reinterpret_cast<float*>(ws + l.part);

    // bf16 W: the dx GEMM reads dy rounded to bf16, written by the rowdot of
    // the first slice that spans all columns and gets gradients (one read of
    // dy), or else by lora_round_bf16.
    uint16_t* dyb = dx && bf ? reinterpret_cast<uint16_t*>(ws + l.dyb) : nullptr;
    int fuse = -1;
    for (int i = 0; dyb && fuse < 0 && i < desc->n_slices; ++i) {
        const mft_lora_slice& s = desc->slices[i];
        if (s.col0 == 0 && s.cols == out && has_grad(desc, s)) fuse = i;
    }
    if (dyb && fuse < 0) {
        const hipError_t e = mft::launch_lora_round_bf16(dy, dyb, N * out, stream);
        if (e != hipSuccess) return hip_status(e, "mft_lora_bwd launch");
    }
    const void* dyo = dyb ? static_cast<const void*>(dyb) : dy;

    auto lock = mft::blas::lock();
    rocblas_handle h;
    if ((r = mft::blas::bind(who, stream, ws + l.blas, kBlasWorkspace, &h)) != MFT_OK) return r;
    int64_t ro = 0;
    for (int i = 0; i < desc->n_slices; ++i) {
        const mft_lora_slice& s = desc->slices[i];
        const int64_t rk = s.rank;
        if (has_grad(desc, s)) {
            const float* dys = dy + s.col0;
            // g_i[N, r] = scale * dy_slice . B_eff^T, B_eff(j, o) = B[j, o] or B[o, j]
            if ((r = rowdot(dys, out, N, s.cols, s.B, s.b_transposed ? rk : 1, s.b_transposed ? 1 : s.cols, g + ro, R,
                            rk, s.scale, reinterpret_cast<float*>(ws + l.pt), stream, "mft_lora_bwd launch",
                            i == fuse ? dyb : nullptr)) != MFT_OK)
                return r;
            // grad_B(o, j) = scale * sum_n dy[n, col0 + o] u_i[n, j], stored [r, cols] or [cols, r]
            if (s.grad_B && (r = coldot(dys, out, N, s.cols, u + ro, R, rk, s.scale, part, s.grad_B,
                                        s.b_transposed ? rk : 1, s.b_transposed ? 1 : s.cols, stream,
                                        "mft_lora_bwd launch")) != MFT_OK)
                return r;
            // grad_A(i, j) = sum_n x[n, i] g_i[n, j], stored [in, r] or [r, in]
            if (s.grad_A && (r = coldot(x, in, N, in, g + ro, R, rk, 1.f, part, s.grad_A, s.a_transposed ? 1 : rk,
                                        s.a_transposed ? in : 1, stream, "mft_lora_bwd launch")) != MFT_OK)
                return r;
        }
        ro += rk;
    }
    if (!dx) return MFT_OK;
    const WOperand wo = w_for_backward(desc);
    if ((r = mft::blas::gemm_rm(who, h, N, in, out, 1.f, dyo, out, false, W, wo.ld, wo.t, 0.f, dx, in, bf)) != MFT_OK)
        return r;
    ro = 0;
    for (int i = 0; i < desc->n_slices; ++i) {
        const mft_lora_slice& s = desc->slices[i];
        // dx += g_i . A_i^T
        if (has_grad(desc, s) &&
            (r = mft::blas::gemm_rm(who, h, N, in, s.rank, 1.f, g + ro, R, false, s.A, s.a_transposed ? in : s.rank,
                                    s.a_transposed == 0, 1.f, dx, in, false)) != MFT_OK)
            return r;
        ro += s.rank;
    }
    return MFT_OK;
}

mft_status mft_lora_merge(const mft_lora_desc* desc, void* W, float sign, hipStream_t stream) {
    mft_status r = check(desc, "mft_lora_merge");
    if (r != MFT_OK) return r;
    if (!W) return fail(MFT_ERR_INVALID_ARG, "mft_lora_merge: W must be non-NULL");
    for (int i = 0; i < desc->n_slices; ++i) {
        const mft_lora_slice& s = desc->slices[i];
        mft::LoraMergeArgs a{};
        a.W = W;
        a.A = s.A;
        a.B = s.B;
        a.sign_scale = sign * s.scale;
        a.w_bf16 = desc->w_dtype == MFT_BF16;
        a.w_transposed = desc->w_transposed;
        a.a_transposed = s.a_transposed;
        a.b_transposed = s.b_transposed;
        a.in = desc->in_dim;
        a.out = desc->out_dim;
        a.rank = s.rank;
        a.col0 = s.col0;
        a.cols = s.cols;
        const hipError_t e = mft::launch_lora_merge(a, stream);
        if (e != hipSuccess) return hip_status(e, "mft_lora_merge launch");
    }
    return MFT_OK;
}

}  // extern "C"
