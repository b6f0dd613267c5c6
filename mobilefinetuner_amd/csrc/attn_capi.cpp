// C ABI of the fused attention (declared in include/mft/attention.h).
//
// Validates the request the way the reference validates its operator inputs
// (core/memory_efficient_attention.cpp:85-103: 4-D shapes, matching sizes,
// scale <= 0 meaning 1/sqrt(D)), resolves the workspace layout, and enqueues
// the kernels.  Errors are reported as a status plus a thread-local message;
// nothing is allocated here.
#include "mft/attention.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <mutex>
#include <string>

#include "attn_kernels.h"
#include "capi_util.h"

namespace mft {
namespace capi {

thread_local std::string g_last_error;

mft_status fail(mft_status st, const std::string& msg) {
    g_last_error = msg;
    return st;
}

mft_status resolve_layout(const mft_strides& st, int64_t H, int64_t S, int64_t D, int64_t esz, const char* who,
                          const char* name, Strides* out, bool* dense_out) {
    const Strides dense{H * S * D, S * D, (int)D};
    if ((st.b == 0 && st.h == 0 && st.s == 0) || (st.b == dense.b && st.h == dense.h && st.s == dense.s)) {
        *out = dense;  // contiguous [B, H, S, D]
        *dense_out = true;
        return MFT_OK;
    }
    const int64_t unit = 16 / esz;  // 16-byte rows
    if (st.b <= 0 || st.h <= 0 || st.s <= 0 || st.b % unit || st.h % unit || st.s % unit)
        return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": strides of " + name +
                                             " must be positive multiples of 16 bytes (or all zero)");
    if (st.s < D)
        return fail(MFT_ERR_INVALID_ARG, std::string(who) + ": sequence stride of " + name +
                                             " is shorter than a row (D)");
    if ((S - 1) * st.s + D > (int64_t(1) << 31) - 1)
        return fail(MFT_ERR_UNSUPPORTED, std::string(who) + ": one (batch, head) block of " + name +
                                             " spans 2^31 elements or more");
    *out = Strides{st.b, st.h, (int)st.s};
    *dense_out = false;
    return MFT_OK;
}

// Tensors are read and written in 16-byte vectors.
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

mft_status hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return MFT_OK;
    return fail(MFT_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace capi
}  // namespace mft

namespace {

using namespace mft::capi;

mft_status check_desc(const mft_attn_desc* d, mft::AttnShape* s) {
    if (!d) return fail(MFT_ERR_INVALID_ARG, "mft_attn: desc is NULL");
    if (d->B <= 0 || d->Hq <= 0 || d->Hkv <= 0 || d->S <= 0 || d->D <= 0)
        return fail(MFT_ERR_INVALID_ARG, "mft_attn: B, Hq, Hkv, S, D must be positive (inputs must be 4D [B,H,S,D])");
    if (d->Hq % d->Hkv != 0)
        return fail(MFT_ERR_INVALID_ARG, "mft_attn: query heads (" + std::to_string(d->Hq) +
                                             ") must be a multiple of kv heads (" + std::to_string(d->Hkv) + ")");
    if (d->dtype != MFT_F32 && d->dtype != MFT_BF16)
        return fail(MFT_ERR_INVALID_ARG, "mft_attn: dtype must be MFT_F32 or MFT_BF16");
    if (d->D > 256) return fail(MFT_ERR_UNSUPPORTED, "mft_attn: head_dim > 256 is not supported");
    if (d->S > (int64_t(1) << 24)) return fail(MFT_ERR_UNSUPPORTED, "mft_attn: sequence length > 2^24");
    if (d->S * d->D > (int64_t(1) << 31) - 1)
        return fail(MFT_ERR_UNSUPPORTED, "mft_attn: one head block exceeds 2^31 elements");
    if (d->B * d->Hq > 65535 || d->B > 65535 || d->Hq > 65535)
        return fail(MFT_ERR_UNSUPPORTED, "mft_attn: batch/head grid dimensions too large");
    if (!(std::isfinite(d->scale)))
        return fail(MFT_ERR_INVALID_ARG, "mft_attn: scale must be finite");
    if (d->window < 0) return fail(MFT_ERR_INVALID_ARG, "mft_attn: window must be >= 0");
    if (d->window > 0 && !d->causal)
        return fail(MFT_ERR_INVALID_ARG, "mft_attn: a sliding window needs causal = 1 (j <= i && i - j < window)");
    if ((reinterpret_cast<uintptr_t>(d->kv_len) & 3u) != 0)
        return fail(MFT_ERR_INVALID_ARG, "mft_attn: kv_len must be 4-byte aligned");
    const int64_t esize = d->dtype == MFT_BF16 ? 2 : 4;
    struct Named {
        const mft_strides* st;
        const char* name;
        int64_t H;
        int64_t esz;
    };
    const Named layouts[] = {{&d->q, "q", d->Hq, esize},  {&d->k, "k", d->Hkv, esize}, {&d->v, "v", d->Hkv, esize},
                             {&d->o, "o", d->Hq, esize},  {&d->dO, "dO", d->Hq, esize}, {&d->dq, "dq", d->Hq, 4},
                             {&d->dk, "dk", d->Hkv, 4},  {&d->dv, "dv", d->Hkv, 4}};
    mft::Strides* out[] = {&s->q, &s->k, &s->v, &s->o, &s->dO, &s->dq, &s->dk, &s->dv};
    s->contiguous = true;
    for (int i = 0; i < 8; ++i) {
        bool dense = true;
        const mft_status r = resolve_layout(*layouts[i].st, layouts[i].H, d->S, d->D, layouts[i].esz, "mft_attn",
                                            layouts[i].name, out[i], &dense);
        if (r != MFT_OK) return r;
        s->contiguous = s->contiguous && dense;
    }
    s->B = d->B;
    s->Hq = d->Hq;
    s->Hkv = d->Hkv;
    s->S = d->S;
    s->D = d->D;
    s->scale = d->scale > 0.f ? d->scale : 1.0f / std::sqrt(static_cast<float>(d->D));
    s->causal = d->causal != 0;
    s->bf16 = d->dtype == MFT_BF16;
    // A window of S or more keys hides nothing beyond the causal mask.
    s->window = d->window < d->S ? d->window : 0;
    s->kv_len = d->kv_len;
    // Mask mode.
    const mft_mask* masks[2] = {&d->mask0, &d->mask1};
    mft::MaskView* views[2] = {&s->m0, &s->m1};
    for (int i = 0; i < 2; ++i) {
        const mft_mask& m = *masks[i];
        *views[i] = mft::MaskView{m.ptr, m.sb, m.sh, m.si, m.sj};
        if (!m.ptr) continue;
        if ((reinterpret_cast<uintptr_t>(m.ptr) & 3u) != 0)
            return fail(MFT_ERR_INVALID_ARG, "mft_attn: masks must be 4-byte aligned fp32");
        if (m.sb < 0 || m.sh < 0 || m.si < 0 || m.sj < 0)
            return fail(MFT_ERR_INVALID_ARG, "mft_attn: mask strides must be >= 0");
    }
    s->masked = d->mask0.ptr || d->mask1.ptr;
    if (s->masked && (d->window != 0 || d->kv_len))
        return fail(MFT_ERR_UNSUPPORTED, "mft_attn: with mask0/mask1, window must be 0 and kv_len NULL "
                                         "(express them in the masks)");
    return MFT_OK;
}

// Each call plans its work once (plan_fwd_split / plan_bwd_fast) and passes
// the plan to the workspace layout and the launches.  The planners keep at
// most kSplitMaxSlots partial slots per tile (fit_unit_split lowers the unit
// count until that holds; tests/native/plan_check.cpp sweeps it), which the
// merge kernels' LDS slot lists rely on.

// Scratch of mft_attn_bwd_noalloc: the backward workspace (row terms, fp32
// partial tiles) of callers that cannot allocate.  One copy per GPU, held
// until the process ends; the host only ever uses its per-device address.
constexpr size_t kNoAllocScratchBytes = size_t(128) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's copy of `scratch`, looked up once per device (with
// that device current) on its first use.
mft_status scratch_for_current_device(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, "mft_attn_bwd_noalloc: hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices)
        return fail(MFT_ERR_UNSUPPORTED, "mft_attn_bwd_noalloc: device index " + std::to_string(dev) +
                                             " is beyond the " + std::to_string(kMaxDevices) + " supported");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_status(e, "mft_attn_bwd_noalloc: hipGetSymbolAddress(scratch)");
        if (!p) return fail(MFT_ERR_HIP, "mft_attn_bwd_noalloc: hipGetSymbolAddress(scratch) returned NULL");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return MFT_OK;
}

}  // namespace

extern "C" {

int mft_version(void) { return 7; }

const char* mft_last_error(void) { return mft::capi::g_last_error.c_str(); }

mft_status mft_attn_workspace_size(const mft_attn_desc* desc, size_t* fwd_bytes, size_t* bwd_bytes) {
    mft::AttnShape s;
    const mft_status st = check_desc(desc, &s);
    if (st != MFT_OK) return st;
    if (fwd_bytes) *fwd_bytes = mft::fwd_workspace_bytes(s, mft::plan_fwd_split(s));
    if (bwd_bytes) *bwd_bytes = mft::bwd_layout(s, mft::plan_bwd_fast(s)).total;
    return MFT_OK;
}

mft_status mft_attn_fwd(const mft_attn_desc* desc, const void* q, const void* k, const void* v, void* o,
                        float* lse, void* workspace, hipStream_t stream) {
    mft::AttnShape s;
    const mft_status st = check_desc(desc, &s);
    if (st != MFT_OK) return st;
    if (!q || !k || !v || !o) return fail(MFT_ERR_INVALID_ARG, "mft_attn_fwd: q, k, v, o must be non-NULL");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || !aligned16(lse) || !aligned16(workspace))
        return fail(MFT_ERR_INVALID_ARG, "mft_attn_fwd: buffers must be 16-byte aligned");
    return hip_status(mft::launch_attn_fwd(s, mft::plan_fwd_split(s), q, k, v, o, lse, workspace, stream),
                      "mft_attn_fwd launch");
}

}  // extern "C"

namespace {

// mft_attn_bwd_stage for a checked shape and its plan.
mft_status bwd_stage(const mft::AttnShape& s, const mft::BwdPlan& p, int stages, const void* q, const void* k,
                     const void* v, const void* o, const void* dO, const float* lse, float* dq, float* dk, float* dv,
                     void* workspace, hipStream_t stream) {
    if (stages <= 0 || (stages & ~MFT_BWD_ALL) != 0)
        return fail(MFT_ERR_INVALID_ARG, "mft_attn_bwd_stage: stages must be a non-empty mask of MFT_BWD_*");
    if (!q || !k || !v || !o || !dO || !lse || !dq || !dk || !dv)
        return fail(MFT_ERR_INVALID_ARG, "mft_attn_bwd: q, k, v, o, dO, lse, dq, dk, dv must be non-NULL");
    if (!workspace) return fail(MFT_ERR_INVALID_ARG, "mft_attn_bwd: workspace is NULL (see mft_attn_workspace_size)");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || !aligned16(dO) || !aligned16(lse) ||
        !aligned16(dq) || !aligned16(dk) || !aligned16(dv) || !aligned16(workspace))
        return fail(MFT_ERR_INVALID_ARG, "mft_attn_bwd: buffers must be 16-byte aligned");
    return hip_status(mft::launch_attn_bwd(s, p, q, k, v, o, dO, lse, dq, dk, dv, workspace, stages, stream),
                      "mft_attn_bwd launch");
}

}  // namespace

extern "C" {

mft_status mft_attn_bwd_stage(const mft_attn_desc* desc, int stages, const void* q, const void* k,
                              const void* v, const void* o, const void* dO, const float* lse, float* dq,
                              float* dk, float* dv, void* workspace, hipStream_t stream) {
    mft::AttnShape s;
    const mft_status st = check_desc(desc, &s);
    if (st != MFT_OK) return st;
    return bwd_stage(s, mft::plan_bwd_fast(s), stages, q, k, v, o, dO, lse, dq, dk, dv, workspace, stream);
}

mft_status mft_attn_bwd(const mft_attn_desc* desc, const void* q, const void* k, const void* v, const void* o,
                        const void* dO, const float* lse, float* dq, float* dk, float* dv, void* workspace,
                        hipStream_t stream) {
    return mft_attn_bwd_stage(desc, MFT_BWD_ALL, q, k, v, o, dO, lse, dq, dk, dv, workspace, stream);
}

mft_status mft_attn_bwd_noalloc(const mft_attn_desc* desc, const void* q, const void* k, const void* v,
                                const void* o, const void* dO, const float* lse, float* dq, float* dk, float* dv,
                                hipStream_t stream) {
    mft::AttnShape s;
    const mft_status st = check_desc(desc, &s);
    if (st != MFT_OK) return st;
    const mft::BwdPlan plan = mft::plan_bwd_fast(s);
    const size_t need = mft::bwd_layout(s, plan).total;
    if (need > kNoAllocScratchBytes)
        return fail(MFT_ERR_UNSUPPORTED,
                    "mft_attn_bwd_noalloc: this shape needs " + std::to_string(need) +
                        " bytes of backward workspace, more than the library's fixed scratch of " +
                        std::to_string(kNoAllocScratchBytes) +
                        " bytes; call mft_attn_bwd with a workspace of mft_attn_workspace_size bytes");
    void* ws = nullptr;
    const mft_status sp = scratch_for_current_device(&ws);
    if (sp != MFT_OK) return sp;
    // Every workspace byte the backward reads is written earlier in the same
    // call (row terms by DELTA, partial tiles by their work units), so
    // nothing has to start at zero.
    return bwd_stage(s, plan, MFT_BWD_ALL, q, k, v, o, dO, lse, dq, dk, dv, ws, stream);
}

mft_status mft_repeat_kv_fwd(const void* kv, void* out, int64_t B, int64_t Hkv, int64_t S, int64_t D, int64_t r,
                             mft_dtype dtype, hipStream_t stream) {
    if (!kv || !out) return fail(MFT_ERR_INVALID_ARG, "mft_repeat_kv_fwd: kv and out must be non-NULL");
    if (B <= 0 || Hkv <= 0 || S <= 0 || D <= 0 || r <= 0)
        return fail(MFT_ERR_INVALID_ARG, "repeat_kv_heads expects 4D tensor with positive sizes and repeat factor");
    if (dtype != MFT_F32 && dtype != MFT_BF16)
        return fail(MFT_ERR_INVALID_ARG, "mft_repeat_kv_fwd: dtype must be MFT_F32 or MFT_BF16");
    const int esize = dtype == MFT_F32 ? 4 : 2;
    return hip_status(mft::launch_repeat_kv_fwd(kv, out, B, Hkv, S, D, r, esize, stream), "mft_repeat_kv_fwd launch");
}

mft_status mft_repeat_kv_bwd(const float* g, float* dkv, int64_t B, int64_t Hkv, int64_t S, int64_t D, int64_t r,
                             hipStream_t stream) {
    if (!g || !dkv) return fail(MFT_ERR_INVALID_ARG, "mft_repeat_kv_bwd: g and dkv must be non-NULL");
    if (B <= 0 || Hkv <= 0 || S <= 0 || D <= 0 || r <= 0)
        return fail(MFT_ERR_INVALID_ARG, "RepeatKVHeadsBackward expects 4D gradient with positive sizes");
    return hip_status(mft::launch_repeat_kv_bwd(g, dkv, B, Hkv, S, D, r, stream), "mft_repeat_kv_bwd launch");
}

}  // extern "C"
