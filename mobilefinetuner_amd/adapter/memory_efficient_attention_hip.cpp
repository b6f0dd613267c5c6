// finetune_ops adapter: ops::memory_efficient_attention on the MI355X kernels.
//
// Drop-in replacement for operator/finetune_ops/core/memory_efficient_attention.cpp
// (the reference's translation unit of core/memory_efficient_attention.h).  It is
// compiled against the reference's own headers (tensor.h, ops.h, autograd_engine.h,
// backward_functions.h, memory_efficient_attention.h) and links libmft_attn.so
// through the C ABI of include/mft/attention.h; the rest of finetune_ops is
// unchanged.  Behaviour versus the reference:
//
//   * Same signature and config (core/memory_efficient_attention.h:26-55); the
//     scale rule (config.scale > 0 else 1/sqrt(D), .cpp:103) and the shape
//     errors (std::runtime_error, .cpp:85-100) are kept.
//   * With grad (.cpp:106-108 routes to the S x S composite), the fused forward
//     runs instead and ONE autograd node is registered,
//     (O, {q, k, v}, FusedAttentionBackward), which keeps Q, K, V, O and the
//     per-row log-sum-exp on the device: O(S) per head instead of the four
//     S x S fp32 tensors the composite's nodes hold.  apply() returns fp32
//     {dQ, dK, dV} shaped like the inputs (core/backward_functions.h:12-16).
//   * Without grad (.cpp:110-200), the same fused forward (no LSE kept).
//   * Extensions: k/v may have Hkv heads with Hkv | Hq (the reference throws:
//     GQA callers materialise repeat_kv_heads first); q/k/v may be bf16
//     (computed bf16 x bf16 -> fp32 on MFMA).  The output is fp32 as in the
//     reference (.cpp:122).
//   * Masks: nullptr, an all-zero [S,S] mask, or the canonical causal mask
//     (create_causal_mask, core/ops.cpp:2167-2180: 0 on/below the diagonal,
//     <= -1e9 above) map to the kernels' causal flag with the reference's
//     precedence.  Other additive masks are rejected with an error (there is
//     no CPU fallback).
//   * Tensors are the reference's host tensors: inputs are copied to the GPU,
//     results back (PCIe-inclusive).  Device-resident callers use the C ABI.
#include "memory_efficient_attention.h"

#include <cmath>
#include <cstring>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include <hip/hip_runtime.h>

#include "autograd_engine.h"
#include "backward_functions.h"
#include "mft/attention.h"
#include "ops.h"

namespace ops {
namespace {

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string("memory_efficient_attention: ") + what + ": " +
                                                  hipGetErrorString(e));
}

void mft_check(mft_status st) {
    if (st != MFT_OK) throw std::runtime_error(std::string("memory_efficient_attention: ") + mft_last_error());
}

// One stream for the adapter's work (default priority), created on first use.
hipStream_t adapter_stream() {
    static std::once_flag once;
    static hipStream_t s = nullptr;
    std::call_once(once, [] { hip_check(hipStreamCreate(&s), "hipStreamCreate"); });
    return s;
}

// Device buffer owned by the adapter (freed when the last owner goes away).
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t bytes) : bytes_(bytes) {
        if (bytes) hip_check(hipMalloc(&ptr_, bytes), "hipMalloc");
    }
    ~DeviceBuffer() {
        if (ptr_) (void)hipFree(ptr_);
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    void* get() const { return ptr_; }
    size_t bytes() const { return bytes_; }

private:
    void* ptr_ = nullptr;
    size_t bytes_ = 0;
};

size_t elt_size(DType t) { return t == kBFloat16 ? 2 : 4; }

std::unique_ptr<DeviceBuffer> upload(const TensorPtr& t) {
    const size_t n = static_cast<size_t>(t->numel()) * elt_size(t->dtype());
    auto buf = std::make_unique<DeviceBuffer>(n);
    hip_check(hipMemcpyAsync(buf->get(), t->data_ptr(), n, hipMemcpyHostToDevice, adapter_stream()),
              "copy to device");
    return buf;
}

// Device O (input dtype) -> a new fp32 host tensor.
TensorPtr download_as_f32(const DeviceBuffer& src, const std::vector<int64_t>& shape, DType dtype) {
    auto out = zeros(shape, kFloat32, kCPU);
    const size_t n = static_cast<size_t>(out->numel());
    if (dtype == kFloat32) {
        hip_check(hipMemcpyAsync(out->data<float>(), src.get(), n * 4, hipMemcpyDeviceToHost, adapter_stream()),
                  "copy to host");
        hip_check(hipStreamSynchronize(adapter_stream()), "synchronize");
    } else {
        std::vector<uint16_t> bits(n);
        hip_check(hipMemcpyAsync(bits.data(), src.get(), n * 2, hipMemcpyDeviceToHost, adapter_stream()),
                  "copy to host");
        hip_check(hipStreamSynchronize(adapter_stream()), "synchronize");
        float* o = out->data<float>();
        for (size_t i = 0; i < n; ++i) o[i] = bf16_bits_to_float32(bits[i]);
    }
    return out;
}

TensorPtr download_f32(const DeviceBuffer& src, const std::vector<int64_t>& shape) {
    auto out = zeros(shape, kFloat32, kCPU);
    hip_check(hipMemcpyAsync(out->data<float>(), src.get(), static_cast<size_t>(out->numel()) * 4,
                             hipMemcpyDeviceToHost, adapter_stream()),
              "copy to host");
    return out;
}

enum class MaskKind { kNone, kZero, kCausal, kOther };

// Classifies an additive [S,S] mask (the reference adds it to the scaled
// scores, core/ops.cpp:415-442).  Entries <= -1e9 are "masked": exp(-1e9 - m)
// underflows to exactly 0 in fp32 for any score range the ops produce.
MaskKind classify_mask(const TensorPtr& mask, int64_t S) {
    if (!mask) return MaskKind::kNone;
    if (mask->shape().size() != 2 || mask->shape()[0] != S || mask->shape()[1] != S)
        throw std::runtime_error("memory_efficient_attention: causal_mask must be [S,S]");
    if (mask->dtype() != kFloat32) return MaskKind::kOther;
    const float* m = mask->data<float>();
    bool zero = true, causal = true;
    for (int64_t i = 0; i < S && (zero || causal); ++i) {
        for (int64_t j = 0; j < S; ++j) {
            const float x = m[i * S + j];
            if (j <= i) {
                if (x != 0.0f) zero = causal = false;
            } else {
                if (x != 0.0f) zero = false;
                if (!(x <= -1e9f)) causal = false;
            }
        }
    }
    return zero ? MaskKind::kZero : causal ? MaskKind::kCausal : MaskKind::kOther;
}

// What the kernels hold between forward and backward.
struct SavedForBackward {
    mft_attn_desc desc{};
    std::vector<int64_t> q_shape, kv_shape;
    std::unique_ptr<DeviceBuffer> q, k, v, o, lse;
};

class FusedAttentionBackward : public BackwardFunction {
public:
    explicit FusedAttentionBackward(std::shared_ptr<SavedForBackward> s) : s_(std::move(s)) {}

    // grad_output: fp32 [B, Hq, S, D].  Returns fp32 {dQ, dK, dV} (dK, dV
    // summed over the query heads that share each kv head).
    std::vector<TensorPtr> apply(const TensorPtr& grad_output) override {
        if (!s_) throw std::runtime_error("FusedAttentionBackward: applied twice");
        if (!grad_output || grad_output->shape() != s_->q_shape || grad_output->dtype() != kFloat32)
            throw std::runtime_error("FusedAttentionBackward: grad_output must be fp32 shaped like q");
        const mft_attn_desc& d = s_->desc;
        const size_t n_q = static_cast<size_t>(grad_output->numel());
        const size_t n_kv = static_cast<size_t>(d.B * d.Hkv * d.S * d.D);
        hipStream_t st = adapter_stream();

        DeviceBuffer dO(n_q * (d.dtype == MFT_BF16 ? 2 : 4));
        std::vector<uint16_t> bits;
        if (d.dtype == MFT_BF16) {
            // dO enters the bf16 kernels rounded like every other bf16 operand
            // (core/dtype.h:114-121).
            bits.resize(n_q);
            const float* g = grad_output->data<float>();
            for (size_t i = 0; i < n_q; ++i) bits[i] = float32_to_bf16_bits(g[i]);
            hip_check(hipMemcpyAsync(dO.get(), bits.data(), n_q * 2, hipMemcpyHostToDevice, st), "copy dO");
        } else {
            hip_check(hipMemcpyAsync(dO.get(), grad_output->data<float>(), n_q * 4, hipMemcpyHostToDevice, st),
                      "copy dO");
        }
        size_t fwd_ws = 0, bwd_ws = 0;
        mft_check(mft_attn_workspace_size(&d, &fwd_ws, &bwd_ws));
        DeviceBuffer ws(bwd_ws), dq(n_q * 4), dk(n_kv * 4), dv(n_kv * 4);
        mft_check(mft_attn_bwd(&d, s_->q->get(), s_->k->get(), s_->v->get(), s_->o->get(), dO.get(),
                               static_cast<const float*>(s_->lse->get()), static_cast<float*>(dq.get()),
                               static_cast<float*>(dk.get()), static_cast<float*>(dv.get()), ws.get(), st));
        auto gq = download_f32(dq, s_->q_shape);
        auto gk = download_f32(dk, s_->kv_shape);
        auto gv = download_f32(dv, s_->kv_shape);
        hip_check(hipStreamSynchronize(st), "synchronize");
        s_.reset();  // the graph is single-use (Engine::clear_graph, core/autograd_engine.cpp:275-287)
        return {gq, gk, gv};
    }

private:
    std::shared_ptr<SavedForBackward> s_;
};

}  // namespace

// Not on the hot path: the reference's per-row helper (unused by its own
// operator), kept so that the replacement defines every symbol the header
// declares.  Two passes: the double-precision normaliser, then the weighted sum.
void online_softmax_weighted_sum(const float* logits, const float* values, int64_t seq_len, int64_t head_dim,
                                 float* output, float max_val) {
    double norm = 0.0;
    for (int64_t j = 0; j < seq_len; ++j) norm += std::exp(logits[j] - max_val);
    const float inv = 1.0f / static_cast<float>(norm);
    for (int64_t j = 0; j < seq_len; ++j) {
        const float w = std::exp(logits[j] - max_val) * inv;
        for (int64_t d = 0; d < head_dim; ++d) output[d] += w * values[j * head_dim + d];
    }
}

TensorPtr memory_efficient_attention(const TensorPtr& q, const TensorPtr& k, const TensorPtr& v,
                                     const TensorPtr& causal_mask, const MemoryEfficientAttentionConfig& config) {
    if (!q || !k || !v) throw std::runtime_error("memory_efficient_attention: null input");
    const auto& qs = q->shape();
    const auto& ks = k->shape();
    const auto& vs = v->shape();
    if (qs.size() != 4 || ks.size() != 4 || vs.size() != 4)
        throw std::runtime_error("memory_efficient_attention: inputs must be 4D [B,H,S,D]");
    const int64_t B = qs[0], Hq = qs[1], S = qs[2], D = qs[3], Hkv = ks[1];
    if (ks[0] != B || ks[2] != S || ks[3] != D || Hkv <= 0 || Hq % Hkv != 0)
        throw std::runtime_error("memory_efficient_attention: k shape mismatch");
    if (vs != ks) throw std::runtime_error("memory_efficient_attention: v shape mismatch");
    const DType dt = q->dtype();
    if ((dt != kFloat32 && dt != kBFloat16) || k->dtype() != dt || v->dtype() != dt)
        throw std::runtime_error("memory_efficient_attention: q, k, v must all be float32 or all bfloat16");
    if (!q->device().is_cpu() || !k->device().is_cpu() || !v->device().is_cpu())
        throw std::runtime_error("memory_efficient_attention: expects host tensors");
    const float scale = (config.scale > 0) ? config.scale : (1.0f / std::sqrt(static_cast<float>(D)));
    const bool needs_grad = q->requires_grad() || k->requires_grad() || v->requires_grad();

    // Causal flag with the reference's precedence: the grad path (composite,
    // .cpp:23-43) uses the given mask instead of use_causal_mask; the no-grad
    // path (.cpp:163-172) applies use_causal_mask and then adds the mask.
    const MaskKind mk = classify_mask(causal_mask, S);
    bool causal = config.use_causal_mask;
    if (mk == MaskKind::kOther)
        throw std::runtime_error(
            "memory_efficient_attention: only the causal mask (or none) is supported on the GPU path");
    if (mk == MaskKind::kCausal) causal = true;
    if (mk == MaskKind::kZero && needs_grad) causal = false;

    mft_attn_desc d{};
    d.B = B;
    d.Hq = Hq;
    d.Hkv = Hkv;
    d.S = S;
    d.D = D;
    d.scale = scale;
    d.causal = causal ? 1 : 0;
    d.dtype = dt == kBFloat16 ? MFT_BF16 : MFT_F32;

    auto saved = std::make_shared<SavedForBackward>();
    saved->desc = d;
    saved->q_shape = qs;
    saved->kv_shape = ks;
    saved->q = upload(q);
    saved->k = upload(k);
    saved->v = upload(v);
    saved->o = std::make_unique<DeviceBuffer>(static_cast<size_t>(q->numel()) * elt_size(dt));
    if (needs_grad) saved->lse = std::make_unique<DeviceBuffer>(static_cast<size_t>(B * Hq * S) * 4);
    size_t fwd_ws = 0, bwd_ws = 0;
    mft_check(mft_attn_workspace_size(&d, &fwd_ws, &bwd_ws));
    DeviceBuffer ws(fwd_ws);
    mft_check(mft_attn_fwd(&d, saved->q->get(), saved->k->get(), saved->v->get(), saved->o->get(),
                           needs_grad ? static_cast<float*>(saved->lse->get()) : nullptr, ws.get(),
                           adapter_stream()));
    auto out = download_as_f32(*saved->o, qs, dt);

    if (needs_grad) {
        out->set_requires_grad(true);
        autograd::Engine::instance().register_node(out, {q, k, v},
                                                   std::make_shared<FusedAttentionBackward>(saved));
    }
    return out;
}

}  // namespace ops
