// finetune_ops adapter: the language-model losses on the MI355X kernels.
//
// Drop-in replacement for operator/finetune_ops/core/lm_loss.cpp (the
// reference's translation unit of core/lm_loss.h), compiled against the
// reference's own headers and linked to libmft_attn.so through the C ABI of
// include/mft/lm_loss.h.  Behaviour versus the reference:
//
//   * lm_cross_entropy (core/lm_loss.cpp:268-382): the HF shift, ignore_index,
//     "mean" (NaN with nothing scored), "sum", "sum_debug" (scored like
//     "sum"; its backward, like "sum"'s, is not normalised) and "none" ([B, S]
//     per-position NLL).  Any other reduction string scores like "mean" but,
//     as in the reference (LMCrossEntropyBackward normalises only for exactly
//     "mean", core/lm_loss.cpp:96-100), its backward is not normalised.  The
//     backward node (inputs {logits}) runs mft_lm_ce_bwd.
//   * selected_token_lm_cross_entropy / streaming_lm_cross_entropy
//     (core/lm_loss.cpp:384-481): the loss from hidden and lm_head_weight
//     without a [B, S, V] logits tensor, "mean" or "sum" only; the backward
//     node (inputs {hidden, lm_head_weight, labels}) runs
//     mft_lm_ce_streaming_bwd and returns a gradient only for the inputs that
//     require one.  An fp16 / bf16 weight is widened to fp32 exactly, as
//     tensor_row_value does, so the arithmetic stays fp32 like the reference's.
//   * A label outside [0, V) that is not ignore_index throws
//     "lm_cross_entropy: label out of range" from the forward; the kernels
//     detect it and report it through the C ABI's status word.
//   * Tensors are the reference's host tensors: inputs are copied to the GPU,
//     results back (PCIe-inclusive).  What the backward needs stays on the
//     device in the node.  Device-resident callers use the C ABI.
#include "lm_loss.h"

#include <cmath>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include <hip/hip_runtime.h>

#include "autograd_engine.h"
#include "backward_functions.h"
#include "ops.h"
#include "mft/lm_loss.h"
#include "dropin_device.h"

namespace ops {
namespace {

constexpr const char* kWho = "lm_loss";
void hip_check(hipError_t e, const char* what) { dropin::hip_check(kWho, e, what); }
void mft_check(mft_status st) { dropin::mft_check(kWho, st); }
hipStream_t loss_stream() { return dropin::stream(); }
using dropin::Buf;
using dropin::DeviceBuffer;
using dropin::download_f32;
using dropin::upload_bytes;
using dropin::upload_f32;

Buf upload_labels(const TensorPtr& labels, const char* who) {
    if (labels->dtype() != kInt32) throw std::runtime_error(std::string(who) + ": labels must be int32");
    return upload_bytes(labels->data<int32_t>(), static_cast<size_t>(labels->numel()) * 4);
}

// grad_output as the C ABI's device grad_loss: n values (1, or B*S for
// "none"); an absent or empty gradient means 1, as in the reference.
Buf upload_grad_loss(const TensorPtr& grad_output, int64_t n) {
    std::vector<float> g(static_cast<size_t>(n), 1.0f);
    if (grad_output && grad_output->numel() > 0) {
        if (grad_output->dtype() != kFloat32 || grad_output->numel() < n)
            throw std::runtime_error("lm_loss backward: grad_output must be fp32 with one value per loss element");
        std::memcpy(g.data(), grad_output->data<float>(), static_cast<size_t>(n) * 4);
    }
    auto buf = upload_bytes(g.data(), g.size() * 4);
    hip_check(hipStreamSynchronize(loss_stream()), "synchronize");  // g is a local
    return buf;
}

// The forward's device state, kept by the backward node.
struct Saved {
    mft_lm_loss_desc desc{};
    int32_t bwd_reduction = MFT_REDUCE_MEAN;  // the backward's scaling (MEAN: 1 / scored count)
    std::vector<int64_t> in_shape, w_shape;
    Buf x, w, labels, lse;  // x: logits (dense) or hidden (streaming)
    bool grad_x = false, grad_w = false;
};

// Forward of either variant: returns the host loss tensor, throws on an
// out-of-range label (the status word the kernels set).
TensorPtr run_forward(Saved& s, const std::vector<int64_t>& loss_shape) {
    const mft_lm_loss_desc* d = &s.desc;
    size_t fwd_ws = 0, bwd_ws = 0;
    mft_check(mft_lm_ce_workspace_size(d, &fwd_ws, &bwd_ws));
    int64_t n_loss = 1;
    for (int64_t e : loss_shape) n_loss *= e;
    DeviceBuffer loss(static_cast<size_t>(n_loss) * 4), ws(fwd_ws), status(4);
    s.lse = std::make_unique<DeviceBuffer>(static_cast<size_t>(d->B * d->S) * 4);
    hip_check(hipMemsetAsync(status.get(), 0, 4, loss_stream()), "clear status");
    if (d->H == 0)
        mft_check(mft_lm_ce_fwd(d, s.x->get(), static_cast<const int32_t*>(s.labels->get()), loss.f(), s.lse->f(),
                                static_cast<int32_t*>(status.get()), ws.get(), loss_stream()));
    else
        mft_check(mft_lm_ce_streaming_fwd(d, s.x->get(), s.w->get(), static_cast<const int32_t*>(s.labels->get()),
                                          loss.f(), s.lse->f(), static_cast<int32_t*>(status.get()), ws.get(),
                                          loss_stream()));
    int32_t bad = 0;
    hip_check(hipMemcpyAsync(&bad, status.get(), 4, hipMemcpyDeviceToHost, loss_stream()), "copy to host");
    auto out = download_f32(loss, loss_shape);
    hip_check(hipStreamSynchronize(loss_stream()), "synchronize");
    if (bad) throw std::runtime_error("lm_cross_entropy: label out of range");
    return out;
}

class LMCrossEntropyBackwardHip : public BackwardFunction {
public:
    explicit LMCrossEntropyBackwardHip(std::shared_ptr<Saved> s) : s_(std::move(s)) {}

    std::vector<TensorPtr> apply(const TensorPtr& grad_output) override {
        if (!s_) throw std::runtime_error("LMCrossEntropyBackwardHip: applied twice");
        mft_lm_loss_desc bwd_desc = s_->desc;
        bwd_desc.reduction = s_->bwd_reduction;
        const mft_lm_loss_desc* d = &bwd_desc;
        const int64_t n_loss = d->reduction == MFT_REDUCE_NONE ? d->B * d->S : 1;
        Buf g = upload_grad_loss(grad_output, n_loss);
        size_t fwd_ws = 0, bwd_ws = 0;
        mft_check(mft_lm_ce_workspace_size(d, &fwd_ws, &bwd_ws));
        DeviceBuffer ws(bwd_ws), grad(static_cast<size_t>(d->B * d->S * d->V) * 4);
        mft_check(mft_lm_ce_bwd(d, s_->x->get(), static_cast<const int32_t*>(s_->labels->get()), s_->lse->f(), g->f(),
                                grad.f(), ws.get(), loss_stream()));
        auto grad_logits = download_f32(grad, s_->in_shape);
        hip_check(hipStreamSynchronize(loss_stream()), "synchronize");
        s_.reset();
        return {grad_logits};
    }

private:
    std::shared_ptr<Saved> s_;
};

class SelectedTokenLMCrossEntropyBackwardHip : public BackwardFunction {
public:
    explicit SelectedTokenLMCrossEntropyBackwardHip(std::shared_ptr<Saved> s) : s_(std::move(s)) {}

    std::vector<TensorPtr> apply(const TensorPtr& grad_output) override {
        if (!s_) throw std::runtime_error("SelectedTokenLMCrossEntropyBackwardHip: applied twice");
        const mft_lm_loss_desc* d = &s_->desc;
        Buf g = upload_grad_loss(grad_output, 1);
        size_t fwd_ws = 0, bwd_ws = 0;
        mft_check(mft_lm_ce_workspace_size(d, &fwd_ws, &bwd_ws));
        DeviceBuffer ws(bwd_ws);
        Buf gh = s_->grad_x ? std::make_unique<DeviceBuffer>(static_cast<size_t>(d->B * d->S * d->H) * 4) : nullptr;
        Buf gw = s_->grad_w ? std::make_unique<DeviceBuffer>(static_cast<size_t>(d->V * d->H) * 4) : nullptr;
        mft_check(mft_lm_ce_streaming_bwd(d, s_->x->get(), s_->w->get(),
                                          static_cast<const int32_t*>(s_->labels->get()), s_->lse->f(), g->f(),
                                          gh ? gh->f() : nullptr, gw ? gw->f() : nullptr, ws.get(), loss_stream()));
        TensorPtr grad_hidden = gh ? download_f32(*gh, s_->in_shape) : nullptr;
        TensorPtr grad_weight = gw ? download_f32(*gw, s_->w_shape) : nullptr;
        hip_check(hipStreamSynchronize(loss_stream()), "synchronize");
        s_.reset();
        return {grad_hidden, grad_weight, nullptr};
    }

private:
    std::shared_ptr<Saved> s_;
};

}  // namespace

TensorPtr lm_cross_entropy(const TensorPtr& logits, const TensorPtr& labels, int ignore_index,
                           const std::string& reduction) {
    if (logits->ndim() != 3) throw std::runtime_error("lm_cross_entropy: logits must be [B,S,V]");
    if (labels->ndim() != 2) throw std::runtime_error("lm_cross_entropy: labels must be [B,S]");
    const auto& shape = logits->shape();
    if (labels->shape()[0] != shape[0] || labels->shape()[1] != shape[1])
        throw std::runtime_error("lm_cross_entropy: labels shape must match logits [B,S]");

    auto s = std::make_shared<Saved>();
    s->desc.B = shape[0];
    s->desc.S = shape[1];
    s->desc.V = shape[2];
    s->desc.H = 0;
    s->desc.dtype = MFT_F32;
    s->desc.ignore_index = ignore_index;
    s->desc.reduction = reduction == "none" ? MFT_REDUCE_NONE
                        : (reduction == "sum" || reduction == "sum_debug") ? MFT_REDUCE_SUM
                                                                           : MFT_REDUCE_MEAN;
    s->bwd_reduction = reduction == "mean" ? MFT_REDUCE_MEAN
                       : reduction == "none" ? MFT_REDUCE_NONE
                                             : MFT_REDUCE_SUM;
    s->in_shape = shape;
    s->x = upload_f32(logits, "lm_cross_entropy");
    s->labels = upload_labels(labels, "lm_cross_entropy");
    const std::vector<int64_t> loss_shape =
        s->desc.reduction == MFT_REDUCE_NONE ? std::vector<int64_t>{shape[0], shape[1]} : std::vector<int64_t>{1};
    auto out = run_forward(*s, loss_shape);
    if (logits->requires_grad()) {
        out->set_requires_grad(true);
        autograd::Engine::instance().register_node(out, {logits}, std::make_shared<LMCrossEntropyBackwardHip>(s));
    }
    return out;
}

TensorPtr selected_token_lm_cross_entropy(const TensorPtr& hidden, const TensorPtr& lm_head_weight,
                                         const TensorPtr& labels, int ignore_index, const std::string& reduction) {
    if (!hidden || !lm_head_weight || !labels)
        throw std::runtime_error("selected_token_lm_cross_entropy: inputs must not be null");
    if (hidden->ndim() != 3) throw std::runtime_error("selected_token_lm_cross_entropy: hidden must be [B,S,H]");
    if (lm_head_weight->ndim() != 2)
        throw std::runtime_error("selected_token_lm_cross_entropy: lm_head_weight must be [V,H]");
    if (labels->ndim() != 2) throw std::runtime_error("selected_token_lm_cross_entropy: labels must be [B,S]");
    if (reduction != "mean" && reduction != "sum")
        throw std::runtime_error("selected_token_lm_cross_entropy: only mean and sum reductions are supported");
    const auto& hs = hidden->shape();
    const auto& ws = lm_head_weight->shape();
    if (ws[1] != hs[2]) throw std::runtime_error("selected_token_lm_cross_entropy: hidden H and weight H mismatch");
    if (labels->shape()[0] != hs[0] || labels->shape()[1] != hs[1])
        throw std::runtime_error("selected_token_lm_cross_entropy: labels shape must match hidden [B,S]");
    if (hidden->dtype() != kFloat32)
        throw std::runtime_error("selected_token_lm_cross_entropy: hidden must be float32");

    auto s = std::make_shared<Saved>();
    s->desc.B = hs[0];
    s->desc.S = hs[1];
    s->desc.V = ws[0];
    s->desc.H = hs[2];
    s->desc.dtype = MFT_F32;
    s->desc.ignore_index = ignore_index;
    s->desc.reduction = reduction == "sum" ? MFT_REDUCE_SUM : MFT_REDUCE_MEAN;
    s->desc.chunk = 0;
    s->in_shape = hs;
    s->w_shape = ws;
    s->x = upload_f32(hidden, "selected_token_lm_cross_entropy");
    s->w = upload_f32(lm_head_weight, "selected_token_lm_cross_entropy");
    s->labels = upload_labels(labels, "selected_token_lm_cross_entropy");
    auto out = run_forward(*s, {1});
    if (hidden->requires_grad() || lm_head_weight->requires_grad()) {
        s->grad_x = hidden->requires_grad();
        s->grad_w = lm_head_weight->requires_grad();
        out->set_requires_grad(true);
        autograd::Engine::instance().register_node(out, {hidden, lm_head_weight, labels},
                                                   std::make_shared<SelectedTokenLMCrossEntropyBackwardHip>(s));
    }
    return out;
}

TensorPtr streaming_lm_cross_entropy(const TensorPtr& hidden, const TensorPtr& lm_head_weight,
                                    const TensorPtr& labels, int ignore_index, const std::string& reduction) {
    return selected_token_lm_cross_entropy(hidden, lm_head_weight, labels, ignore_index, reduction);
}

}  // namespace ops
