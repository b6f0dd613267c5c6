// finetune_ops adapter: ops::LoRALinear on the MI355X kernels.
//
// Drop-in replacement for operator/finetune_ops/nn/lora_linear.cpp (the
// reference's translation unit of nn/lora_linear.h), compiled against the
// reference's own headers and linked to libmft_attn.so through the C ABI of
// include/mft/lora.h.  Behaviour versus the reference:
//
//   * Same class and members (nn/lora_linear.h:36-95).  Shape inference of A
//     and B (either orientation, nn/lora_linear.cpp:52-88), W as [in, out] or
//     [out, in] (the matmul's on-the-fly transpose, core/ops.cpp:649-654) and
//     the error messages are the reference's.
//   * forward runs mft_lora_fwd and, when x or a slice's A / B needs a
//     gradient, registers ONE autograd node (y, {x, A0, B0, A1, B1, ...})
//     whose apply runs mft_lora_bwd.  As in the reference, a slice over a
//     column range adds to y but gets no gradient and adds nothing to dx
//     (nn/lora_linear.cpp:417-434); W and b are frozen.
//   * merge_to_base bakes scale * A . B into W with mft_lora_merge (the
//     double-sum, fp32-add, bf16-rounding arithmetic of
//     apply_lora_delta_to_base) after keeping a byte copy of W, which
//     unmerge_from_base restores, as the reference does.
//   * Tensors are the reference's host tensors: inputs are copied to the GPU,
//     results back (PCIe-inclusive).  Device-resident callers use the C ABI.
#include "lora_linear.h"

#include <algorithm>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include <hip/hip_runtime.h>

#include "../core/autograd_engine.h"
#include "../core/backward_functions.h"
#include "../core/ops.h"
#include "mft/lora.h"
#include "dropin_device.h"

namespace ops {
namespace {

constexpr const char* kWho = "LoRALinear";
void hip_check(hipError_t e, const char* what) { dropin::hip_check(kWho, e, what); }
void mft_check(mft_status st) { dropin::mft_check(kWho, st); }
hipStream_t lora_stream() { return dropin::stream(); }
using dropin::DeviceBuffer;
using dropin::download_f32;
using dropin::upload_bytes;

// Any floating-point host tensor as fp32 values on the device (the C ABI's
// A, B, x and bias are fp32; the reference reads them through
// read_tensor_float, nn/lora_linear.cpp:19-31).
std::unique_ptr<DeviceBuffer> upload_f32(const TensorPtr& t) { return dropin::upload_f32(t, kWho); }

int32_t w_dtype(const TensorPtr& W) {
    if (W->dtype() == kFloat32) return MFT_F32;
    if (W->dtype() == kBFloat16) return MFT_BF16;
    throw std::runtime_error("matmul: unsupported right operand dtype " + DTypeUtils::to_string(W->dtype()));
}

// A as [in, rank] (or transposed) and B as [rank, out] (or transposed), the
// rules of infer_effective_lora_shape.
struct SliceShape {
    int64_t rank = 0, out = 0;
    bool a_t = false, b_t = false;
};
SliceShape infer(const TensorPtr& A, const TensorPtr& B, int64_t in_dim) {
    if (!A || !B || A->ndim() != 2 || B->ndim() != 2)
        throw std::runtime_error("LoRALinear: LoRA A/B must be 2D tensors");
    SliceShape s;
    if (A->shape()[0] == in_dim) s.rank = A->shape()[1];
    else if (A->shape()[1] == in_dim) s.rank = A->shape()[0], s.a_t = true;
    else throw std::runtime_error("LoRALinear: LoRA A shape is incompatible with input dimension");
    if (B->shape()[0] == s.rank) s.out = B->shape()[1];
    else if (B->shape()[1] == s.rank) s.out = B->shape()[0], s.b_t = true;
    else throw std::runtime_error("LoRALinear: LoRA B shape is incompatible with rank");
    return s;
}

size_t tensor_bytes(const TensorPtr& t) { return static_cast<size_t>(t->numel()) * DTypeUtils::size_of(t->dtype()); }

// What the kernels hold between forward and backward.
struct Saved {
    int64_t N = 0, in = 0, out = 0;
    int32_t wdt = MFT_F32, w_t = 0;
    std::vector<int64_t> x_shape, y_shape;
    std::vector<std::vector<int64_t>> a_shape, b_shape;
    std::vector<SliceShape> shape;
    std::vector<float> scale;
    std::vector<int64_t> col0;
    std::vector<bool> x_a_b_grad;  // x, then A_i, B_i need a gradient
    std::unique_ptr<DeviceBuffer> x, W, u;
    std::vector<std::unique_ptr<DeviceBuffer>> A, B;
};

class LoRALinearBackwardHip : public BackwardFunction {
public:
    explicit LoRALinearBackwardHip(std::shared_ptr<Saved> s) : s_(std::move(s)) {}

    // grad_output: fp32 shaped like y.  Returns {dx, dA0, dB0, ...}; nullptr
    // where the input needs no gradient or the slice gets none.
    std::vector<TensorPtr> apply(const TensorPtr& grad_output) override {
        if (!s_) throw std::runtime_error("LoRALinearBackwardHip: applied twice");
        if (!grad_output || grad_output->shape() != s_->y_shape || grad_output->dtype() != kFloat32)
            throw std::runtime_error("LoRADeltaBackward: grad_output must be fp32 shaped like the output");
        const size_t n = s_->shape.size();
        std::vector<mft_lora_slice> sl(n);
        std::vector<std::unique_ptr<DeviceBuffer>> gA(n), gB(n);
        for (size_t i = 0; i < n; ++i) {
            const SliceShape& sh = s_->shape[i];
            const bool full = s_->col0[i] == 0 && sh.out == s_->out;
            sl[i] = mft_lora_slice{};
            sl[i].A = s_->A[i]->f();
            sl[i].B = s_->B[i]->f();
            sl[i].scale = s_->scale[i];
            sl[i].a_transposed = sh.a_t;
            sl[i].b_transposed = sh.b_t;
            sl[i].rank = sh.rank;
            sl[i].col0 = s_->col0[i];
            sl[i].cols = sh.out;
            if (full && s_->x_a_b_grad[1 + 2 * i]) {
                gA[i] = std::make_unique<DeviceBuffer>(static_cast<size_t>(sh.rank * s_->in) * 4);
                sl[i].grad_A = gA[i]->f();
            }
            if (full && s_->x_a_b_grad[2 + 2 * i]) {
                gB[i] = std::make_unique<DeviceBuffer>(static_cast<size_t>(sh.rank * sh.out) * 4);
                sl[i].grad_B = gB[i]->f();
            }
        }
        mft_lora_desc d{};
        d.N = s_->N;
        d.in_dim = s_->in;
        d.out_dim = s_->out;
        d.w_dtype = s_->wdt;
        d.w_transposed = s_->w_t;
        d.n_slices = static_cast<int32_t>(n);
        d.slices = sl.data();
        size_t fws = 0, bws = 0;
        mft_check(mft_lora_workspace_size(&d, &fws, &bws));
        hipStream_t st = lora_stream();
        auto dy = upload_bytes(grad_output->data<float>(), tensor_bytes(grad_output));
        DeviceBuffer ws(bws);
        std::unique_ptr<DeviceBuffer> dx;
        if (s_->x_a_b_grad[0]) dx = std::make_unique<DeviceBuffer>(static_cast<size_t>(s_->N * s_->in) * 4);
        mft_check(mft_lora_bwd(&d, s_->x->f(), s_->W->get(), dy->f(), s_->u->f(), dx ? dx->f() : nullptr, ws.get(),
                               st));
        std::vector<TensorPtr> grads;
        grads.push_back(dx ? download_f32(*dx, s_->x_shape) : nullptr);
        for (size_t i = 0; i < n; ++i) {
            grads.push_back(gA[i] ? download_f32(*gA[i], s_->a_shape[i]) : nullptr);
            grads.push_back(gB[i] ? download_f32(*gB[i], s_->b_shape[i]) : nullptr);
        }
        hip_check(hipStreamSynchronize(st), "synchronize");
        s_.reset();  // the graph is single-use (Engine::clear_graph, core/autograd_engine.cpp:275-287)
        return grads;
    }

private:
    std::shared_ptr<Saved> s_;
};

// W[in, out] += sign * scale * A . B over every slice, on the device, in W's
// own storage type.
void merge_on_device(const TensorPtr& W, const std::vector<LoRASlice>& slices, float sign) {
    if (!DTypeUtils::is_floating_point(W->dtype()))
        throw std::runtime_error("LoRALinear: merge requires floating-point base weights");
    if (W->ndim() != 2) throw std::runtime_error("LoRALinear: merge requires a 2D base weight");
    const int64_t in_dim = W->shape()[0], out_dim = W->shape()[1];
    std::vector<mft_lora_slice> sl;
    std::vector<std::unique_ptr<DeviceBuffer>> keep;
    for (const auto& s : slices) {
        const SliceShape sh = infer(s.A, s.B, in_dim);
        const int64_t cols = s.cols > 0 ? s.cols : sh.out;
        if (cols != sh.out) throw std::runtime_error("LoRALinear: LoRA slice cols do not match B output dimension");
        if (s.col0 < 0 || s.col0 + sh.out > out_dim)
            throw std::runtime_error("LoRALinear: LoRA slice range exceeds base weight width");
        keep.push_back(upload_f32(s.A));
        const float* A = keep.back()->f();
        keep.push_back(upload_f32(s.B));
        mft_lora_slice m{};
        m.A = A;
        m.B = keep.back()->f();
        m.scale = s.scale;
        m.a_transposed = sh.a_t;
        m.b_transposed = sh.b_t;
        m.rank = sh.rank;
        m.col0 = s.col0;
        m.cols = sh.out;
        sl.push_back(m);
    }
    mft_lora_desc d{};
    d.N = 1;
    d.in_dim = in_dim;
    d.out_dim = out_dim;
    d.w_dtype = w_dtype(W);
    d.n_slices = static_cast<int32_t>(sl.size());
    d.slices = sl.data();
    auto w = upload_bytes(W->data_ptr(), tensor_bytes(W));
    mft_check(mft_lora_merge(&d, w->get(), sign, lora_stream()));
    hip_check(hipMemcpyAsync(W->data_ptr(), w->get(), tensor_bytes(W), hipMemcpyDeviceToHost, lora_stream()),
              "copy to host");
    hip_check(hipStreamSynchronize(lora_stream()), "synchronize");
}

}  // namespace

void LoRALinear::attach_lora(const TensorPtr& A, const TensorPtr& B, float scale, int col0, int cols) {
    if (!A || !B) throw std::runtime_error("LoRALinear::attach_lora: A and B must not be null");
    if (A->ndim() != 2 || B->ndim() != 2) throw std::runtime_error("LoRALinear::attach_lora: A and B must be 2D");
    int64_t out_cols = cols;
    if (out_cols <= 0) out_cols = infer(A, B, W_->shape().empty() ? A->shape()[0] : W_->shape()[0]).out;
    A->set_requires_grad(true);
    B->set_requires_grad(true);
    slices_.emplace_back(A, B, scale, col0, static_cast<int>(out_cols));
}

void LoRALinear::clear_lora() {
    if (merged_) unmerge_from_base();
    slices_.clear();
    merged_ = false;
    merge_backup_.clear();
}

std::vector<std::pair<std::string, TensorPtr>> LoRALinear::debug_params() const {
    // the names the PEFT export expects (graph/lora_saver.cpp reads them)
    std::vector<std::pair<std::string, TensorPtr>> out;
    for (size_t i = 0; i < slices_.size(); ++i) {
        const std::string base = debug_name_.empty() ? "lora_" + std::to_string(i) : debug_name_;
        out.emplace_back(base + "_lora_A_default_weight", slices_[i].A);
        out.emplace_back(base + "_lora_B_default_weight", slices_[i].B);
    }
    return out;
}

TensorPtr LoRALinear::forward(const TensorPtr& x) const {
    if (!x || x->ndim() != 3) throw std::runtime_error("LoRALinear: x must be [B, S, in]");
    if (x->dtype() != kFloat32)
        throw TensorError("matmul: left operand must be float32 for mixed-precision CPU kernels");
    if (!W_ || W_->ndim() != 2) throw TensorError("matmul requires tensors with at least 2 dimensions");
    const int64_t in = x->shape()[2];
    const int64_t w0 = W_->shape()[0], w1 = W_->shape()[1];
    int32_t w_t = 0;
    if (w0 != in) {
        if (w1 != in) throw TensorError("matmul dimension mismatch");
        w_t = 1;
    }
    const int64_t out = w_t ? w0 : w1;
    auto s = std::make_shared<Saved>();
    s->N = x->shape()[0] * x->shape()[1];
    s->in = in;
    s->out = out;
    s->wdt = w_dtype(W_);
    s->w_t = w_t;
    s->x_shape = x->shape();
    s->y_shape = {x->shape()[0], x->shape()[1], out};
    s->x_a_b_grad.push_back(x->requires_grad());
    std::vector<mft_lora_slice> sl;
    int64_t R = 0;
    if (!merged_) {
        for (const auto& slice : slices_) {
            if (!slice.A->requires_grad()) const_cast<Tensor*>(slice.A.get())->set_requires_grad(true);
            if (!slice.B->requires_grad()) const_cast<Tensor*>(slice.B.get())->set_requires_grad(true);
            const SliceShape sh = infer(slice.A, slice.B, in);
            if (slice.col0 < 0 || slice.col0 + sh.out > out)
                throw std::runtime_error("LoRALinear: LoRA slice range exceeds base weight width");
            s->shape.push_back(sh);
            s->scale.push_back(slice.scale);
            s->col0.push_back(slice.col0);
            s->a_shape.push_back(slice.A->shape());
            s->b_shape.push_back(slice.B->shape());
            s->x_a_b_grad.push_back(slice.A->requires_grad());
            s->x_a_b_grad.push_back(slice.B->requires_grad());
            s->A.push_back(upload_f32(slice.A));
            s->B.push_back(upload_f32(slice.B));
            mft_lora_slice m{};
            m.A = s->A.back()->f();
            m.B = s->B.back()->f();
            m.scale = slice.scale;
            m.a_transposed = sh.a_t;
            m.b_transposed = sh.b_t;
            m.rank = sh.rank;
            m.col0 = slice.col0;
            m.cols = sh.out;
            sl.push_back(m);
            R += sh.rank;
        }
    }
    mft_lora_desc d{};
    d.N = s->N;
    d.in_dim = in;
    d.out_dim = out;
    d.w_dtype = s->wdt;
    d.w_transposed = w_t;
    d.n_slices = static_cast<int32_t>(sl.size());
    d.slices = sl.data();
    size_t fws = 0, bws = 0;
    mft_check(mft_lora_workspace_size(&d, &fws, &bws));
    s->x = upload_bytes(x->data<float>(), tensor_bytes(x));
    s->W = upload_bytes(W_->data_ptr(), tensor_bytes(W_));
    std::unique_ptr<DeviceBuffer> bias;
    if (b_) bias = upload_f32(b_);
    s->u = std::make_unique<DeviceBuffer>(static_cast<size_t>(s->N * std::max<int64_t>(R, 1)) * 4);
    DeviceBuffer y(static_cast<size_t>(s->N * out) * 4), ws(fws);
    mft_check(mft_lora_fwd(&d, s->x->f(), s->W->get(), bias ? bias->f() : nullptr, y.f(), s->u->f(), ws.get(),
                           lora_stream()));
    auto result = download_f32(y, s->y_shape);
    hip_check(hipStreamSynchronize(lora_stream()), "synchronize");

    const bool any_grad = std::any_of(s->x_a_b_grad.begin(), s->x_a_b_grad.end(), [](bool g) { return g; });
    if (any_grad) {
        std::vector<TensorPtr> inputs{x};
        for (const auto& slice : (merged_ ? std::vector<LoRASlice>{} : slices_)) {
            inputs.push_back(slice.A);
            inputs.push_back(slice.B);
        }
        result->set_requires_grad(true);
        autograd::Engine::instance().register_node(result, inputs, std::make_shared<LoRALinearBackwardHip>(s));
    }
    return result;
}

void LoRALinear::merge_to_base() {
    if (merged_ || slices_.empty()) return;
    const size_t n = tensor_bytes(W_);
    merge_backup_.resize(n);
    if (n) std::memcpy(merge_backup_.data(), W_->data_ptr(), n);
    merge_on_device(W_, slices_, +1.0f);
    merged_ = true;
}

void LoRALinear::unmerge_from_base() {
    if (!merged_ || slices_.empty()) return;
    const size_t n = tensor_bytes(W_);
    if (!merge_backup_.empty()) {
        if (merge_backup_.size() != n)
            throw std::runtime_error("LoRALinear::unmerge_from_base: merge backup size mismatch");
        if (n) std::memcpy(W_->data_ptr(), merge_backup_.data(), n);
        merge_backup_.clear();
        merged_ = false;
        return;
    }
    merge_on_device(W_, slices_, -1.0f);
    merged_ = false;
}

std::vector<TensorPtr> LoRALinear::trainable_parameters() const {
    std::vector<TensorPtr> params;
    for (const auto& s : slices_) {
        params.push_back(s.A);
        params.push_back(s.B);
    }
    return params;
}

}  // namespace ops
