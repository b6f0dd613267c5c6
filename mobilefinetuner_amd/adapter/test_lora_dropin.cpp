// Parity of the drop-in ops::LoRALinear (MI355X kernels) against the layer
// built from the reference's own operators, through the unchanged
// finetune_ops API.
//
// Reference side: y = matmul(x, W) (+ add(b)) + mul(matmul(matmul(x2d, A_eff),
// B_eff), scale), the graph nn/lora_linear.cpp:384-434 builds for a slice over
// all columns, backward by autograd::Engine::run_backward.  A slice over a
// column range is added to y in place there and gets no gradient; the drop-in
// must leave its A / B gradients empty as well.
//
// Bars: fp32 W max-rel 1e-4 (y, dx, dA, dB); bf16 W 2e-2 for y and dx (the
// products with W run on the bf16 MFMA path), 1e-4 for dA and dB (fp32).
#include <cmath>
#include <cstdint>
#include <iostream>
#include <string>
#include <vector>

#include "autograd_engine.h"
#include "lora_linear.h"
#include "ops.h"

using namespace ops;

namespace {

float max_rel(const TensorPtr& a, const TensorPtr& b) {
    const float* pa = a->data<float>();
    const float* pb = b->data<float>();
    double num = 0.0, den = 0.0;
    for (int64_t i = 0; i < a->numel(); ++i) {
        num = std::max(num, std::fabs(double(pa[i]) - double(pb[i])));
        den = std::max(den, std::fabs(double(pb[i])));
    }
    return den > 0 ? float(num / den) : float(num);
}

uint64_t splitmix(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// Seeded uniform values in [-a, a).
TensorPtr rnd(const std::vector<int64_t>& shape, uint64_t seed, float a) {
    auto t = zeros(shape, kFloat32, kCPU);
    for (int64_t i = 0; i < t->numel(); ++i)
        t->data<float>()[i] = float(a * (2.0 * ((splitmix(seed * 7919 + i) >> 11) * (1.0 / 9007199254740992.0)) - 1.0));
    return t;
}

TensorPtr clone(const TensorPtr& t, bool grad) {
    auto c = zeros(t->shape(), kFloat32, kCPU);
    std::copy(t->data<float>(), t->data<float>() + t->numel(), c->data<float>());
    c->set_requires_grad(grad);
    return c;
}

TensorPtr to_bf16(const TensorPtr& t) {
    auto c = std::make_shared<Tensor>(t->shape(), kBFloat16, kCPU);
    for (int64_t i = 0; i < t->numel(); ++i) c->data<uint16_t>()[i] = float32_to_bf16_bits(t->data<float>()[i]);
    return c;
}

TensorPtr round_bf16(const TensorPtr& t) {
    auto c = zeros(t->shape(), kFloat32, kCPU);
    for (int64_t i = 0; i < t->numel(); ++i)
        c->data<float>()[i] = bf16_bits_to_float32(float32_to_bf16_bits(t->data<float>()[i]));
    return c;
}

int failures = 0;
void check(const std::string& what, float err, float tol) {
    std::cout << "  " << what << " max-rel " << err << (err <= tol ? "" : "  FAIL") << std::endl;
    if (!(err <= tol)) ++failures;
}

// One full-width slice: drop-in vs the reference operators' graph.
void full_slice(bool w_bf16, bool injector_layout) {
    std::cout << "[case] full slice, W " << (w_bf16 ? "bf16 [out, in]" : "fp32 [in, out]")
              << (injector_layout ? ", A [r, in], B [out, r]" : ", A [in, r], B [r, out]") << std::endl;
    const int64_t B = 2, S = 10, IN = 64, OUT = 48, R = 8;
    const float scale = 2.0f;
    auto x = rnd({B, S, IN}, 1, 1.0f);
    auto W = rnd(w_bf16 ? std::vector<int64_t>{OUT, IN} : std::vector<int64_t>{IN, OUT}, 2, 0.2f);
    if (w_bf16) W = round_bf16(W);
    auto bias = rnd({OUT}, 3, 0.5f);
    auto A = rnd(injector_layout ? std::vector<int64_t>{R, IN} : std::vector<int64_t>{IN, R}, 4, 0.3f);
    auto Bm = rnd(injector_layout ? std::vector<int64_t>{OUT, R} : std::vector<int64_t>{R, OUT}, 5, 0.3f);
    auto dy = rnd({B, S, OUT}, 6, 1.0f);

    // reference operators
    auto xr = clone(x, true), Ar = clone(A, true), Br = clone(Bm, true);
    auto Wr = clone(W, false);
    auto Weff = w_bf16 ? transpose(Wr, 0, 1) : Wr;
    auto Aeff = injector_layout ? transpose(Ar, 0, 1) : Ar;
    auto Beff = injector_layout ? transpose(Br, 0, 1) : Br;
    auto yr = add(matmul(xr, Weff), clone(bias, false));
    auto x2d = reshape(xr, {B * S, IN});
    auto delta = reshape(mul(matmul(matmul(x2d, Aeff), Beff), scale), {B, S, OUT});
    yr = add(yr, delta);
    autograd::Engine::instance().run_backward({yr}, {clone(dy, false)});
    auto gx_r = xr->grad(), gA_r = Ar->grad(), gB_r = Br->grad();
    autograd::Engine::instance().clear_graph();

    // drop-in
    auto xd = clone(x, true), Ad = clone(A, false), Bd = clone(Bm, false);
    LoRALinear layer(w_bf16 ? to_bf16(W) : clone(W, false), clone(bias, false));
    // explicit columns, as the injectors attach (graph/gemma_lora_injector.cpp:151); with
    // cols = -1 attach_lora infers them from W's first dimension, which a [out, in] W defeats
    layer.attach_lora(Ad, Bd, scale, 0, static_cast<int>(OUT));
    auto yd = layer.forward(xd);
    autograd::Engine::instance().run_backward({yd}, {clone(dy, false)});
    const float tw = w_bf16 ? 2e-2f : 1e-4f;
    check("y", max_rel(yd, yr), tw);
    check("dx", max_rel(xd->grad(), gx_r), tw);
    check("dA", max_rel(Ad->grad(), gA_r), 1e-4f);
    check("dB", max_rel(Bd->grad(), gB_r), 1e-4f);
    autograd::Engine::instance().clear_graph();
}

// A slice over columns [16, 32): y gets the delta there, A / B get no gradient.
void column_slice() {
    std::cout << "[case] column slice (fp32)" << std::endl;
    const int64_t B = 1, S = 7, IN = 40, OUT = 48, R = 4, C0 = 16, C = 16;
    const float scale = 0.5f;
    auto x = rnd({B, S, IN}, 11, 1.0f);
    auto W = rnd({IN, OUT}, 12, 0.2f);
    auto A = rnd({IN, R}, 13, 0.3f), Bm = rnd({R, C}, 14, 0.3f);
    auto yr = matmul(clone(x, false), clone(W, false));
    auto d = mul(matmul(matmul(reshape(clone(x, false), {B * S, IN}), clone(A, false)), clone(Bm, false)), scale);
    float* py = yr->data<float>();
    for (int64_t t = 0; t < B * S; ++t)
        for (int64_t c = 0; c < C; ++c) py[t * OUT + C0 + c] += d->data<float>()[t * C + c];
    auto xd = clone(x, true), Ad = clone(A, false), Bd = clone(Bm, false);
    LoRALinear layer(clone(W, false));
    layer.attach_lora(Ad, Bd, scale, static_cast<int>(C0), static_cast<int>(C));
    auto yd = layer.forward(xd);
    check("y", max_rel(yd, yr), 1e-4f);
    autograd::Engine::instance().run_backward({yd}, {rnd({B, S, OUT}, 15, 1.0f)});
    const bool none = !Ad->grad() && !Bd->grad();
    std::cout << "  A/B gradients empty: " << (none ? "yes" : "no  FAIL") << std::endl;
    if (!none) ++failures;
    autograd::Engine::instance().clear_graph();
}

}  // namespace

int main() {
    try {
        full_slice(false, false);
        full_slice(true, true);
        column_slice();
    } catch (const std::exception& e) {
        std::cout << "exception: " << e.what() << std::endl;
        return 1;
    }
    std::cout << (failures ? "[FAIL]" : "[PASS]") << " LoRALinear drop-in parity" << std::endl;
    return failures ? 1 : 0;
}
