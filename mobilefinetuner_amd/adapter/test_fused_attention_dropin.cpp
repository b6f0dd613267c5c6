// Parity of the drop-in ops::memory_efficient_attention (MI355X kernels)
// against the reference's own composite, through the unchanged finetune_ops
// API, in the style of core/test_memory_efficient_attention_grad.cpp.
//
// Reference side: repeat_kv_heads -> transpose -> matmul -> mul(scale) ->
// add(create_causal_mask) -> softmax -> matmul, backward by
// autograd::Engine::run_backward (the composite of
// core/memory_efficient_attention.cpp:23-43 and graph/gemma_model.cpp:481-505).
// Fused side: memory_efficient_attention(q, k_unrepeated, v_unrepeated, mask).
//
// Bar: max_i |x - ref| / max_i |ref| <= 1e-4 (fp32 inputs) and <= 2e-2 (bf16
// inputs vs the fp32 composite on the same bf16-rounded values), for O, dQ,
// dK, dV.
#include <cmath>
#include <cstdint>
#include <functional>
#include <iostream>
#include <stdexcept>
#include <string>
#include <vector>

#include "autograd_engine.h"
#include "fused_attention.h"
#include "memory_efficient_attention.h"
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

// Seeded N(0,1) values (splitmix64 + Box-Muller), rounded to bf16 when asked
// so that the fp32 composite sees exactly what the bf16 kernels see.
uint64_t splitmix(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

void fill_normal(const TensorPtr& t, uint64_t seed, float sigma, bool bf16_round) {
    float* p = t->data<float>();
    for (int64_t i = 0; i < t->numel(); i += 2) {
        const double u1 = ((splitmix(seed * 1315423911ull + i) >> 11) + 1.0) * (1.0 / 9007199254740993.0);
        const double u2 = (splitmix(seed * 2654435761ull + i + 1) >> 11) * (1.0 / 9007199254740992.0);
        const double r = std::sqrt(-2.0 * std::log(u1));
        p[i] = float(sigma * r * std::cos(6.283185307179586 * u2));
        if (i + 1 < t->numel()) p[i + 1] = float(sigma * r * std::sin(6.283185307179586 * u2));
    }
    if (bf16_round)
        for (int64_t i = 0; i < t->numel(); ++i) p[i] = bf16_bits_to_float32(float32_to_bf16_bits(p[i]));
}

TensorPtr make(const std::vector<int64_t>& shape, uint64_t seed, float sigma, bool bf16_round, bool grad) {
    auto t = zeros(shape, kFloat32, kCPU);
    fill_normal(t, seed, sigma, bf16_round);
    t->set_requires_grad(grad);
    return t;
}

TensorPtr to_bf16(const TensorPtr& t, bool grad) {
    auto out = zeros(t->shape(), kBFloat16, kCPU);
    const float* s = t->data<float>();
    uint16_t* d = out->data<uint16_t>();
    for (int64_t i = 0; i < t->numel(); ++i) d[i] = float32_to_bf16_bits(s[i]);
    out->set_requires_grad(grad);
    return out;
}

TensorPtr copy_of(const TensorPtr& t, bool grad) {
    auto out = t->clone();
    out->set_requires_grad(grad);
    return out;
}

struct Result {
    float o, dq, dk, dv;
};

// One case: B, Hq, Hkv, S, D, scale, causal, bf16 inputs.
Result run_case(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D, float scale, bool causal, bool bf16,
                uint64_t seed) {
    const int r = int(Hq / Hkv);
    auto q0 = make({B, Hq, S, D}, seed, 1.0f, bf16, false);
    auto k0 = make({B, Hkv, S, D}, seed + 1, 1.0f, bf16, false);
    auto v0 = make({B, Hkv, S, D}, seed + 2, 1.0f, bf16, false);
    auto g = make({B, Hq, S, D}, seed + 3, 0.1f, bf16, false);

    // Reference composite (fp32) with explicit GQA repeat.
    auto qr = copy_of(q0, true), kr = copy_of(k0, true), vr = copy_of(v0, true);
    auto kk = r > 1 ? repeat_kv_heads(kr, r) : kr;
    auto vv = r > 1 ? repeat_kv_heads(vr, r) : vr;
    auto scores = mul(matmul(qr, transpose(kk, 2, 3)), scale);
    if (causal) scores = add(scores, create_causal_mask(int(S), kFloat32, kCPU));
    auto out_ref = matmul(softmax(scores, -1), vv);
    autograd::Engine::instance().run_backward({out_ref}, {g});

    // Fused drop-in with un-repeated K/V.
    auto qf = bf16 ? to_bf16(q0, true) : copy_of(q0, true);
    auto kf = bf16 ? to_bf16(k0, true) : copy_of(k0, true);
    auto vf = bf16 ? to_bf16(v0, true) : copy_of(v0, true);
    MemoryEfficientAttentionConfig cfg;
    cfg.use_causal_mask = causal;
    cfg.scale = scale;
    auto out = memory_efficient_attention(qf, kf, vf, causal ? create_causal_mask(int(S), kFloat32, kCPU) : nullptr,
                                          cfg);
    autograd::Engine::instance().run_backward({out}, {g});
    if (!qf->grad() || !kf->grad() || !vf->grad()) throw std::runtime_error("missing fused grads");
    return {max_rel(out, out_ref), max_rel(qf->grad(), qr->grad()), max_rel(kf->grad(), kr->grad()),
            max_rel(vf->grad(), vr->grad())};
}

// Gemma's build_sliding_mask (graph/gemma_model.cpp:272-285): j <= i and
// i - j < window, else kMaskValue (-1e10).
TensorPtr sliding_mask(int64_t S, int64_t window) {
    auto m = zeros({S, S}, kFloat32, kCPU);
    float* p = m->data<float>();
    for (int64_t i = 0; i < S; ++i)
        for (int64_t j = 0; j < S; ++j)
            if (!(j <= i && i - j < window)) p[i * S + j] = -1e10f;
    return m;
}

// The [B,1,1,S] padding mask of a right-padded attention_mask
// (graph/gemma_model.cpp:287-320 with value -1e10; graph/qwen_model.cpp:338-353
// with -1e9).
TensorPtr pad_mask(int64_t B, int64_t S, const std::vector<int>& lengths, float value) {
    auto m = zeros({B, 1, 1, S}, kFloat32, kCPU);
    float* p = m->data<float>();
    for (int64_t b = 0; b < B; ++b)
        for (int64_t j = lengths[size_t(b)]; j < S; ++j) p[b * S + j] = value;
    return m;
}

// The model graphs' composite (graph/gemma_model.cpp:481-505: repeat_kv_heads,
// scores + base_mask, then + pad_mask) against memory_efficient_attention_masked
// (or, without padding, memory_efficient_attention with the base mask).
Result run_masked_case(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D, int64_t window,
                       const std::vector<int>& lengths, float pad_value, bool bf16, uint64_t seed) {
    const int r = int(Hq / Hkv);
    auto q0 = make({B, Hq, S, D}, seed, 1.0f, bf16, false);
    auto k0 = make({B, Hkv, S, D}, seed + 1, 1.0f, bf16, false);
    auto v0 = make({B, Hkv, S, D}, seed + 2, 1.0f, bf16, false);
    auto g = make({B, Hq, S, D}, seed + 3, 0.1f, bf16, false);
    auto base = window > 0 ? sliding_mask(S, window) : create_causal_mask(int(S), kFloat32, kCPU);
    auto pad = lengths.empty() ? nullptr : pad_mask(B, S, lengths, pad_value);
    const float scale = 1.0f / std::sqrt(float(D));

    auto qr = copy_of(q0, true), kr = copy_of(k0, true), vr = copy_of(v0, true);
    auto kk = r > 1 ? repeat_kv_heads(kr, r) : kr;
    auto vv = r > 1 ? repeat_kv_heads(vr, r) : vr;
    auto scores = add(mul(matmul(qr, transpose(kk, 2, 3)), scale), base);
    if (pad) scores = add(scores, pad);
    auto out_ref = matmul(softmax(scores, -1), vv);
    autograd::Engine::instance().run_backward({out_ref}, {g});

    auto qf = bf16 ? to_bf16(q0, true) : copy_of(q0, true);
    auto kf = bf16 ? to_bf16(k0, true) : copy_of(k0, true);
    auto vf = bf16 ? to_bf16(v0, true) : copy_of(v0, true);
    MemoryEfficientAttentionConfig cfg;
    cfg.scale = scale;
    auto out = pad ? memory_efficient_attention_masked(qf, kf, vf, base, pad, cfg)
                   : memory_efficient_attention(qf, kf, vf, base, cfg);
    autograd::Engine::instance().run_backward({out}, {g});
    if (!qf->grad() || !kf->grad() || !vf->grad()) throw std::runtime_error("missing fused grads");
    return {max_rel(out, out_ref), max_rel(qf->grad(), qr->grad()), max_rel(kf->grad(), kr->grad()),
            max_rel(vf->grad(), vr->grad())};
}

// Any additive masks (the kernels' mask mode): the composite adds base, then
// pad (core/memory_efficient_attention.cpp:29-38 with ops::add's broadcast)
// against memory_efficient_attention(q, k, v, base) (pad null) or
// memory_efficient_attention_masked(q, k, v, base, pad).
Result run_any_mask_case(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D, const TensorPtr& base,
                         const TensorPtr& pad, bool bf16, uint64_t seed) {
    const int r = int(Hq / Hkv);
    auto q0 = make({B, Hq, S, D}, seed, 1.0f, bf16, false);
    auto k0 = make({B, Hkv, S, D}, seed + 1, 1.0f, bf16, false);
    auto v0 = make({B, Hkv, S, D}, seed + 2, 1.0f, bf16, false);
    auto g = make({B, Hq, S, D}, seed + 3, 0.1f, bf16, false);
    const float scale = 1.0f / std::sqrt(float(D));
    auto qr = copy_of(q0, true), kr = copy_of(k0, true), vr = copy_of(v0, true);
    auto kk = r > 1 ? repeat_kv_heads(kr, r) : kr;
    auto vv = r > 1 ? repeat_kv_heads(vr, r) : vr;
    auto scores = mul(matmul(qr, transpose(kk, 2, 3)), scale);
    if (base) scores = add(scores, base);
    if (pad) scores = add(scores, pad);
    auto out_ref = matmul(softmax(scores, -1), vv);
    autograd::Engine::instance().run_backward({out_ref}, {g});

    auto qf = bf16 ? to_bf16(q0, true) : copy_of(q0, true);
    auto kf = bf16 ? to_bf16(k0, true) : copy_of(k0, true);
    auto vf = bf16 ? to_bf16(v0, true) : copy_of(v0, true);
    MemoryEfficientAttentionConfig cfg;
    cfg.scale = scale;
    auto out = pad ? memory_efficient_attention_masked(qf, kf, vf, base, pad, cfg)
                   : memory_efficient_attention(qf, kf, vf, base, cfg);
    autograd::Engine::instance().run_backward({out}, {g});
    if (!qf->grad() || !kf->grad() || !vf->grad()) throw std::runtime_error("missing fused grads");
    return {max_rel(out, out_ref), max_rel(qf->grad(), qr->grad()), max_rel(kf->grad(), kr->grad()),
            max_rel(vf->grad(), vr->grad())};
}

// No grad with an [S,S] mask: the operator's rule (.cpp:160-172), -1e10
// above the diagonal when use_causal_mask, then + mask, against the same
// scores through the composite's ops (the operator's double row sum differs
// from the composite's float sum by rounding only).
float run_nograd_mask_case(int64_t B, int64_t H, int64_t S, int64_t D, const TensorPtr& mask, bool causal,
                           uint64_t seed) {
    auto q = make({B, H, S, D}, seed, 1.0f, false, false);
    auto k = make({B, H, S, D}, seed + 1, 1.0f, false, false);
    auto v = make({B, H, S, D}, seed + 2, 1.0f, false, false);
    const float scale = 1.0f / std::sqrt(float(D));
    auto scores = mul(matmul(q, transpose(k, 2, 3)), scale);
    if (causal) {
        float* p = scores->data<float>();
        for (int64_t bh = 0; bh < B * H; ++bh)
            for (int64_t i = 0; i < S; ++i)
                for (int64_t j = i + 1; j < S; ++j) p[(bh * S + i) * S + j] = -1e10f;
    }
    auto ref = matmul(softmax(add(scores, mask), -1), v);
    MemoryEfficientAttentionConfig cfg;
    cfg.use_causal_mask = causal;
    cfg.scale = scale;
    auto out = memory_efficient_attention(q, k, v, mask, cfg);
    return max_rel(out, ref);
}

TensorPtr random_mask(const std::vector<int64_t>& shape, uint64_t seed, float hole_every) {
    auto m = make(shape, seed, 1.0f, false, false);
    float* p = m->data<float>();
    for (int64_t i = 0; i < m->numel(); ++i)
        if (std::fmod(float(i) * 0.618034f, 1.0f) < hole_every) p[i] = -1e10f;
    return m;
}

bool expect_throw(const char* what, const std::function<void()>& fn) {
    try {
        fn();
    } catch (const std::exception& e) {
        std::cout << "[dropin] " << what << " -> throws: " << e.what() << std::endl;
        return true;
    }
    std::cout << "[dropin] " << what << " -> did NOT throw" << std::endl;
    return false;
}

}  // namespace

int main() {
    struct Case {
        int64_t B, Hq, Hkv, S, D;
        bool causal, bf16;
    };
    const Case cases[] = {
        {1, 2, 2, 4, 3, true, false},      // the reference unit test's shape
        {2, 4, 4, 37, 64, true, false},    // MHA, ragged S
        {1, 4, 1, 70, 256, true, false},   // Gemma-shaped group of 4
        {1, 14, 2, 33, 64, true, false},   // Qwen-shaped group of 7
        {1, 4, 2, 50, 128, false, false},  // no mask
        {1, 4, 1, 96, 256, true, true},    // bf16 inputs
        {2, 6, 3, 65, 64, true, true},
    };
    bool ok = true;
    uint64_t seed = 4242;
    for (const Case& c : cases) {
        const float scale = 1.0f / std::sqrt(float(c.D));
        const Result r = run_case(c.B, c.Hq, c.Hkv, c.S, c.D, scale, c.causal, c.bf16, seed += 17);
        const float tol = c.bf16 ? 2e-2f : 1e-4f;
        const bool pass = r.o <= tol && r.dq <= tol && r.dk <= tol && r.dv <= tol;
        std::cout << "[dropin] B=" << c.B << " Hq=" << c.Hq << " Hkv=" << c.Hkv << " S=" << c.S << " D=" << c.D
                  << (c.causal ? " causal" : " full") << (c.bf16 ? " bf16" : " fp32") << "  max-rel o=" << r.o
                  << " dq=" << r.dq << " dk=" << r.dk << " dv=" << r.dv << (pass ? "  ok" : "  FAIL") << std::endl;
        ok = ok && pass;
    }
    // The model graphs' masked composite: sliding window (Gemma) and padding
    // (Gemma -1e10, Qwen -1e9), including rows left with no visible key.
    struct MCase {
        int64_t B, Hq, Hkv, S, D, window;
        std::vector<int> lengths;
        float pad_value;
        bool bf16;
    };
    const MCase mcases[] = {
        {1, 2, 2, 40, 32, 8, {}, 0.f, false},              // sliding mask via memory_efficient_attention
        {2, 4, 1, 70, 64, 16, {70, 30}, -1e10f, false},    // Gemma: window + padding, rows 45.. see no key
        {2, 4, 1, 96, 256, 32, {50, 96}, -1e10f, true},
        {2, 14, 2, 33, 64, 0, {20, 33}, -1e9f, false},     // Qwen: causal + padding
        {2, 2, 1, 24, 32, 0, {0, 24}, -1e9f, false},       // an all-padding sequence
        {2, 2, 1, 40, 32, 8, {40, 40}, -1e10f, false},     // window + an all-ones attention_mask (pad mask of zeros)
    };
    for (const MCase& c : mcases) {
        const Result r = run_masked_case(c.B, c.Hq, c.Hkv, c.S, c.D, c.window, c.lengths, c.pad_value, c.bf16,
                                         seed += 17);
        const float tol = c.bf16 ? 2e-2f : 1e-4f;
        const bool pass = r.o <= tol && r.dq <= tol && r.dk <= tol && r.dv <= tol;
        std::cout << "[dropin] masked B=" << c.B << " Hq=" << c.Hq << " Hkv=" << c.Hkv << " S=" << c.S
                  << " D=" << c.D << " window=" << c.window << " padded=" << !c.lengths.empty()
                  << (c.bf16 ? " bf16" : " fp32") << "  max-rel o=" << r.o << " dq=" << r.dq << " dk=" << r.dk
                  << " dv=" << r.dv << (pass ? "  ok" : "  FAIL") << std::endl;
        ok = ok && pass;
    }
    // Any other additive mask (the kernels' mask mode): an arbitrary [S,S]
    // mask with -1e10 holes and a row masked everywhere, a 4-D [B,1,S,S]
    // mask, left padding, and a window with padding of another value.
    {
        struct AnyCase {
            const char* what;
            int64_t B, Hq, Hkv, S, D;
            TensorPtr base, pad;
            bool bf16;
        };
        auto ss = random_mask({40, 40}, 91, 0.3f);
        for (int64_t j = 0; j < 40; ++j) ss->data<float>()[7 * 40 + j] = -1e10f;
        auto left = pad_mask(2, 36, {36, 36}, 0.f);
        for (int64_t j = 0; j < 5; ++j) left->data<float>()[36 + j] = -1e10f;  // batch 1: the first keys masked
        const AnyCase any[] = {
            {"[S,S] mask", 2, 4, 2, 40, 64, ss, nullptr, false},
            {"[S,S] mask bf16", 1, 4, 1, 40, 256, ss, nullptr, true},
            {"[B,1,S,S] mask", 2, 2, 1, 33, 32, random_mask({2, 1, 33, 33}, 92, 0.2f), nullptr, false},
            {"left padding", 2, 4, 2, 36, 64, create_causal_mask(36, kFloat32, kCPU), left, false},
            {"window + padding of another value", 1, 2, 2, 24, 32, sliding_mask(24, 3), pad_mask(1, 24, {17}, -1e9f),
             false},
        };
        for (const AnyCase& c : any) {
            const Result r = run_any_mask_case(c.B, c.Hq, c.Hkv, c.S, c.D, c.base, c.pad, c.bf16, seed += 17);
            const float tol = c.bf16 ? 2e-2f : 1e-4f;
            const bool pass = r.o <= tol && r.dq <= tol && r.dk <= tol && r.dv <= tol;
            std::cout << "[dropin] mask mode, " << c.what << "  max-rel o=" << r.o << " dq=" << r.dq
                      << " dk=" << r.dk << " dv=" << r.dv << (pass ? "  ok" : "  FAIL") << std::endl;
            ok = ok && pass;
        }
        // One mask tensor passed again and again (a model passes its mask to
        // every layer), edited in place between calls: causal, then a sliding
        // window, then arbitrary values.  Each call must see the current values.
        {
            const int64_t S = 48;
            auto m = create_causal_mask(int(S), kFloat32, kCPU);
            float* p = m->data<float>();
            for (int step = 0; step < 4; ++step) {
                if (step == 2)
                    for (int64_t i = 0; i < S; ++i)
                        for (int64_t j = 0; j <= i; ++j) p[i * S + j] = (i - j < 5) ? 0.f : -1e10f;
                if (step == 3)
                    for (int64_t i = 0; i < S * S; ++i) p[i] = std::fmod(float(i) * 0.618034f, 1.0f) - 0.5f;
                const Result r = run_any_mask_case(1, 2, 1, S, 32, m, nullptr, false, seed += 17);
                const bool pass = r.o <= 1e-4f && r.dq <= 1e-4f && r.dk <= 1e-4f && r.dv <= 1e-4f;
                std::cout << "[dropin] reused mask tensor, call " << step << "  max-rel o=" << r.o << " dq=" << r.dq
                          << " dk=" << r.dk << " dv=" << r.dv << (pass ? "  ok" : "  FAIL") << std::endl;
                ok = ok && pass;
            }
        }
        for (bool causal : {false, true}) {
            const float e = run_nograd_mask_case(2, 3, 40, 32, ss, causal, seed += 17);
            std::cout << "[dropin] mask mode, no grad" << (causal ? " causal" : "") << "  max-rel o=" << e
                      << (e <= 1e-5f ? "  ok" : "  FAIL") << std::endl;
            ok = ok && e <= 1e-5f;
        }
        autograd::Engine::instance().clear_graph();
    }
    // No-grad path equals the grad path's output (same kernels, no LSE kept).
    {
        auto q = make({1, 2, 20, 16}, 7, 1.0f, false, false);
        auto k = make({1, 2, 20, 16}, 8, 1.0f, false, false);
        auto v = make({1, 2, 20, 16}, 9, 1.0f, false, false);
        auto a = memory_efficient_attention(q, k, v, nullptr, {});
        auto qg = copy_of(q, true);
        auto b = memory_efficient_attention(qg, k, v, nullptr, {});
        const float d = max_rel(a, b);
        std::cout << "[dropin] no-grad vs grad output max-rel " << d << std::endl;
        ok = ok && d == 0.0f;
        autograd::Engine::instance().clear_graph();
    }
    // Errors keep the reference's exception convention.
    auto q = make({1, 2, 8, 16}, 1, 1.0f, false, false);
    auto k3 = make({1, 3, 8, 16}, 2, 1.0f, false, false);
    auto mask4 = make({1, 1, 8, 8}, 3, 1.0f, false, false);
    ok = expect_throw("q 2 heads, k 3 heads", [&] { memory_efficient_attention(q, k3, k3, nullptr, {}); }) && ok;
    // the reference's no-grad operator takes only [S,S] masks (.cpp:114-120)
    ok = expect_throw("4-D mask without grad", [&] { memory_efficient_attention(q, q, q, mask4, {}); }) && ok;
    ok = expect_throw("mask of another length", [&] {
        memory_efficient_attention(q, q, q, make({9, 9}, 4, 1.0f, false, false), {});
    }) && ok;
    ok = expect_throw("3-D input", [&] {
        auto t = zeros({2, 8, 16}, kFloat32, kCPU);
        memory_efficient_attention(t, t, t, nullptr, {});
    }) && ok;
    std::cout << (ok ? "[PASS]" : "[FAIL]") << std::endl;
    return ok ? 0 : 1;
}
