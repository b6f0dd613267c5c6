// Parity test of the drop-in LM losses (lm_loss_hip.cpp) through the
// reference API (core/lm_loss.h), on shapes larger than the reference's own
// unit test: a vocabulary that spans several streaming chunks, ignored and
// shifted labels, every reduction, an fp32 and a bf16 lm_head_weight.
// Expected values are the reference's formulas (core/lm_loss.cpp:74-163,
// 165-266, 268-382, 384-481) evaluated here in double precision.
#include "lm_loss.h"
#include "ops.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

using namespace ops;

namespace {

int failures = 0;

void check(const std::string& name, const float* got, const std::vector<double>& want, double rtol) {
    double scale = 0.0, err = 0.0;
    for (double w : want) scale = std::max(scale, std::fabs(w));
    for (size_t i = 0; i < want.size(); ++i) err = std::max(err, std::fabs(double(got[i]) - want[i]));
    const bool ok = err <= rtol * scale + 1e-7;
    std::printf("%-44s max_abs_err=%.3e scale=%.3e %s\n", name.c_str(), err, scale, ok ? "ok" : "FAIL");
    if (!ok) ++failures;
}

struct Problem {
    int64_t B, S, H, V;
    std::vector<float> hidden, weight;  // weight as the fp32 values the kernels see
    std::vector<uint16_t> weight_bf16;
    std::vector<int32_t> labels;
};

uint16_t to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return static_cast<uint16_t>((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

Problem make(int64_t B, int64_t S, int64_t H, int64_t V, bool bf16, unsigned seed) {
    Problem p{B, S, H, V, {}, {}, {}, {}};
    std::mt19937 rng(seed);
    std::normal_distribution<float> n(0.f, 1.f);
    p.hidden.resize(B * S * H);
    for (auto& v : p.hidden) v = n(rng);
    p.weight.resize(V * H);
    for (auto& v : p.weight) v = n(rng) * 0.2f;
    if (bf16) {
        p.weight_bf16.resize(p.weight.size());
        for (size_t i = 0; i < p.weight.size(); ++i) {
            p.weight_bf16[i] = to_bf16(p.weight[i]);
            p.weight[i] = bf16_bits_to_float32(p.weight_bf16[i]);
        }
    }
    std::uniform_int_distribution<int32_t> cls(0, static_cast<int32_t>(V - 1));
    p.labels.resize(B * S);
    for (auto& l : p.labels) l = (rng() % 4 == 0) ? -100 : cls(rng);
    return p;
}

// Loss, per-position NLL, dlogits, dhidden, dweight of the reference formulas.
struct Expected {
    double sum = 0;
    int64_t count = 0;
    std::vector<double> nll, logits, dlogits, dhidden, dweight;
};

Expected expected(const Problem& p, bool mean, double g) {
    Expected e;
    const int64_t B = p.B, S = p.S, H = p.H, V = p.V;
    e.nll.assign(B * S, 0.0);
    e.logits.assign(B * S * V, 0.0);
    e.dlogits.assign(B * S * V, 0.0);
    e.dhidden.assign(B * S * H, 0.0);
    e.dweight.assign(V * H, 0.0);
    for (int64_t r = 0; r < B * S; ++r)
        for (int64_t v = 0; v < V; ++v) {
            double z = 0;
            for (int64_t h = 0; h < H; ++h) z += double(p.hidden[r * H + h]) * p.weight[v * H + h];
            e.logits[r * V + v] = static_cast<float>(z);  // the dense path gets fp32 logits
        }
    for (int64_t b = 0; b < B; ++b)
        for (int64_t s = 0; s + 1 < S; ++s)
            if (p.labels[b * S + s + 1] != -100) ++e.count;
    const double coeff = mean ? (e.count ? g / double(e.count) : 0.0) : g;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t s = 0; s + 1 < S; ++s) {
            const int32_t y = p.labels[b * S + s + 1];
            if (y == -100) continue;
            const int64_t r = b * S + s;
            const double* z = &e.logits[r * V];
            double m = z[0], den = 0;
            for (int64_t v = 0; v < V; ++v) m = std::max(m, z[v]);
            for (int64_t v = 0; v < V; ++v) den += std::exp(z[v] - m);
            const double lse = m + std::log(den);
            e.nll[r] = lse - z[y];
            e.sum += e.nll[r];
            for (int64_t v = 0; v < V; ++v) {
                const double gz = (std::exp(z[v] - lse) - (v == y ? 1.0 : 0.0)) * coeff;
                e.dlogits[r * V + v] = gz;
                for (int64_t h = 0; h < H; ++h) {
                    e.dhidden[r * H + h] += gz * p.weight[v * H + h];
                    e.dweight[v * H + h] += gz * p.hidden[r * H + h];
                }
            }
        }
    return e;
}

TensorPtr hidden_tensor(const Problem& p) {
    auto t = std::make_shared<Tensor>(std::vector<int64_t>{p.B, p.S, p.H}, p.hidden.data(), kFloat32, kCPU);
    t->set_requires_grad(true);
    return t;
}

TensorPtr weight_tensor(const Problem& p) {
    auto t = p.weight_bf16.empty()
                 ? std::make_shared<Tensor>(std::vector<int64_t>{p.V, p.H}, p.weight.data(), kFloat32, kCPU)
                 : std::make_shared<Tensor>(std::vector<int64_t>{p.V, p.H}, p.weight_bf16.data(), kBFloat16, kCPU);
    t->set_requires_grad(true);
    return t;
}

void run_selected(const std::string& tag, const Problem& p, const std::string& red) {
    const Expected e = expected(p, red == "mean", 1.0);
    auto labels = std::make_shared<Tensor>(std::vector<int64_t>{p.B, p.S}, const_cast<int32_t*>(p.labels.data()),
                                           kInt32, kCPU);
    auto h = hidden_tensor(p);
    auto w = weight_tensor(p);
    auto loss = streaming_lm_cross_entropy(h, w, labels, -100, red);
    loss->backward();
    const std::vector<double> want{red == "mean" ? e.sum / double(e.count) : e.sum};
    check(tag + " " + red + " loss", loss->data<float>(), want, 1e-5);
    check(tag + " " + red + " grad_hidden", h->grad()->data<float>(), e.dhidden, 1e-4);
    check(tag + " " + red + " grad_weight", w->grad()->data<float>(), e.dweight, 1e-4);
}

// Dense lm_cross_entropy.  The reference scores "sum" and "sum_debug" as a
// sum and any other string but "none" as a mean, and normalises the gradient
// only for exactly "mean" (core/lm_loss.cpp:96-100, 318-364).
void run_dense(const std::string& tag, const Problem& p, const std::string& red) {
    const bool sum_loss = red == "sum" || red == "sum_debug";
    const Expected e = expected(p, red == "mean", 1.0);
    std::vector<float> z(e.logits.begin(), e.logits.end());
    auto logits = std::make_shared<Tensor>(std::vector<int64_t>{p.B, p.S, p.V}, z.data(), kFloat32, kCPU);
    logits->set_requires_grad(true);
    auto labels = std::make_shared<Tensor>(std::vector<int64_t>{p.B, p.S}, const_cast<int32_t*>(p.labels.data()),
                                           kInt32, kCPU);
    auto loss = lm_cross_entropy(logits, labels, -100, red);
    if (red == "none") {
        check(tag + " none nll", loss->data<float>(), e.nll, 1e-5);
        return;
    }
    loss->backward();
    const std::vector<double> want{sum_loss ? e.sum : e.sum / double(e.count)};
    check(tag + " dense " + red + " loss", loss->data<float>(), want, 1e-5);
    check(tag + " dense " + red + " grad_logits", logits->grad()->data<float>(), e.dlogits, 1e-4);
}

template <class F>
void expect_throw(const std::string& name, F f) {
    bool threw = false;
    try {
        f();
    } catch (const std::runtime_error& ex) {
        threw = true;
        std::printf("%-44s threw: %s\n", name.c_str(), ex.what());
    }
    if (!threw) {
        std::printf("%-44s FAIL (no exception)\n", name.c_str());
        ++failures;
    }
}

}  // namespace

int main() {
    // 20000 rows: two vocabulary chunks of the streaming path (16384 each).
    const Problem a = make(2, 37, 64, 20000, false, 1);
    const Problem b = make(3, 19, 96, 1537, true, 2);
    for (const char* red : {"mean", "sum"}) {
        run_selected("fp32 B2 S37 H64 V20000", a, red);
        run_selected("bf16w B3 S19 H96 V1537", b, red);
    }
    for (const char* red : {"mean", "sum", "none", "sum_debug", "avg"}) run_dense("B3 S19 V1537", b, red);

    Problem bad = b;
    bad.labels[1] = static_cast<int32_t>(bad.V);
    auto bad_labels = std::make_shared<Tensor>(std::vector<int64_t>{bad.B, bad.S}, bad.labels.data(), kInt32, kCPU);
    expect_throw("selected: label out of range", [&] {
        selected_token_lm_cross_entropy(hidden_tensor(bad), weight_tensor(bad), bad_labels, -100, "mean");
    });
    expect_throw("selected: reduction none", [&] {
        auto ok = std::make_shared<Tensor>(std::vector<int64_t>{b.B, b.S}, const_cast<int32_t*>(b.labels.data()),
                                           kInt32, kCPU);
        selected_token_lm_cross_entropy(hidden_tensor(b), weight_tensor(b), ok, -100, "none");
    });
    if (failures) {
        std::printf("[FAIL] %d checks\n", failures);
        return 1;
    }
    std::printf("[PASS] drop-in LM losses match the reference formulas\n");
    return 0;
}
