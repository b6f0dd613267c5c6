// Measurements of the drop-in ops::memory_efficient_attention through the
// reference's own API (host Tensors in, host gradients out):
//
//   dropin_probe saved B Hq Hkv S D f32|bf16
//       bytes the forward's autograd node keeps alive until backward: device
//       bytes (the adapters' allocator's live-byte count) and host bytes
//       (MemoryManager::get_memory_usage(), core/memory_manager.h:144, plus
//       the adapters' pinned result blocks), each after the forward minus
//       before it, with the output still referenced.
//   dropin_probe step B Hq Hkv S D f32|bf16 WARMUP ITERS [mask]
//       wall time of forward + Engine backward per step, host copies (PCIe)
//       included, and the hipMalloc calls made during the timed steps; with
//       "mask", an [S,S] causal mask tensor built once and passed to every
//       step (as a model passes its mask to every layer).  Also the transfer
//       floor: the step's host<->device bytes (q, k, v and the fp32 dO in;
//       the fp32 O, dQ, dK and dV out) over this box's pinned-copy rates,
//       measured here with hipMemcpy of 64 MiB between hipHostMalloc memory
//       and the device.
//
// Prints one JSON object.  Inputs are seeded N(0,1) (dO N(0,0.1)), causal.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include <hip/hip_runtime.h>

#include "autograd_engine.h"
#include "memory_efficient_attention.h"
#include "memory_manager.h"
#include "ops.h"

extern "C" void mft_dropin_pool_stats(size_t* live_bytes, size_t* cached_bytes, size_t* device_mallocs);
extern "C" size_t mft_dropin_pinned_bytes();

using namespace ops;

namespace {

uint64_t mix(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// fp32 host tensor of N(0, sigma^2) values, or its bf16 rounding.
TensorPtr make(const std::vector<int64_t>& shape, uint64_t seed, float sigma, bool bf16, bool grad) {
    auto f = zeros(shape, kFloat32, kCPU);
    float* p = f->data<float>();
    for (int64_t i = 0; i < f->numel(); ++i) {
        const double u1 = ((mix(seed * 977 + 2 * i) >> 11) + 1.0) * (1.0 / 9007199254740993.0);
        const double u2 = (mix(seed * 977 + 2 * i + 1) >> 11) * (1.0 / 9007199254740992.0);
        p[i] = float(sigma * std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
    }
    if (!bf16) {
        f->set_requires_grad(grad);
        return f;
    }
    auto b = zeros(shape, kBFloat16, kCPU);
    uint16_t* d = b->data<uint16_t>();
    for (int64_t i = 0; i < f->numel(); ++i) d[i] = float32_to_bf16_bits(p[i]);
    b->set_requires_grad(grad);
    return b;
}

size_t pool_live() {
    size_t live = 0;
    mft_dropin_pool_stats(&live, nullptr, nullptr);
    return live;
}

// Pinned host <-> device copy rates in bytes/s (best of 5 copies of 64 MiB).
void pinned_rates(double* h2d, double* d2h) {
    const size_t n = size_t(64) << 20;
    void* host = nullptr;
    void* dev = nullptr;
    if (hipHostMalloc(&host, n, hipHostMallocDefault) != hipSuccess || hipMalloc(&dev, n) != hipSuccess)
        throw std::runtime_error("pinned_rates: allocation failed");
    std::memset(host, 1, n);
    auto best = [&](hipMemcpyKind kind) {
        double t = 1e30;
        for (int r = 0; r < 6; ++r) {
            const auto t0 = std::chrono::steady_clock::now();
            if (kind == hipMemcpyHostToDevice ? hipMemcpy(dev, host, n, kind) : hipMemcpy(host, dev, n, kind))
                throw std::runtime_error("pinned_rates: copy failed");
            const double s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
            if (r) t = std::min(t, s);  // the first copy warms up
        }
        return n / t;
    };
    *h2d = best(hipMemcpyHostToDevice);
    *d2h = best(hipMemcpyDeviceToHost);
    (void)hipFree(dev);
    (void)hipHostFree(host);
}

size_t pool_mallocs() {
    size_t n = 0;
    mft_dropin_pool_stats(nullptr, nullptr, &n);
    return n;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 8) {
        std::fprintf(stderr, "usage: %s saved|step B Hq Hkv S D f32|bf16 [WARMUP ITERS]\n", argv[0]);
        return 2;
    }
    const std::string mode = argv[1];
    const int64_t B = std::atoll(argv[2]), Hq = std::atoll(argv[3]), Hkv = std::atoll(argv[4]),
                  S = std::atoll(argv[5]), D = std::atoll(argv[6]);
    const bool bf16 = std::string(argv[7]) == "bf16";
    try {
        auto q = make({B, Hq, S, D}, 1, 1.0f, bf16, true);
        auto k = make({B, Hkv, S, D}, 2, 1.0f, bf16, true);
        auto v = make({B, Hkv, S, D}, 3, 1.0f, bf16, true);
        auto g = make({B, Hq, S, D}, 4, 0.1f, false, false);  // Engine gradients are fp32
        MemoryEfficientAttentionConfig cfg;
        cfg.use_causal_mask = true;
        if (mode == "saved") {
            const size_t dev0 = pool_live();
            const size_t host0 = MemoryManager::instance().get_memory_usage() + mft_dropin_pinned_bytes();
            auto out = memory_efficient_attention(q, k, v, nullptr, cfg);
            const size_t dev1 = pool_live();
            const size_t host1 = MemoryManager::instance().get_memory_usage() + mft_dropin_pinned_bytes();
            std::printf("{\"device_bytes\": %lld, \"host_bytes\": %lld}\n", (long long)(dev1 - dev0),
                        (long long)host1 - (long long)host0);
            autograd::Engine::instance().run_backward({out}, {g});
            return 0;
        }
        if (mode == "step" && argc >= 10) {
            const int warmup = std::atoi(argv[8]), iters = std::atoi(argv[9]);
            const bool with_mask = argc >= 11 && std::string(argv[10]) == "mask";
            TensorPtr mask;
            if (with_mask) {
                mask = zeros({S, S}, kFloat32, kCPU);
                float* m = mask->data<float>();
                for (int64_t i = 0; i < S; ++i)
                    for (int64_t j = i + 1; j < S; ++j) m[i * S + j] = -1e10f;
            }
            auto one = [&] {
                auto out = memory_efficient_attention(q, k, v, mask, cfg);
                autograd::Engine::instance().run_backward({out}, {g});
                // Gradients dropped between steps (not zero_grad): with kept
                // gradients the reference Engine adds the new ones into them
                // on the host (core/autograd_engine.cpp:248-262), a cost of
                // this probe's leaf tensors, where in a model q, k and v come
                // from earlier ops and their gradients flow on to those.
                q->set_grad(nullptr);
                k->set_grad(nullptr);
                v->set_grad(nullptr);
            };
            for (int i = 0; i < warmup; ++i) one();
            const size_t m0 = pool_mallocs();
            const auto t0 = std::chrono::steady_clock::now();
            for (int i = 0; i < iters; ++i) one();
            const auto t1 = std::chrono::steady_clock::now();
            const double ms = std::chrono::duration<double, std::milli>(t1 - t0).count() / iters;
            const long long mallocs = (long long)(pool_mallocs() - m0);
            double h2d = 0, d2h = 0;
            pinned_rates(&h2d, &d2h);
            const double in_b = double(q->numel() + k->numel() + v->numel()) * (bf16 ? 2 : 4) + double(g->numel()) * 4;
            const double out_b = double(q->numel() + q->numel() + k->numel() + v->numel()) * 4;
            const double floor_ms = 1e3 * (in_b / h2d + out_b / d2h);
            std::printf("{\"ms_per_step\": %.5f, \"iters\": %d, \"device_mallocs_timed\": %lld, \"mask\": %s, "
                        "\"h2d_bytes\": %.0f, \"d2h_bytes\": %.0f, \"h2d_gbs\": %.2f, \"d2h_gbs\": %.2f, "
                        "\"floor_ms\": %.5f, \"x_floor\": %.2f}\n",
                        ms, iters, mallocs, with_mask ? "true" : "false", in_b, out_b, h2d / 1e9, d2h / 1e9, floor_ms,
                        ms / floor_ms);
            return 0;
        }
        std::fprintf(stderr, "bad mode or arguments\n");
        return 2;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "dropin_probe: %s\n", e.what());
        return 1;
    }
}
