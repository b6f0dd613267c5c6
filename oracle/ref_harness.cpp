// ref_harness — C entry points over the REAL reference operators.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles this file together with
// the reference's own sources (read in place under /root/reference, never
// copied) into oracle/_ref/libmftref.so.  It is used to
//   * pin the restatement in refcpu.cpp bit for bit (tests/test_oracle.py),
//   * write the golden fixtures (tests/golden/make_golden.py), and
//   * time the reference CPU path beside the GPU (bench.py cpu_baseline).
//
// The graph built here is the one the reference's model code builds for
// attention (graph/gemma_model.cpp:481-505, graph/qwen_model.cpp:302-318,
// core/memory_efficient_attention.cpp:23-43):
//   repeat_kv_heads -> transpose -> matmul -> mul(scale) -> add(causal mask)
//   -> softmax -> matmul, then autograd::Engine::run_backward({out}, {dO}).
#include "core/autograd_engine.h"
#include "core/lm_loss.h"
#include "core/memory_efficient_attention.h"
#include "core/memory_manager.h"
#include "core/ops.h"
#include "nn/lora_linear.h"

#include <chrono>
#include <cstring>
#include <exception>
#include <iostream>
#include <vector>

using namespace ops;

namespace {

TensorPtr from_host(const float* src, const std::vector<int64_t>& shape, bool requires_grad) {
    auto t = zeros(shape, kFloat32, kCPU);
    std::memcpy(t->data<float>(), src, sizeof(float) * static_cast<size_t>(t->numel()));
    t->set_requires_grad(requires_grad);
    return t;
}

void to_host(const TensorPtr& t, float* dst) {
    if (!dst) return;
    if (!t) return;
    std::memcpy(dst, t->data<float>(), sizeof(float) * static_cast<size_t>(t->numel()));
}

double now_s() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

}  // namespace

extern "C" {

// Returns 0 on success.  Timings in seconds; held_bytes = MemoryManager bytes
// in use after the forward minus before it (what the autograd graph keeps
// alive until backward), the reference's saved-activation measure.
static int composite_impl(const float* q, const float* k, const float* v, const float* dO,
                          int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D,
                          float scale, int causal,
                          float* o, float* dq, float* dk, float* dv,
                          double* t_fwd, double* t_bwd, int64_t* held_bytes, bool keep_graph_only) {
    try {
        const bool grad = dO != nullptr || keep_graph_only;
        auto qt = from_host(q, {B, Hq, S, D}, grad);
        auto kt = from_host(k, {B, Hkv, S, D}, grad);
        auto vt = from_host(v, {B, Hkv, S, D}, grad);
        TensorPtr gt;
        if (dO) gt = from_host(dO, {B, Hq, S, D}, false);
        const size_t before = MemoryManager::instance().get_memory_usage();

        const double t0 = now_s();
        TensorPtr k_use = kt, v_use = vt;
        if (Hq != Hkv) {
            const int rep = static_cast<int>(Hq / Hkv);
            k_use = repeat_kv_heads(kt, rep);
            v_use = repeat_kv_heads(vt, rep);
        }
        auto k_t = transpose(k_use, 2, 3);
        auto scores = mul(matmul(qt, k_t), scale);
        if (causal) scores = add(scores, create_causal_mask(static_cast<int>(S), kFloat32, kCPU));
        auto probs = softmax(scores, -1);
        auto out = matmul(probs, v_use);
        const double t1 = now_s();
        const size_t after = MemoryManager::instance().get_memory_usage();
        // Drop the local handles that are not graph-held so that the count
        // below reflects what the graph itself keeps.
        k_t.reset(); scores.reset(); probs.reset(); k_use.reset(); v_use.reset();
        to_host(out, o);
        if (t_fwd) *t_fwd = t1 - t0;
        if (held_bytes) *held_bytes = static_cast<int64_t>(after) - static_cast<int64_t>(before);

        if (dO) {
            const double t2 = now_s();
            autograd::Engine::instance().run_backward({out}, {gt});
            const double t3 = now_s();
            if (t_bwd) *t_bwd = t3 - t2;
            to_host(qt->grad(), dq);
            to_host(kt->grad(), dk);
            to_host(vt->grad(), dv);
        } else if (t_bwd) {
            *t_bwd = 0.0;
        }
        autograd::Engine::instance().clear_graph();
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "[mftref_composite] " << e.what() << std::endl;
        return -1;
    }
}

int mftref_composite(const float* q, const float* k, const float* v, const float* dO,
                     int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D,
                     float scale, int causal,
                     float* o, float* dq, float* dk, float* dv,
                     double* t_fwd, double* t_bwd, int64_t* held_bytes) {
    return composite_impl(q, k, v, dO, B, Hq, Hkv, S, D, scale, causal, o, dq, dk, dv, t_fwd, t_bwd, held_bytes,
                          false);
}

// The forward of mftref_composite with inputs that require grad, so that the
// autograd graph is built, and no backward: held_bytes is what that graph
// keeps for the backward (the saved-activation figure) at a fraction of the
// cost of the full step.
int mftref_composite_saved(const float* q, const float* k, const float* v,
                           int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D,
                           float scale, int causal, float* o, int64_t* held_bytes) {
    return composite_impl(q, k, v, nullptr, B, Hq, Hkv, S, D, scale, causal, o, nullptr, nullptr, nullptr,
                          nullptr, nullptr, held_bytes, true);
}

// The composite with explicit additive masks, as graph/gemma_model.cpp:481-505
// applies them: scores = add(scores, base_mask [S,S]) (causal or sliding
// window), then add(scores, pad_mask [B,1,1,S]).  Either mask may be NULL.
int mftref_composite_masked(const float* q, const float* k, const float* v, const float* dO,
                            int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D,
                            float scale, const float* base_mask, const float* pad_mask,
                            float* o, float* dq, float* dk, float* dv) {
    try {
        const bool grad = dO != nullptr;
        auto qt = from_host(q, {B, Hq, S, D}, grad);
        auto kt = from_host(k, {B, Hkv, S, D}, grad);
        auto vt = from_host(v, {B, Hkv, S, D}, grad);
        TensorPtr gt;
        if (grad) gt = from_host(dO, {B, Hq, S, D}, false);
        TensorPtr k_use = kt, v_use = vt;
        if (Hq != Hkv) {
            const int rep = static_cast<int>(Hq / Hkv);
            k_use = repeat_kv_heads(kt, rep);
            v_use = repeat_kv_heads(vt, rep);
        }
        auto scores = mul(matmul(qt, transpose(k_use, 2, 3)), scale);
        if (base_mask) scores = add(scores, from_host(base_mask, {S, S}, false));
        if (pad_mask) scores = add(scores, from_host(pad_mask, {B, 1, 1, S}, false));
        auto out = matmul(softmax(scores, -1), v_use);
        to_host(out, o);
        if (grad) {
            autograd::Engine::instance().run_backward({out}, {gt});
            to_host(qt->grad(), dq);
            to_host(kt->grad(), dk);
            to_host(vt->grad(), dv);
        }
        autograd::Engine::instance().clear_graph();
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "[mftref_composite_masked] " << e.what() << std::endl;
        return -1;
    }
}

// The composite with up to two additive masks given as dense tensors of
// shape [mb, mh, mi, S] (mb in {1, B}, mh in {1, Hq}, mi in {1, S}), added to
// the scaled scores by ops::add with its broadcasting (core/ops.cpp:299-377),
// mask 0 first; no causal mask (the composite of
// core/memory_efficient_attention.cpp:23-43 with a mask given).
int mftref_composite_mask4(const float* q, const float* k, const float* v, const float* dO,
                           int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D, float scale,
                           const float* m0, int64_t m0b, int64_t m0h, int64_t m0i,
                           const float* m1, int64_t m1b, int64_t m1h, int64_t m1i,
                           float* o, float* dq, float* dk, float* dv) {
    try {
        const bool grad = dO != nullptr;
        auto qt = from_host(q, {B, Hq, S, D}, grad);
        auto kt = from_host(k, {B, Hkv, S, D}, grad);
        auto vt = from_host(v, {B, Hkv, S, D}, grad);
        TensorPtr gt;
        if (grad) gt = from_host(dO, {B, Hq, S, D}, false);
        TensorPtr k_use = kt, v_use = vt;
        if (Hq != Hkv) {
            const int rep = static_cast<int>(Hq / Hkv);
            k_use = repeat_kv_heads(kt, rep);
            v_use = repeat_kv_heads(vt, rep);
        }
        auto scores = mul(matmul(qt, transpose(k_use, 2, 3)), scale);
        if (m0) scores = add(scores, from_host(m0, {m0b, m0h, m0i, S}, false));
        if (m1) scores = add(scores, from_host(m1, {m1b, m1h, m1i, S}, false));
        auto out = matmul(softmax(scores, -1), v_use);
        to_host(out, o);
        if (grad) {
            autograd::Engine::instance().run_backward({out}, {gt});
            to_host(qt->grad(), dq);
            to_host(kt->grad(), dk);
            to_host(vt->grad(), dv);
        }
        autograd::Engine::instance().clear_graph();
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "[mftref_composite_mask4] " << e.what() << std::endl;
        return -1;
    }
}

// ops::memory_efficient_attention without grad and with an [S,S] mask: the
// streaming path applies the causal rule, then adds the mask
// (core/memory_efficient_attention.cpp:160-172).
int mftref_memeff_nograd_mask(const float* q, const float* k, const float* v,
                              int64_t B, int64_t H, int64_t S, int64_t D,
                              float scale, int causal, const float* mask, float* o) {
    try {
        auto qt = from_host(q, {B, H, S, D}, false);
        auto kt = from_host(k, {B, H, S, D}, false);
        auto vt = from_host(v, {B, H, S, D}, false);
        MemoryEfficientAttentionConfig cfg;
        cfg.use_causal_mask = causal != 0;
        cfg.scale = scale;
        auto out = memory_efficient_attention(qt, kt, vt, from_host(mask, {S, S}, false), cfg);
        to_host(out, o);
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "[mftref_memeff_nograd_mask] " << e.what() << std::endl;
        return -1;
    }
}

// ops::memory_efficient_attention with no input requiring grad: the
// reference's streaming path (core/memory_efficient_attention.cpp:110-200).
int mftref_memeff_nograd(const float* q, const float* k, const float* v,
                         int64_t B, int64_t H, int64_t S, int64_t D,
                         float scale, int causal, float* o) {
    try {
        auto qt = from_host(q, {B, H, S, D}, false);
        auto kt = from_host(k, {B, H, S, D}, false);
        auto vt = from_host(v, {B, H, S, D}, false);
        MemoryEfficientAttentionConfig cfg;
        cfg.use_causal_mask = causal != 0;
        cfg.scale = scale;
        auto out = memory_efficient_attention(qt, kt, vt, nullptr, cfg);
        to_host(out, o);
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "[mftref_memeff_nograd] " << e.what() << std::endl;
        return -1;
    }
}

// ops::memory_efficient_attention with inputs requiring grad: the reference
// falls back to the composite (core/memory_efficient_attention.cpp:106-108);
// gradients come from Engine::run_backward.
int mftref_memeff_grad(const float* q, const float* k, const float* v, const float* dO,
                       int64_t B, int64_t H, int64_t S, int64_t D,
                       float scale, int causal,
                       float* o, float* dq, float* dk, float* dv) {
    try {
        auto qt = from_host(q, {B, H, S, D}, true);
        auto kt = from_host(k, {B, H, S, D}, true);
        auto vt = from_host(v, {B, H, S, D}, true);
        auto gt = from_host(dO, {B, H, S, D}, false);
        MemoryEfficientAttentionConfig cfg;
        cfg.use_causal_mask = causal != 0;
        cfg.scale = scale;
        auto out = memory_efficient_attention(qt, kt, vt, nullptr, cfg);
        to_host(out, o);
        autograd::Engine::instance().run_backward({out}, {gt});
        to_host(qt->grad(), dq);
        to_host(kt->grad(), dk);
        to_host(vt->grad(), dv);
        autograd::Engine::instance().clear_graph();
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "[mftref_memeff_grad] " << e.what() << std::endl;
        return -1;
    }
}

// repeat_kv_heads forward and its Engine backward (RepeatKVHeadsBackward).
int mftref_repeat_kv(const float* kv, const float* g, int64_t B, int64_t Hkv, int64_t S,
                     int64_t D, int64_t r, float* out, float* dkv) {
    try {
        auto kt = from_host(kv, {B, Hkv, S, D}, g != nullptr);
        auto rep = repeat_kv_heads(kt, static_cast<int>(r));
        to_host(rep, out);
        if (g) {
            auto gt = from_host(g, {B, Hkv * r, S, D}, false);
            autograd::Engine::instance().run_backward({rep}, {gt});
            to_host(kt->grad(), dkv);
        }
        autograd::Engine::instance().clear_graph();
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "[mftref_repeat_kv] " << e.what() << std::endl;
        return -1;
    }
}

// The reference's bf16 rounding (core/dtype.h:114-121), for pinning refcpu's.
uint16_t mftref_f32_to_bf16_bits(float x) { return float32_to_bf16_bits(x); }

// The q/k prologue of graph/gemma_model.cpp:459-471: ops::rms_norm (norm 1)
// or ops::rms_norm_affine (norm 2) or nothing (norm 0), then ops::apply_rope
// when theta > 0; backward by Engine::run_backward({y}, {dy}).  x is
// [B, H, S, D]; w is [D]; dw, dx, dy may be NULL (dy NULL skips the backward).
int mftref_prologue(const float* x, const float* w, const float* dy, int64_t B, int64_t H, int64_t S,
                    int64_t D, int norm, float eps, float theta, float* y, float* dx, float* dw) {
    try {
        const bool grad = dy != nullptr;
        auto xt = from_host(x, {B, H, S, D}, grad);
        TensorPtr wt;
        if (norm != 0) wt = from_host(w, {D}, grad);
        TensorPtr t = xt;
        if (norm == 1) t = rms_norm(t, wt, eps);
        if (norm == 2) t = rms_norm_affine(t, wt, eps);
        if (theta > 0.f) t = apply_rope(t, static_cast<int>(S), static_cast<int>(D), theta);
        to_host(t, y);
        if (grad) {
            autograd::Engine::instance().run_backward({t}, {from_host(dy, {B, H, S, D}, false)});
            to_host(xt->grad(), dx);
            if (wt) to_host(wt->grad(), dw);
        }
        autograd::Engine::instance().clear_graph();
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "[mftref_prologue] " << e.what() << std::endl;
        return -1;
    }
}

// ops::lm_cross_entropy with its Engine backward (core/lm_loss.cpp:268-382).
// reduction 0 mean, 1 sum, 2 none; grad_out [1] or [B, S] (NULL: no
// backward).  Returns -1 when the reference throws.
int mftref_lm_ce(const float* logits, const int32_t* labels, int64_t B, int64_t S, int64_t V, int ignore_index,
                 int reduction, const float* grad_out, float* loss, float* grad_logits) {
    try {
        static const char* red[] = {"mean", "sum", "none"};
        auto lt = from_host(logits, {B, S, V}, grad_out != nullptr);
        auto yt = std::make_shared<Tensor>(std::vector<int64_t>{B, S}, labels, kInt32, kCPU);
        auto out = lm_cross_entropy(lt, yt, ignore_index, red[reduction]);
        to_host(out, loss);
        if (grad_out) {
            auto g = reduction == 2 ? from_host(grad_out, {B, S}, false) : from_host(grad_out, {1}, false);
            autograd::Engine::instance().run_backward({out}, {g});
            to_host(lt->grad(), grad_logits);
        }
        autograd::Engine::instance().clear_graph();
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "[mftref_lm_ce] " << e.what() << std::endl;
        autograd::Engine::instance().clear_graph();
        return -1;
    }
}

// ops::streaming_lm_cross_entropy (= selected_token_lm_cross_entropy) with its
// Engine backward (core/lm_loss.cpp:165-266, 384-481); reduction 0 mean, 1 sum.
int mftref_streaming_ce(const float* hidden, const float* weight, const int32_t* labels, int64_t B, int64_t S,
                        int64_t H, int64_t V, int ignore_index, int reduction, float grad_out, float* loss,
                        float* grad_hidden, float* grad_weight) {
    try {
        static const char* red[] = {"mean", "sum"};
        const bool grad = grad_hidden || grad_weight;
        auto ht = from_host(hidden, {B, S, H}, grad);
        auto wt = from_host(weight, {V, H}, grad);
        auto yt = std::make_shared<Tensor>(std::vector<int64_t>{B, S}, labels, kInt32, kCPU);
        auto out = streaming_lm_cross_entropy(ht, wt, yt, ignore_index, red[reduction]);
        to_host(out, loss);
        if (grad) {
            autograd::Engine::instance().run_backward({out}, {from_host(&grad_out, {1}, false)});
            if (grad_hidden) to_host(ht->grad(), grad_hidden);
            if (grad_weight) to_host(wt->grad(), grad_weight);
        }
        autograd::Engine::instance().clear_graph();
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "[mftref_streaming_ce] " << e.what() << std::endl;
        autograd::Engine::instance().clear_graph();
        return -1;
    }
}


// ops::LoRALinear (nn/lora_linear.cpp) forward and Engine backward, slices
// packed as in orc_lora (refcpu.h).  W is built fp32 or, with w_bf16, bf16
// from its (bf16-exact) values; x, A, B require grad.  A slice without a
// gradient (the reference gives column-range slices none) leaves its dA/dB
// untouched and has_grad[i] = 0.
int mftref_lora(const float* x, const float* W, const float* bias, int64_t N, int64_t in, int64_t out,
                int w_transposed, int w_bf16, int n, const int64_t* meta, const float* scale, const float* A_all,
                const float* B_all, const float* dy, float* y, float* dx, float* dA_all, float* dB_all,
                int32_t* has_grad) {
    try {
        const std::vector<int64_t> wshape = w_transposed ? std::vector<int64_t>{out, in} : std::vector<int64_t>{in, out};
        TensorPtr Wt;
        if (w_bf16) {
            Wt = std::make_shared<Tensor>(wshape, kBFloat16, kCPU);
            for (int64_t i = 0; i < in * out; ++i) Wt->data<uint16_t>()[i] = float32_to_bf16_bits(W[i]);
        } else {
            Wt = from_host(W, wshape, false);
        }
        TensorPtr bt = bias ? from_host(bias, {out}, false) : nullptr;
        LoRALinear layer(Wt, bt);
        std::vector<TensorPtr> As, Bs;
        const float* Ap = A_all;
        const float* Bp = B_all;
        for (int i = 0; i < n; ++i) {
            const int64_t* m = meta + 5 * i;
            const int64_t r = m[0], cols = m[2];
            As.push_back(from_host(Ap, m[3] ? std::vector<int64_t>{r, in} : std::vector<int64_t>{in, r}, true));
            Bs.push_back(from_host(Bp, m[4] ? std::vector<int64_t>{cols, r} : std::vector<int64_t>{r, cols}, true));
            layer.attach_lora(As.back(), Bs.back(), scale[i], (int)m[1], (int)cols);
            Ap += in * r;
            Bp += r * cols;
        }
        auto xt = from_host(x, {1, N, in}, dy != nullptr);
        auto yt = layer.forward(xt);
        to_host(yt, y);
        if (dy) {
            autograd::Engine::instance().run_backward({yt}, {from_host(dy, {1, N, out}, false)});
            if (dx) to_host(xt->grad(), dx);
            float* dA = dA_all;
            float* dB = dB_all;
            for (int i = 0; i < n; ++i) {
                const int64_t r = meta[5 * i], cols = meta[5 * i + 2];
                if (has_grad) has_grad[i] = As[i]->grad() != nullptr;
                to_host(As[i]->grad(), dA);
                to_host(Bs[i]->grad(), dB);
                dA += in * r;
                dB += r * cols;
            }
        }
        autograd::Engine::instance().clear_graph();
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "[mftref_lora] " << e.what() << std::endl;
        autograd::Engine::instance().clear_graph();
        return -1;
    }
}

// LoRALinear::merge_to_base (nn/lora_linear.cpp:446-460) on W [in, out]
// (fp32, or bf16 with w_bf16: values in and out as floats).
int mftref_lora_merge(float* W, int w_bf16, int64_t in, int64_t out, int n, const int64_t* meta, const float* scale,
                      const float* A_all, const float* B_all) {
    try {
        TensorPtr Wt;
        if (w_bf16) {
            Wt = std::make_shared<Tensor>(std::vector<int64_t>{in, out}, kBFloat16, kCPU);
            for (int64_t i = 0; i < in * out; ++i) Wt->data<uint16_t>()[i] = float32_to_bf16_bits(W[i]);
        } else {
            Wt = from_host(W, {in, out}, false);
        }
        LoRALinear layer(Wt);
        const float* Ap = A_all;
        const float* Bp = B_all;
        for (int i = 0; i < n; ++i) {
            const int64_t* m = meta + 5 * i;
            const int64_t r = m[0], cols = m[2];
            layer.attach_lora(from_host(Ap, m[3] ? std::vector<int64_t>{r, in} : std::vector<int64_t>{in, r}, false),
                              from_host(Bp, m[4] ? std::vector<int64_t>{cols, r} : std::vector<int64_t>{r, cols}, false),
                              scale[i], (int)m[1], (int)cols);
            Ap += in * r;
            Bp += r * cols;
        }
        layer.merge_to_base();
        for (int64_t i = 0; i < in * out; ++i)
            W[i] = w_bf16 ? bf16_bits_to_float32(Wt->data<uint16_t>()[i]) : Wt->data<float>()[i];
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "[mftref_lora_merge] " << e.what() << std::endl;
        return -1;
    }
}

}  // extern "C"
