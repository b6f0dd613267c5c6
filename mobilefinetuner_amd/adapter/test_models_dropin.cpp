// The reference's model graphs on tiny configurations, forward + Engine
// backward, printing what the GPU-vs-CPU comparison needs.
//
// Built twice by the drop-in Makefile from the same source:
//   test_models_dropin  against the drop-in (attention, LM loss and LoRA on
//                       the MI355X kernels; Gemma's and Qwen's attention
//                       blocks routed through memory_efficient_attention_masked
//                       by route_attention.py; GPT-2 with
//                       use_memory_efficient_attention);
//   test_models_ref     against the reference's own CPU operators and the
//                       unmodified Gemma and Qwen sources.
// Both take GPT-2 from route_attention.py's copy, whose Q/K/V split flag
// (gpt2_qkv_split.h) is off except in the gpt2_mha_d4_qkv_grad case; with
// it off the copy computes what the unmodified source does.
// tests/test_models_dropin.py runs both and compares the lines.
//
// Models and fills are the reference's synthetic-smoke ones
// (optim/smoke_utils.h:109-184, examples/*/src/main.cpp run_synthetic_smoke):
// vocab 64, hidden 16, the smoke initialisers, ids (1 + i) % vocab, labels
// shifted by one.  Every parameter requires grad, so the backward runs
// through attention's dQ, dK and dV.  Per case one JSON line: loss, the L2
// norm of the logits, and the L2 norm of every parameter's gradient.
#include <cmath>
#include <cstdio>
#include <random>
#include <string>
#include <vector>

#include "../graph/gemma_model.h"
#include "../graph/gpt2_model.h"
#include "../graph/qwen_model.h"
#include "autograd_engine.h"
#include "gpt2_qkv_split.h"
#include "lm_loss.h"
#include "smoke_utils.h"

using namespace ops;

namespace {

double l2(const TensorPtr& t) {
    if (!t) return 0.0;
    const float* p = t->data<float>();
    double s = 0.0;
    for (int64_t i = 0; i < t->numel(); ++i) s += double(p[i]) * double(p[i]);
    return std::sqrt(s);
}

// attention_mask [B, S]: 1 on the first lengths[b] positions, 0 after.
TensorPtr padded_mask(int B, int S, const std::vector<int>& lengths) {
    auto m = zeros({B, S}, kFloat32, kCPU);
    float* p = m->data<float>();
    for (int b = 0; b < B; ++b)
        for (int s = 0; s < S; ++s) p[b * S + s] = s < lengths[b] ? 1.0f : 0.0f;
    return m;
}

template <typename Fwd>
void run_case(const char* name, const std::vector<TensorPtr>& params, int vocab, int B, int S, Fwd fwd) {
    for (auto& p : params) p->set_requires_grad(true);
    auto ids = smoke::make_input_ids(B, S, vocab, 1);
    auto labels = smoke::make_shifted_labels(ids, vocab);
    TensorPtr logits = fwd(ids);
    TensorPtr loss = lm_cross_entropy(logits, labels, -100, "mean");
    loss->backward();
    std::printf("{\"case\": \"%s\", \"loss\": %.9g, \"logits_l2\": %.9g, \"grad_l2\": [", name,
                double(loss->data<float>()[0]), l2(logits));
    for (size_t i = 0; i < params.size(); ++i) std::printf("%s%.9g", i ? ", " : "", l2(params[i]->grad()));
    std::printf("]}\n");
    std::fflush(stdout);
    for (auto& p : params) p->zero_grad();
    autograd::Engine::instance().clear_graph();
}

}  // namespace

int main() {
    try {
        for (bool qkv_grad : {false, true}) {
            // optim/test_gpt2_lora_two_step_smoke.cpp's model (no padding:
            // GPT2Model takes the memory-efficient branch only without one).
            // With the split flag the attention's gradient reaches c_attn
            // and runs the fused backward.
            set_gpt2_qkv_grad(qkv_grad);
            GPT2Config cfg;
            cfg.vocab_size = 64;
            cfg.n_positions = 16;
            cfg.n_embd = 16;
            cfg.n_layer = 2;
            cfg.n_head = 4;
            cfg.use_memory_efficient_attention = true;
            GPT2Model model(cfg);
            std::mt19937 rng(7);
            smoke::initialize_tiny_gpt2(model, rng);
            model.tie_weights();
            run_case(qkv_grad ? "gpt2_mha_d4_qkv_grad" : "gpt2_mha_d4", model.parameters(), cfg.vocab_size, 2, 12,
                     [&](const TensorPtr& ids) { return model.forward(ids); });
            set_gpt2_qkv_grad(false);
        }
        for (int variant = 0; variant < 3; ++variant) {
            // Gemma synthetic smoke (examples/gemma_3_270m_lora_finetune):
            // 2 heads over 1 kv head, head_dim 8; sliding layers (window 4
            // < S), mixed sliding/full layers, and right padding.
            GemmaTextConfig cfg;
            cfg.vocab_size = 64;
            cfg.hidden_size = 16;
            cfg.intermediate_size = 32;
            cfg.num_hidden_layers = 2;
            cfg.num_attention_heads = 2;
            cfg.num_key_value_heads = 1;
            cfg.head_dim = 8;
            cfg.max_position_embeddings = 32;
            cfg.sliding_window = 4;
            if (variant == 0) cfg.layer_types.assign(2, "sliding_attention");
            else cfg.layer_types = {"sliding_attention", "full_attention"};
            GemmaModel model(cfg);
            std::mt19937 rng(42);
            smoke::initialize_tiny_gemma(model, rng);
            const int B = 2, S = 10;
            TensorPtr mask = variant == 2 ? padded_mask(B, S, {10, 7}) : smoke::make_attention_mask(B, S);
            const char* names[] = {"gemma_sliding", "gemma_mixed", "gemma_mixed_padded"};
            run_case(names[variant], model.parameters(), cfg.vocab_size, B, S,
                     [&](const TensorPtr& ids) { return model.forward(ids, mask); });
        }
        for (int variant = 0; variant < 2; ++variant) {
            // Qwen synthetic smoke (examples/qwen_lora_finetune): 4 heads
            // over 2 kv heads, head_dim 4; causal, then right padding.
            QwenConfig cfg;
            cfg.vocab_size = 64;
            cfg.hidden_size = 16;
            cfg.intermediate_size = 32;
            cfg.num_hidden_layers = 2;
            cfg.num_attention_heads = 4;
            cfg.num_key_value_heads = 2;
            cfg.max_position_embeddings = 32;
            cfg.eos_token_id = 0;
            QwenModel model(cfg);
            std::mt19937 rng(42);
            smoke::initialize_tiny_qwen(model, rng);
            const int B = 2, S = 9;
            TensorPtr mask = variant == 1 ? padded_mask(B, S, {9, 5}) : smoke::make_attention_mask(B, S);
            run_case(variant ? "qwen_gqa_padded" : "qwen_gqa", model.parameters(), cfg.vocab_size, B, S,
                     [&](const TensorPtr& ids) { return model.forward(ids, mask); });
        }
    } catch (const std::exception& e) {
        std::fprintf(stderr, "test_models: %s\n", e.what());
        return 1;
    }
    std::printf("[DONE]\n");
    return 0;
}
