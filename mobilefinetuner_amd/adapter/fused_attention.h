// Extension of the finetune_ops drop-in (memory_efficient_attention_hip.cpp)
// for the model graphs' own attention composite.
//
// GemmaModel::apply_attention (graph/gemma_model.cpp:481-505) and
// QwenModel::attention (graph/qwen_model.cpp:302-318) build
//   repeat_kv_heads(k), repeat_kv_heads(v)
//   scores = mul(matmul(q, transpose(k)), scale)
//   scores = add(scores, base_mask)   // causal, or Gemma's sliding window
//   scores = add(scores, pad_mask)    // [B,1,1,S] from attention_mask
//   context = matmul(softmax(scores, -1), v)
// memory_efficient_attention_masked is that composite as one op on the MI355X
// kernels, taking the un-repeated k, v.  Replacing the block above with
//   context = ops::memory_efficient_attention_masked(q, k, v, base_mask, pad_mask, cfg)
// (cfg.scale = the composite's scale) is the whole call-site change.
#pragma once

#include "memory_efficient_attention.h"

namespace ops {

// q [B,Hq,S,D]; k, v [B,Hkv,S,D] with Hkv | Hq; float32 or bfloat16 host
// tensors.  base_mask: nullptr or an fp32 [S,S] additive mask; pad_mask:
// nullptr or an fp32 [B,1,1,S] additive mask.  A causal / sliding base
// (create_causal_mask, build_sliding_mask) with right padding (0 on the first
// len[b] keys, <= -1e9 after) runs the fast kernels; any other masks run the
// kernels' mask mode (scores + base_mask, then + pad_mask).  Scale:
// cfg.scale > 0, else 1/sqrt(D); cfg.use_causal_mask is not used (the masks
// say it).  Returns fp32 [B,Hq,S,D]; with grad, one autograd node whose
// backward returns {dQ, dK, dV} (dK, dV summed over each kv head's query
// heads).
TensorPtr memory_efficient_attention_masked(const TensorPtr& q, const TensorPtr& k, const TensorPtr& v,
                                            const TensorPtr& base_mask, const TensorPtr& pad_mask,
                                            const MemoryEfficientAttentionConfig& config = {});

}  // namespace ops
