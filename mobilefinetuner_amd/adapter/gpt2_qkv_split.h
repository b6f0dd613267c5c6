// A flag for GPT-2's Q/K/V split in the drop-in build's model graph.
//
// GPT2Model::forward_block splits the fused c_attn projection [B, S, 3C] by
// memcpy into three fresh tensors (graph/gpt2_model.cpp:559-581).  Those
// tensors carry no autograd edge back to the projection, so the attention's
// gradient never reaches c_attn (its weights or LoRA adapters), on the
// reference's CPU path and on the drop-in alike.  With the flag set, the
// routed graph (route_attention.py) splits with the reference's own
// Tensor::slice instead (core/tensor.cpp:400-480, SliceBackward at
// core/backward_functions.cpp:572-606): the same values, with the gradient
// flowing into the projection.  Off by default, so the graph keeps the
// reference's behaviour unless a caller opts in: set_gpt2_qkv_grad(true), or
// MFT_GPT2_QKV_GRAD=1 in the environment at first use.
#ifndef MFT_GPT2_QKV_SPLIT_H
#define MFT_GPT2_QKV_SPLIT_H

#include <cstdlib>

namespace ops {

inline bool& gpt2_qkv_grad_flag() {
    static bool on = [] {
        const char* e = std::getenv("MFT_GPT2_QKV_GRAD");
        return e != nullptr && e[0] == '1';
    }();
    return on;
}

// Whether the routed GPT-2 graph splits Q/K/V with autograd.
inline bool gpt2_qkv_grad() { return gpt2_qkv_grad_flag(); }

inline void set_gpt2_qkv_grad(bool on) { gpt2_qkv_grad_flag() = on; }

}  // namespace ops

#endif  // MFT_GPT2_QKV_SPLIT_H
