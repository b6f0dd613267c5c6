#!/usr/bin/env python3
"""Generate the drop-in build's Gemma and Qwen model graphs with their
attention composite routed through ops::memory_efficient_attention_masked,
and its GPT-2 graph with a flag for an autograd-preserving Q/K/V split.

    python route_attention.py <REF_DIR>/finetune_ops/graph <OUT_DIR>

GemmaModel's block (graph/gemma_model.cpp:481-505) and QwenModel's block
(graph/qwen_model.cpp:301-318) build repeat_kv_heads -> transpose -> matmul
-> mul(scale) -> add(masks) -> softmax -> matmul.  This script reads each
file where it lies, replaces exactly that block (located by its first and
last statements; it fails loudly if either is missing or ambiguous) with one
call of the fused op on the un-repeated k and v, and writes the result to
OUT_DIR for the drop-in Makefile to compile.  Everything else in the files,
and the files themselves, stay as they are: the output is build output, kept
out of the repository like the objects made from it.

Qwen applies RoPE after repeating K; RoPE acts on every head alike, so the
routed graph applies the same RoPE lines to the un-repeated K (its values
per head are the same) and lets the fused op index each query head's kv
head.  The debug dumps of scores/probs inside Gemma's block go with it: the
fused op never materialises them (as the GPT-2 graph's own
memory-efficient branch, graph/gpt2_model.cpp:616-625).

GPT-2 already calls memory_efficient_attention; its Q/K/V split by memcpy
(graph/gpt2_model.cpp:559-581) drops the autograd edge to c_attn.  The
routed copy keeps that split and adds, behind ops::gpt2_qkv_grad()
(gpt2_qkv_split.h, off by default), the split by the reference's own
Tensor::slice, which keeps it.
"""
from __future__ import annotations

import os
import sys

INCLUDE = '#include "fused_attention.h"  // drop-in build: memory_efficient_attention_masked\n'


def _span(lines, first, last, name):
    starts = [i for i, l in enumerate(lines) if first in l]
    ends = [i for i, l in enumerate(lines) if last in l]
    if len(starts) != 1 or len(ends) != 1 or ends[0] <= starts[0]:
        raise SystemExit(f"route_attention: cannot locate the attention block of {name} "
                         f"({len(starts)} start / {len(ends)} end matches)")
    return starts[0], ends[0]


def _add_include(lines, name):
    for i, l in enumerate(lines):
        if l.startswith('#include "../core/ops.h"'):
            return lines[:i + 1] + [INCLUDE] + lines[i + 1:]
    raise SystemExit(f"route_attention: no ops.h include in {name}")


def route_gemma(src):
    lines = src.splitlines(keepends=True)
    a, b = _span(lines, "repeat_kv_heads(k, n_head / kv_heads)", "matmul(probs, v_full)", "gemma_model.cpp")
    indent = lines[a][:len(lines[a]) - len(lines[a].lstrip())]
    body = [
        f"{indent}// drop-in build: the composite as one fused op on the un-repeated k, v\n",
        f"{indent}MemoryEfficientAttentionConfig mft_attn_cfg;\n",
        f"{indent}mft_attn_cfg.scale = std::pow(config_.query_pre_attn_scalar, -0.5f);\n",
        f"{indent}auto context = memory_efficient_attention_masked(q, k, v, base_mask, pad_mask, mft_attn_cfg);\n",
    ]
    return "".join(_add_include(lines[:a] + body + lines[b + 1:], "gemma_model.cpp"))


def route_qwen(src):
    lines = src.splitlines(keepends=True)
    a, b = _span(lines, "// GQA: repeat kv heads to match H", "auto ctx = matmul(probs, v)", "qwen_model.cpp")
    rope = [l for l in lines[a:b + 1] if "apply_rope(" in l]
    if len(rope) != 2:
        raise SystemExit(f"route_attention: expected the q and k RoPE lines in qwen_model.cpp, found {len(rope)}")
    indent = lines[a][:len(lines[a]) - len(lines[a].lstrip())]
    body = [f"{indent}// drop-in build: RoPE on the un-repeated k, then the composite as one fused op\n"] + rope + [
        f"{indent}MemoryEfficientAttentionConfig mft_attn_cfg;\n",
        f"{indent}mft_attn_cfg.scale = 1.0f / std::sqrt(static_cast<float>(Hd));\n",
        f"{indent}auto ctx = memory_efficient_attention_masked(q, k, v, causal_mask, pad_mask, mft_attn_cfg);\n",
    ]
    return "".join(_add_include(lines[:a] + body + lines[b + 1:], "qwen_model.cpp"))


def route_gpt2(src):
    lines = src.splitlines(keepends=True)
    a, b = _span(lines, "const float* qkv_data = qkv->data<float>();", "std::memcpy(v_ptr, qkv_ptr + 2 * C",
                 "gpt2_model.cpp")
    # the split ends with the two loops' closing braces
    if [l.strip() for l in lines[b + 1:b + 3]] != ["}", "}"]:
        raise SystemExit("route_attention: unexpected end of the Q/K/V split in gpt2_model.cpp")
    b += 2
    decl = [l for l in lines[a:b + 1] if "= zeros({B, S, C}, kFloat32, kCPU);" in l]
    if len(decl) != 3:
        raise SystemExit("route_attention: expected the q, k, v allocations in gpt2_model.cpp's split")
    indent = lines[a][:len(lines[a]) - len(lines[a].lstrip())]
    inner = [("    " + l if l.strip() else l).replace("auto q = zeros", "q = zeros").replace(
        "auto k = zeros", "k = zeros").replace("auto v = zeros", "v = zeros") for l in lines[a:b + 1]]
    body = [
        f"{indent}// drop-in build: with ops::gpt2_qkv_grad() the split keeps the autograd edge to c_attn\n",
        f"{indent}TensorPtr q, k, v;\n",
        f"{indent}if (gpt2_qkv_grad()) {{\n",
        f"{indent}    q = qkv->slice(2, 0, C);\n",
        f"{indent}    k = qkv->slice(2, C, 2 * C);\n",
        f"{indent}    v = qkv->slice(2, 2 * C, 3 * C);\n",
        f"{indent}}} else {{\n",
    ] + inner + [f"{indent}}}\n"]
    out = lines[:a] + body + lines[b + 1:]
    for i, l in enumerate(out):
        if l.startswith('#include "../core/ops.h"'):
            return "".join(out[:i + 1] + ['#include "gpt2_qkv_split.h"  // drop-in build: the Q/K/V split flag\n']
                           + out[i + 1:])
    raise SystemExit("route_attention: no ops.h include in gpt2_model.cpp")


def main():
    if len(sys.argv) != 3:
        raise SystemExit(__doc__)
    graph, out = sys.argv[1], sys.argv[2]
    os.makedirs(out, exist_ok=True)
    for name, fn in (("gemma_model.cpp", route_gemma), ("qwen_model.cpp", route_qwen), ("gpt2_model.cpp", route_gpt2)):
        with open(os.path.join(graph, name)) as fh:
            text = fn(fh.read())
        with open(os.path.join(out, name), "w") as fh:
            fh.write(f"// Generated by mobilefinetuner_amd/adapter/route_attention.py from {os.path.join(graph, name)}\n")
            fh.write(text)


if __name__ == "__main__":
    main()
