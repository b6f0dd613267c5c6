"""MI355X-native fused causal GQA attention for MobileFineTuner's finetune_ops.

The product is ``lib/libmft_attn.so``: hand-written gfx950 HIP kernels
(``csrc/``) behind the C ABI of ``include/mft/attention.h`` (with
``prologue.h``, ``lm_loss.h`` and ``lora.h`` beside it). ``adapter/`` holds
the C++ drop-in that re-implements the reference's
``memory_efficient_attention`` (and the LM loss and LoRA layer) on that ABI.
``build`` compiles the library. ``capi`` is the ctypes binding of the C ABI.
``attention``, ``lm_loss`` and ``lora`` drive it with torch tensors, which
supply device memory and streams only. ``profiling`` summarises rocprofv3
output.
"""
from . import capi  # noqa: F401

__all__ = ["capi"]
