"""MI355X-native fused causal GQA attention for MobileFineTuner's finetune_ops.

The product is ``lib/libmft_attn.so`` (hand-written gfx950 HIP kernels behind
the C ABI of ``include/mft/attention.h``) and the C++ finetune_ops adapter in
``csrc/finetune_ops``.  ``capi`` is the ctypes binding of the C ABI;
``attention`` drives it with torch tensors (device memory and streams only).
"""
from . import capi  # noqa: F401

__all__ = ["capi"]
