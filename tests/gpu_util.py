"""Shared helpers of the GPU parity tests: run the HIP path through the C ABI
on oracle-generated inputs and return numpy results."""
from __future__ import annotations

import numpy as np
import torch

from mobilefinetuner_amd import attention as A

TOL = {"f32": 1e-4, "bf16": 2e-2}  # max-rel vs the fp32 reference


def to_dev(x: np.ndarray, dtype: str, dev) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(dev)
    return t.to(torch.bfloat16) if dtype == "bf16" else t


def run_hip(q, k, v, dO, dtype, scale, causal, dev, backward=True, window=0, lengths=None):
    """Forward (+ backward) of the fused kernels; returns dict of numpy fp32 arrays.
    window: causal sliding window (0 = none); lengths: valid keys per batch."""
    tq, tk, tv = (to_dev(x, dtype, dev) for x in (q, k, v))
    kv_len = None if lengths is None else torch.tensor(np.asarray(lengths, np.int32), device=dev)
    o, lse = A.attention_forward(tq, tk, tv, scale, causal, window=window, kv_len=kv_len)
    out = {"o": o.float().cpu().numpy(), "lse": lse.cpu().numpy()}
    if backward:
        tg = to_dev(dO, dtype, dev)
        dq, dk, dv = A.attention_backward(tq, tk, tv, o, tg, lse, scale, causal, window=window, kv_len=kv_len)
        torch.cuda.synchronize()
        out.update(dq=dq.cpu().numpy(), dk=dk.cpu().numpy(), dv=dv.cpu().numpy())
    torch.cuda.synchronize()
    return out
