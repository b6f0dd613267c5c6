"""The backward run stage by stage through mft_attn_bwd_stage (DELTA, DKDV,
DQ, REDUCE as four calls) against one mft_attn_bwd call: dQ, dK and dV bit
for bit.  The stages share the call's plan and workspace, so each stage must
leave exactly what the next one reads: the row terms (DELTA), the dK/dV
partial tiles and, on the stored-dS plan, the dS tiles (DKDV), the dQ partial
tiles (DQ), and REDUCE's sums.  Shapes cover the fp32 and bf16 fast paths,
whole and partial tiles, split tiles and the stored-dS plan (bf16, D = 256).
Run through the C ABI on the GPU."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from mobilefinetuner_amd import attention as A
from mobilefinetuner_amd import capi

pytestmark = pytest.mark.gpu

# (B, Hq, Hkv, S, D, dtype, causal, window)
CASES = [
    (1, 4, 1, 1024, 256, torch.bfloat16, True, 0),    # stored dS, whole tiles, split tiles
    (1, 4, 1, 1000, 256, torch.bfloat16, True, 0),    # stored dS, partial tiles
    (2, 2, 1, 448, 256, torch.bfloat16, True, 130),   # stored dS with a window
    (1, 2, 1, 384, 256, torch.bfloat16, False, 0),    # stored dS, not causal
    (2, 14, 2, 1024, 64, torch.bfloat16, True, 0),    # combined launch (D = 64)
    (1, 4, 2, 520, 128, torch.bfloat16, True, 0),     # combined launch, partial tiles
    (1, 4, 1, 512, 256, torch.float32, True, 0),      # fp32 fast path, whole tiles
    (2, 4, 4, 300, 64, torch.float32, True, 0),       # fp32 fast path, partial tiles
]


def _id(c):
    B, Hq, Hkv, S, D, dt, causal, W = c
    return f"B{B}H{Hq}KV{Hkv}S{S}D{D}-{'bf16' if dt == torch.bfloat16 else 'f32'}-{'c' if causal else 'nc'}-W{W}"


@pytest.mark.parametrize("case", CASES, ids=[_id(c) for c in CASES])
def test_stages_one_by_one_match_the_full_backward(case):
    B, Hq, Hkv, S, D, dtype, causal, window = case
    print(f"[case] {_id(case)}", flush=True)
    g = torch.Generator().manual_seed(S + D + Hq)
    mk = lambda h, s=1.0: (torch.randn(B, h, S, D, generator=g) * s).to("cuda", dtype)
    q, k, v, dO = mk(Hq), mk(Hkv), mk(Hkv), mk(Hq, 0.3)
    o, lse = A.attention_forward(q, k, v, -1.0, causal, window=window)
    d = A._desc(q, k, -1.0, causal, window)
    ws = torch.empty(max(capi.workspace_size(d)[1], 1), dtype=torch.uint8, device="cuda")
    st = A._stream()

    def run(stage_masks):
        grads = [torch.full_like(t, float("nan"), dtype=torch.float32) for t in (q, k, v)]
        for m in stage_masks:
            capi.attn_bwd_stage(d, m, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), dO.data_ptr(),
                                lse.data_ptr(), *(t.data_ptr() for t in grads), ws.data_ptr(), st)
        torch.cuda.synchronize()
        return [t.cpu().numpy() for t in grads]

    full = run([capi.MFT_BWD_ALL])
    staged = run([capi.MFT_BWD_DELTA, capi.MFT_BWD_DKDV, capi.MFT_BWD_DQ, capi.MFT_BWD_REDUCE])
    for name, a_, b_ in zip(("dq", "dk", "dv"), full, staged):
        assert np.isfinite(a_).all(), name
        assert np.array_equal(a_.view(np.uint32), b_.view(np.uint32)), \
            f"{name}: max |diff| {np.abs(a_ - b_).max()}"
