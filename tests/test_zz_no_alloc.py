"""mft_attn_bwd_noalloc (the backward whose workspace is the library's own
device array) against mft_attn_bwd with a caller workspace: bit-identical
dQ/dK/dV on consecutive calls, each later call smaller than the one before, so
every later call runs over scratch that still holds the previous call's
partial tiles.  Run through the C ABI on the GPU."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from mobilefinetuner_amd import attention as A
from mobilefinetuner_amd import capi

pytestmark = pytest.mark.gpu

# (B, Hq, Hkv, S, D, dtype, window, kv_len): largest first.  The first needs
# about 100 MiB of the 128 MiB scratch (the C5 shape), the others less.
CALLS = [
    (1, 4, 1, 4096, 256, torch.bfloat16, 0, None),
    (1, 8, 2, 2048, 128, torch.bfloat16, 0, None),
    (2, 4, 2, 320, 64, torch.bfloat16, 96, (320, 201)),
    (1, 2, 1, 192, 64, torch.float32, 0, None),
]


def _inputs(B, Hq, Hkv, S, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    mk = lambda h: torch.randn(B, h, S, D, generator=g).to("cuda", dtype)
    return mk(Hq), mk(Hkv), mk(Hkv), mk(Hq)


def _both(B, Hq, Hkv, S, D, dtype, window, lengths, seed):
    q, k, v, dO = _inputs(B, Hq, Hkv, S, D, dtype, seed)
    kv_len = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device="cuda")
    o, lse = A.attention_forward(q, k, v, -1.0, True, window=window, kv_len=kv_len)
    ref = A.attention_backward(q, k, v, o, dO, lse, -1.0, True, window=window, kv_len=kv_len)
    grads = [torch.full_like(t, float("nan"), dtype=torch.float32) for t in (q, k, v)]
    d = A._desc(q, k, -1.0, True, window, kv_len)
    capi.attn_bwd_noalloc(d, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), dO.data_ptr(),
                          lse.data_ptr(), *(g.data_ptr() for g in grads), A._stream())
    torch.cuda.synchronize()
    return ref, grads


def test_noalloc_matches_workspace_backward_on_consecutive_calls():
    prev = None
    for i, (B, Hq, Hkv, S, D, dtype, window, lengths) in enumerate(CALLS):
        d = capi.desc(B, Hq, Hkv, S, D, -1.0, True, A._DT[dtype], window, None)
        need = capi.workspace_size(d)[1]
        assert need <= capi.NOALLOC_SCRATCH_BYTES
        if prev is not None:
            assert need < prev  # each call smaller than the last: stale scratch above and below
        prev = need
        print(f"noalloc call {i}: B={B} Hq={Hq} Hkv={Hkv} S={S} D={D} {dtype} window={window} "
              f"kv_len={lengths} workspace={need}", flush=True)
        ref, got = _both(B, Hq, Hkv, S, D, dtype, window, lengths, seed=100 + i)
        for name, r, g in zip(("dq", "dk", "dv"), ref, got):
            rn, gn = r.cpu().numpy(), g.cpu().numpy()
            assert np.isfinite(gn).all(), name
            assert np.array_equal(rn.view(np.uint32), gn.view(np.uint32)), \
                f"call {i} {name}: max |diff| {np.abs(rn - gn).max()}"


def test_noalloc_rejects_shape_beyond_scratch():
    d = capi.desc(128, 32, 8, 8192, 64, -1.0, True, capi.MFT_BF16, 0, None)
    assert capi.workspace_size(d)[1] > capi.NOALLOC_SCRATCH_BYTES
    with pytest.raises(RuntimeError, match="fixed scratch"):
        capi.attn_bwd_noalloc(d, *([16] * 9), None)
