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


_MEMORY_PROBE = r'''
import ctypes, sys
sys.path.insert(0, sys.argv[1])
import torch
from mobilefinetuner_amd import attention as A, capi
dev = torch.device("cuda:0")
B, H, S, D = 1, 2, 256, 64
mk = lambda: torch.randn(B, H, S, D, device=dev, dtype=torch.bfloat16)
q, k, v, dO = mk(), mk(), mk(), mk()
o, lse = torch.empty_like(q), torch.empty(B, H, S, device=dev)
dq, dk, dv = (torch.empty(B, H, S, D, device=dev) for _ in range(3))
ws = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
torch.cuda.synchronize()
f0 = torch.cuda.mem_get_info()[0]
d = A._desc(q, k, 0.125, True, 0, None)
sp = torch.cuda.current_stream().cuda_stream
L = capi.lib()
capi.check(L.mft_attn_fwd(ctypes.byref(d), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                          ws.data_ptr(), sp))
capi.check(L.mft_attn_bwd(ctypes.byref(d), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), dO.data_ptr(),
                          lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), sp))
torch.cuda.synchronize()
f1 = torch.cuda.mem_get_info()[0]
capi.attn_bwd_noalloc(d, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), dO.data_ptr(), lse.data_ptr(),
                      dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), sp)
torch.cuda.synchronize()
f2 = torch.cuda.mem_get_info()[0]
print("MIB", (f0 - f1) / 2**20, (f1 - f2) / 2**20, flush=True)
'''


def test_scratch_is_taken_only_by_the_first_noalloc_call():
    """In a fresh process, the regular forward and backward leave the 128 MiB
    array's code object unloaded (deferred loading); the first
    mft_attn_bwd_noalloc call on the GPU loads it."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ)
    env.pop("HIP_ENABLE_DEFERRED_LOADING", None)
    res = subprocess.run([sys.executable, "-c", _MEMORY_PROBE, root], capture_output=True, text=True, timeout=110,
                         env=env)
    print(res.stdout[-500:], res.stderr[-1500:], flush=True)
    assert res.returncode == 0
    regular, first_noalloc = (float(x) for x in next(l for l in res.stdout.splitlines() if l.startswith("MIB"))
                              .split()[1:])
    assert regular < 64, regular
    assert first_noalloc >= 128, first_noalloc
