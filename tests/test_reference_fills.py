"""The reference's own hot-path test fills through the HIP kernels, and the
standalone repeat_kv entry points bit for bit.

tests/golden/tiny.npz holds the exact inputs and the reference's outputs of
optim/test_qkt_softmax_grad.cpp:26-59, optim/test_repeat_kv_softmax_grad.cpp:
26-79, optim/test_attention_single_layer_backward.cpp:50-108 and
core/test_memory_efficient_attention_grad.cpp (S = 3..8, D = 3..8, causal and
not, their scales), plus small GQA cases, all written by the reference
operators compiled from their sources (tests/golden/make_golden.py).  The
fp32 HIP path must meet the fp32 bar (max-rel 1e-4) against those outputs.

mft_repeat_kv_fwd / mft_repeat_kv_bwd replace repeat_kv_heads and
RepeatKVHeadsBackward (core/ops.cpp:2260-2335,
core/backward_functions.cpp:693-726): the forward is a copy and the backward
sums ((0 + g_0) + g_1) + ... in fp32, so both are compared bit for bit with
the oracle (itself pinned bit for bit to the live reference), on every copy
width the forward picks (16-, 4- and 2-byte units).
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "tiny.npz")


def _names():
    return [str(n) for n in np.load(GOLDEN, allow_pickle=False)["names"]]


@pytest.mark.parametrize("name", _names())
def test_reference_fill_through_hip(orc, dev, name):
    from gpu_util import TOL, run_hip
    z = np.load(GOLDEN, allow_pickle=False)
    q, k, v, dO = (z[f"{name}/{t}"] for t in ("q", "k", "v", "dO"))
    scale, causal = float(z[f"{name}/scale"]), bool(int(z[f"{name}/causal"]))
    print(f"[case] {name} q{q.shape} k{k.shape} scale={scale} causal={causal}", flush=True)
    got = run_hip(q, k, v, dO, "f32", scale, causal, dev)
    for t in ("o", "dq", "dk", "dv"):
        e = orc.max_rel(got[t], z[f"{name}/{t}"])
        print(f"[errs] {name} {t}: {e:.2e}", flush=True)
        assert e <= TOL["f32"], f"{name} {t}: max-rel {e:.3e}"


# (B, Hkv, S, D, r, dtype): the forward's 16-byte, 4-byte and 2-byte copy
# units, groups of 1, 2, 4 and 7.
REPEAT = [
    (2, 3, 16, 64, 4, "f32"),   # 16-byte units
    (1, 2, 3, 5, 2, "f32"),     # 60-byte blocks: 4-byte units
    (2, 1, 9, 16, 7, "f32"),
    (1, 2, 4, 6, 4, "bf16"),    # 48-byte blocks: 16-byte units
    (1, 3, 3, 5, 2, "bf16"),    # 30-byte blocks: 2-byte units
    (2, 2, 5, 6, 7, "bf16"),    # 60-byte blocks: 4-byte units
    (1, 1, 33, 256, 1, "bf16"),
    (1, 2, 17, 64, 1, "f32"),
]


@pytest.mark.parametrize("B,Hkv,S,D,r,dtype", REPEAT)
def test_repeat_kv_bit_exact(orc, dev, B, Hkv, S, D, r, dtype):
    import torch
    from mobilefinetuner_amd import attention as A
    print(f"[case] repeat_kv B={B} Hkv={Hkv} S={S} D={D} r={r} {dtype}", flush=True)
    kv = orc.normal(B * Hkv * S * D, 11 + D, 0).reshape(B, Hkv, S, D)
    if dtype == "bf16":
        kv = orc.round_bf16(kv)
    g = orc.normal(B * Hkv * r * S * D, 11 + D, 1).reshape(B, Hkv * r, S, D)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    out = A.repeat_kv(torch.from_numpy(kv).to(dev).to(tdt), r)
    dkv = A.repeat_kv_backward(torch.from_numpy(g).to(dev), r)
    torch.cuda.synchronize()
    want = orc.repeat_kv(kv, r)
    got = out.float().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    want_b = orc.repeat_kv_backward(g, r)
    assert np.array_equal(dkv.cpu().numpy().view(np.uint32), want_b.view(np.uint32))
