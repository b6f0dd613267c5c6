"""GPU parity of the mask mode (general additive masks, mft_mask) against the
CPU oracle of the reference with the same masks.

The reference adds any mask to the scaled scores: the grad path's composite
(core/memory_efficient_attention.cpp:23-43, ops::add with broadcasting) and
the no-grad operator, which first replaces the scores above the diagonal by
-1e10 when use_causal_mask is set (:160-172).  The kernels take up to two
masks with broadcast strides; causal = 0 is the composite rule and causal = 1
the no-grad operator's.  Masks include -1e10 entries, a row masked
everywhere (uniform softmax), left padding (not a suffix), per-head biases and
two masks added in order.  lse is the pair (row max, ln sum).

Tolerance as in test_attn_parity.py: max-rel 1e-4 (fp32), 2e-2 (bf16).
"""
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _masks(kind, B, Hq, S, seed):
    rng = np.random.default_rng(seed)
    if kind == "ss":  # any [S,S] mask: random values, -1e10 holes, one row masked everywhere
        m = rng.normal(size=(S, S)).astype(np.float32)
        m[rng.random((S, S)) < 0.25] = -1e10
        m[S // 3, :] = -1e10
        return [m]
    if kind == "leftpad":  # [B,1,1,S] padding on the left (not a suffix)
        m = np.zeros((B, 1, 1, S), np.float32)
        for b in range(B):
            m[b, 0, 0, : (7 * b + 5) % S] = -1e10
        return [m]
    if kind == "bss":  # [B,1,S,S] per-batch masks, one batch's row masked by -1e9
        m = (0.5 * rng.normal(size=(B, 1, S, S))).astype(np.float32)
        m[:, :, 3, :] = -1e9
        return [m]
    if kind == "alibi":  # [1,Hq,1,S] per-head linear bias
        slopes = 2.0 ** (-np.arange(1, Hq + 1))
        return [(-slopes[None, :, None, None] * np.arange(S)[None, None, None, :]).astype(np.float32)]
    if kind == "two":  # [S,S] then [B,1,1,S], added in that order
        m0 = rng.normal(size=(S, S)).astype(np.float32)
        m0[np.triu_indices(S, 1)] = -1e10
        m1 = np.zeros((B, 1, 1, S), np.float32)
        m1[-1, 0, 0, S // 2:] = -1e10
        return [m0, m1]
    raise ValueError(kind)


# (B, Hq, Hkv, S, D, dtype, causal, mask kind)
CASES = [
    (2, 4, 2, 80, 64, "bf16", False, "ss"),
    (2, 4, 2, 80, 64, "f32", True, "ss"),
    (1, 4, 1, 128, 256, "bf16", False, "two"),
    (2, 2, 1, 100, 40, "f32", False, "leftpad"),
    (2, 2, 2, 96, 128, "bf16", True, "leftpad"),
    (2, 2, 1, 70, 64, "f32", False, "bss"),
    (1, 4, 2, 64, 96, "bf16", False, "alibi"),
    (1, 2, 2, 130, 256, "f32", True, "alibi"),
]


def _id(c):
    B, Hq, Hkv, S, D, dt, causal, kind = c
    return f"B{B}H{Hq}KV{Hkv}S{S}D{D}-{dt}-{'c' if causal else 'nc'}-{kind}"


@pytest.mark.parametrize("case", CASES, ids=[_id(c) for c in CASES])
def test_mask_mode_fwd_bwd_matches_oracle(orc, dev, case):
    import torch

    from gpu_util import TOL, to_dev
    from mobilefinetuner_amd import attention as A
    B, Hq, Hkv, S, D, dtype, causal, kind = case
    q, k, v, dO = orc.make_inputs(B, Hq, Hkv, S, D, 900 + S + D, dtype, do_sigma=0.5)
    scale = 1.0 / math.sqrt(D)
    masks = _masks(kind, B, Hq, S, S + D)
    ref = orc.composite_masks(q, k, v, dO, scale=scale, mode=1 if causal else 0, masks=masks, want_lse=True)

    tq, tk, tv, tg = (to_dev(x, dtype, dev) for x in (q, k, v, dO))
    tm = [torch.from_numpy(m).to(dev) for m in masks]
    o, lse = A.attention_forward(tq, tk, tv, scale, causal, masks=tm)
    dq, dk, dv = A.attention_backward(tq, tk, tv, o, tg, lse, scale, causal, masks=tm)
    torch.cuda.synchronize()
    got = dict(o=o.float().cpu().numpy(), dq=dq.cpu().numpy(), dk=dk.cpu().numpy(), dv=dv.cpu().numpy())
    tol = TOL[dtype]
    for n in ("o", "dq", "dk", "dv"):
        err = orc.max_rel(got[n], ref[n])
        assert err <= tol, f"{n}: max-rel {err:.3e} > {tol}"
    # row terms: the row max (absolute, scaled by the score range) and ln sum
    l_got, l_ref = lse.cpu().numpy(), ref["lse2"]
    assert np.allclose(l_got[..., 0], l_ref[..., 0], rtol=1e-6, atol=tol * 10), "row max"
    assert np.allclose(l_got[..., 1], l_ref[..., 1], atol=tol * 10), "ln sum"


def test_mask_mode_uniform_rows_exact(orc, dev):
    """A row masked everywhere by one huge value has a uniform softmax: O is
    the mean of V over all keys and its gradients follow (P = 1/S from the
    row-term pair, which a single fp32 lse could not carry)."""
    import torch

    from gpu_util import to_dev
    from mobilefinetuner_amd import attention as A
    B, Hq, Hkv, S, D = 1, 2, 1, 64, 64
    q, k, v, dO = orc.make_inputs(B, Hq, Hkv, S, D, 31, "f32", do_sigma=1.0)
    m = np.full((S, S), -1e10, np.float32)
    ref = orc.composite_masks(q, k, v, dO, scale=0.125, mode=0, masks=[m])
    assert np.allclose(ref["o"][0, 0], v[0, 0].mean(axis=0), atol=1e-6)  # the oracle: uniform rows
    tq, tk, tv, tg = (to_dev(x, "f32", dev) for x in (q, k, v, dO))
    tm = [torch.from_numpy(m).to(dev)]
    o, lse = A.attention_forward(tq, tk, tv, 0.125, False, masks=tm)
    dq, dk, dv = A.attention_backward(tq, tk, tv, o, tg, lse, 0.125, False, masks=tm)
    torch.cuda.synchronize()
    for n, t in (("o", o), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert orc.max_rel(t.cpu().numpy(), ref[n]) <= 1e-4, n


def test_mask_mode_rejects_window_and_kv_len(dev):
    import torch

    from mobilefinetuner_amd import attention as A
    from mobilefinetuner_amd.capi import MftError
    q = torch.randn(1, 2, 64, 64, device=dev)
    m = torch.zeros(64, 64, device=dev)
    with pytest.raises(MftError):
        A.attention_forward(q, q, q, 0.125, True, window=16, masks=[m])
    with pytest.raises(MftError):
        A.attention_forward(q, q, q, 0.125, True, kv_len=torch.full((1,), 10, dtype=torch.int32, device=dev),
                            masks=[m])


@pytest.mark.parametrize("cfg", ["c4", "c5"])
def test_mask_mode_at_full_size_equals_the_fast_kernels(orc, dev, cfg):
    """At the BASELINE shapes, where the CPU oracle would take minutes: the mask
    mode with an explicit [S,S] causal mask (0 on and below the diagonal, -1e10
    above, the reference's create_causal_mask) and the causal flag off gives
    the causal fast kernels' O and gradients; adding an all-zero [B,1,1,S] mask
    as the second mask changes nothing.  Same bf16 bar as the parity tests,
    elementwise against the fast path (both round the same fp32 values)."""
    import torch

    from gpu_util import TOL, to_dev
    from mobilefinetuner_amd import attention as A
    c = orc.CONFIGS[cfg]
    B, Hq, Hkv, S, D = c["B"], c["Hq"], c["Hkv"], c["S"], c["D"]
    print(f"[case] {cfg} B{B} Hq{Hq} Hkv{Hkv} S{S} D{D}", flush=True)
    q, k, v, dO = orc.make_inputs(B, Hq, Hkv, S, D, 77, "bf16", do_sigma=0.1)
    tq, tk, tv, tg = (to_dev(x, "bf16", dev) for x in (q, k, v, dO))
    causal = torch.zeros(S, S, device=dev)
    causal.masked_fill_(torch.ones(S, S, device=dev, dtype=torch.bool).triu(1), -1e10)
    zero_pad = torch.zeros(B, 1, 1, S, device=dev)
    o0, lse0 = A.attention_forward(tq, tk, tv, c["scale"], True)
    g0 = A.attention_backward(tq, tk, tv, o0, tg, lse0, c["scale"], True)
    for masks in ([causal], [causal, zero_pad]):
        o1, lse1 = A.attention_forward(tq, tk, tv, c["scale"], False, masks=masks)
        g1 = A.attention_backward(tq, tk, tv, o1, tg, lse1, c["scale"], False, masks=masks)
        torch.cuda.synchronize()
        for n, a, b in (("o", o1, o0), ("dq", g1[0], g0[0]), ("dk", g1[1], g0[1]), ("dv", g1[2], g0[2])):
            err = orc.max_rel(a.float().cpu().numpy(), b.float().cpu().numpy())
            print(f"[errs] {len(masks)} masks {n} {err:.3e}", flush=True)
            assert err <= TOL["bf16"], (n, err)
        # the row terms give the same log-sum-exp: row max + ln(sum) = lse
        assert torch.allclose(lse1[..., 0] + lse1[..., 1], lse0, rtol=1e-4, atol=1e-3), "lse"
