"""GPU parity of the sliding-window and key-padding masks against the CPU
oracle of the reference composite with additive masks (scores + base mask +
pad mask, graph/gemma_model.cpp:481-505 and :272-320; qwen_model.cpp:302-353).

window > 0 is the Gemma sliding mask (key j visible to query i iff j <= i and
i - j < window); lengths[b] is the right-padded attention_mask of batch b
(1 on the first lengths[b] positions).  Rows left with no visible key (every
row when lengths[b] = 0; rows i >= lengths[b] + window - 1) take the
reference's value: a uniform softmax over the keys hidden by exactly one mask.

Tolerance as in test_attn_parity.py: max-rel 1e-4 (fp32), 2e-2 (bf16).
"""
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# (B, Hq, Hkv, S, D, dtype, causal, window, lengths)
CASES = [
    # sliding window, no padding
    (1, 4, 1, 1000, 256, "bf16", True, 128, None),
    (1, 2, 1, 700, 64, "bf16", True, 1, None),
    # D = 256 with a window that leaves the last 64-key tile of each query
    # tile invisible to its upper half (W = 65), and with window + padding
    (1, 4, 1, 704, 256, "bf16", True, 65, None),
    (2, 2, 1, 448, 256, "bf16", True, 200, [448, 333]),
    (2, 2, 1, 300, 128, "bf16", True, 64, None),
    (1, 4, 2, 520, 128, "bf16", True, 65, None),
    (1, 2, 2, 333, 96, "f32", True, 50, None),
    (1, 2, 1, 200, 256, "f32", True, 33, None),
    (1, 3, 1, 160, 40, "bf16", True, 17, None),   # general bf16 path (D not a multiple of 8)
    # key padding, causal
    (2, 4, 2, 300, 64, "bf16", True, 0, [300, 123]),
    (3, 2, 2, 129, 256, "bf16", True, 0, [1, 64, 129]),
    (2, 2, 1, 200, 48, "f32", True, 0, [77, 0]),
    # key padding, not causal (Qwen's pad mask without the causal one)
    (2, 2, 2, 200, 128, "bf16", False, 0, [50, 200]),
    (2, 2, 1, 150, 64, "f32", False, 0, [0, 7]),
    # window and padding together: rows with no visible key
    (2, 4, 1, 512, 128, "bf16", True, 96, [100, 512]),
    (1, 2, 1, 260, 256, "bf16", True, 32, [40]),
    (2, 2, 2, 190, 64, "f32", True, 20, [30, 0]),
    # fp32 whole tiles (S a multiple of 64, D = 256 / 128): the direct loads' fixed offsets
    (1, 4, 1, 512, 256, "f32", True, 100, None),
    (2, 2, 1, 256, 128, "f32", True, 0, [256, 100]),
]


def _id(c):
    B, Hq, Hkv, S, D, dt, causal, W, L = c
    return f"B{B}H{Hq}KV{Hkv}S{S}D{D}-{dt}-{'c' if causal else 'nc'}-W{W}-L{'x' if L is None else '_'.join(map(str, L))}"


def _reference(orc, q, k, v, dO, scale, causal, window, lengths):
    S = q.shape[2]
    base = orc.sliding_mask(S, window) if window else None
    pad = None if lengths is None else orc.padding_mask(orc.lengths_attention_mask(lengths, S))
    return orc.composite_masked(q, k, v, dO, scale=scale, base_mask=base, pad_mask=pad, causal=causal,
                                want_lse=True)


def _no_key_rows(S, causal, window, lengths, B):
    """[B, S] bool: rows that see no key."""
    i = np.arange(S)
    out = np.zeros((B, S), bool)
    if lengths is None:
        return out
    for b, n in enumerate(lengths):
        out[b] = (n == 0) | ((window > 0) & (i - window + 1 >= n))
    return out


@pytest.mark.parametrize("case", CASES, ids=[_id(c) for c in CASES])
def test_masked_fwd_bwd_matches_oracle(orc, dev, case):
    from gpu_util import TOL, run_hip
    B, Hq, Hkv, S, D, dtype, causal, window, lengths = case
    q, k, v, dO = orc.make_inputs(B, Hq, Hkv, S, D, 500 + S + D + window, dtype, do_sigma=0.5)
    scale = 1.0 / math.sqrt(D)
    print(f"[case] {_id(case)}", flush=True)
    ref = _reference(orc, q, k, v, dO, scale, causal, window, lengths)
    got = run_hip(q, k, v, dO, dtype, scale, causal, dev, window=window, lengths=lengths)
    tol = TOL[dtype]
    errs = {n: orc.max_rel(got[n], ref[n]) for n in ("o", "dq", "dk", "dv")}
    print(f"[errs] {errs}", flush=True)
    for n, e in errs.items():
        assert e <= tol, f"{n}: max-rel {e:.3e} > {tol}"
    empty = _no_key_rows(S, causal, window, lengths, B)[:, None, :].repeat(Hq, 1)
    assert np.all(np.isposinf(got["lse"][empty]))
    lse_err = float(np.max(np.abs(got["lse"][~empty] - ref["lse"][~empty])))
    assert lse_err <= (1e-4 if dtype == "f32" else 1e-3), lse_err


def test_padded_rows_with_zero_grad_give_exact_zero_terms(orc, dev):
    """Training masks the padded positions out of the loss, so their dO rows
    are zero; the rows with no visible key then add nothing to any gradient,
    and the result equals the reference exactly where it is exactly zero."""
    from gpu_util import TOL, run_hip
    B, Hq, Hkv, S, D, W, L = 2, 4, 1, 400, 128, 64, [150, 400]
    q, k, v, dO = orc.make_inputs(B, Hq, Hkv, S, D, 42, "bf16", do_sigma=0.5)
    for b, n in enumerate(L):
        dO[b, :, n:, :] = 0.0
    ref = _reference(orc, q, k, v, dO, 1 / math.sqrt(D), True, W, L)
    got = run_hip(q, k, v, dO, "bf16", 1 / math.sqrt(D), True, dev, window=W, lengths=L)
    for n in ("o", "dq", "dk", "dv"):
        assert orc.max_rel(got[n], ref[n]) <= TOL["bf16"], n
    # padded keys get exactly zero gradient (no unmasked row sees them)
    assert np.all(got["dk"][0, :, L[0]:, :] == 0) and np.all(got["dv"][0, :, L[0]:, :] == 0)
    assert np.all(got["dq"][0, :, L[0]:, :] == 0)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_window_of_s_or_more_is_the_causal_mask(orc, dev, dtype):
    """window >= S hides nothing beyond the causal mask: bitwise the causal run."""
    from gpu_util import run_hip
    B, Hq, Hkv, S, D = 1, 4, 1, 300, 64
    q, k, v, dO = orc.make_inputs(B, Hq, Hkv, S, D, 3, dtype, do_sigma=0.5)
    a = run_hip(q, k, v, dO, dtype, 0.125, True, dev)
    for W in (S, S + 1000):
        b = run_hip(q, k, v, dO, dtype, 0.125, True, dev, window=W)
        for n in ("o", "lse", "dq", "dk", "dv"):
            assert np.array_equal(a[n], b[n]), (W, n)


def test_full_lengths_equal_no_padding(orc, dev):
    """kv_len = S everywhere: same bits as no padding (the masked-row passes
    find no row to fix)."""
    from gpu_util import run_hip
    B, Hq, Hkv, S, D = 2, 4, 2, 257, 128
    q, k, v, dO = orc.make_inputs(B, Hq, Hkv, S, D, 8, "bf16", do_sigma=0.5)
    a = run_hip(q, k, v, dO, "bf16", 0.1, True, dev, window=100)
    b = run_hip(q, k, v, dO, "bf16", 0.1, True, dev, window=100, lengths=[S, S])
    for n in ("o", "lse", "dq", "dk", "dv"):
        assert np.array_equal(a[n], b[n]), n


def test_window_forward_launch_shapes_agree(orc, dev):
    """Window geometry in both forward launches (balanced with split query
    tiles, and one workgroup per tile) against the oracle, at a length where
    tiles split across units."""
    import torch
    from gpu_util import TOL, to_dev
    from mobilefinetuner_amd import attention as A
    B, Hq, Hkv, S, D, W = 1, 4, 1, 2048, 256, 512
    q, k, v, _ = orc.make_inputs(B, Hq, Hkv, S, D, 71, "bf16")
    ref = _reference(orc, q, k, v, None, 1 / 16, True, W, None)
    tq, tk, tv = (to_dev(x, "bf16", dev) for x in (q, k, v))
    for balanced in (True, False):
        o, lse = A.attention_forward(tq, tk, tv, 1 / 16, True, balanced=balanced, window=W)
        torch.cuda.synchronize()
        assert orc.max_rel(o.float().cpu().numpy(), ref["o"]) <= TOL["bf16"], balanced
        assert np.max(np.abs(lse.cpu().numpy() - ref["lse"])) <= 1e-3, balanced
