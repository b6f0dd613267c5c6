"""The LoRA linear oracle (orc_lora, orc_lora_merge) pinned three ways:

  * bit for bit against tests/golden/lora.npz, which the REAL reference wrote
    (ops::LoRALinear forward, Engine backward and merge_to_base;
    tests/golden/make_golden.py), including the hand-written weights of
    nn/test_lora_linear.cpp;
  * against oracle/_ref itself on fresh inputs where that library is built;
  * against what the mathematics fixes, in float64: y = x W + b + sum s (x A) B,
    dx = dy W^T + sum s (dy_c B^T) A^T, grad_A = s x^T (dy_c B^T),
    grad_B = s (x A)^T dy_c, with every operand layout (transposed A, B, W);
    merging then running the plain layer reproduces the unmerged output (the
    reference test's own check); a slice over a column range gets no
    gradient unless asked for.
"""
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def _z():
    return np.load(os.path.join(HERE, "golden", "lora.npz"), allow_pickle=False)


def fixture_case(z, name):
    wt, wb, n, has_bias = (int(v) for v in z[f"{name}_flags"])
    slices = []
    for j in range(n):
        col0, at, bt = (int(v) for v in z[f"{name}_s{j}_meta"])
        slices.append(dict(A=z[f"{name}_s{j}_A"], B=z[f"{name}_s{j}_B"], scale=float(z[f"{name}_s{j}_scale"]),
                           col0=col0, a_transposed=bool(at), b_transposed=bool(bt)))
    bias = z[f"{name}_bias"] if has_bias else None
    return z[f"{name}_x"], z[f"{name}_W"], bias, slices, bool(wt), bool(wb), z[f"{name}_dy"]


def _eff(s):
    A = s["A"].T if s.get("a_transposed") else s["A"]
    B = s["B"].T if s.get("b_transposed") else s["B"]
    return A.astype(np.float64), B.astype(np.float64)


def closed_form(x, W, bias, slices, wt, dy, all_grads=False):
    x, dy = x.astype(np.float64), dy.astype(np.float64)
    We = (W.T if wt else W).astype(np.float64)
    out = We.shape[1]
    y = x @ We + (0 if bias is None else bias.astype(np.float64))
    dx = dy @ We.T
    gA, gB = [], []
    for s in slices:
        A, B = _eff(s)
        c0, cols = s.get("col0", 0), B.shape[1]
        y[:, c0:c0 + cols] += s["scale"] * (x @ A) @ B
        if all_grads or (c0 == 0 and cols == out):
            g = s["scale"] * dy[:, c0:c0 + cols] @ B.T
            dx += g @ A.T
            ga, gb = x.T @ g, s["scale"] * (x @ A).T @ dy[:, c0:c0 + cols]
            gA.append(ga.T if s.get("a_transposed") else ga)
            gB.append(gb.T if s.get("b_transposed") else gb)
        else:
            gA.append(None)
            gB.append(None)
    return dict(y=y, dx=dx, grad_A=gA, grad_B=gB)


def rel(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / max(1e-30, np.max(np.abs(b))))


def test_fixture_was_written_by_the_reference_and_matched_the_oracle():
    assert bool(_z()["refcpu_bitwise"])


@pytest.mark.parametrize("name", ["unit", "merge_bf16", "clear", "rand0", "rand1", "rand2"])
def test_oracle_matches_reference_fixture_bitwise(orc, name):
    z = _z()
    x, W, bias, slices, wt, wb, dy = fixture_case(z, name)
    got = orc.lora(x, W, bias, slices, w_transposed=wt, dy=dy, w_bf16=wb)
    assert np.array_equal(got["y"], z[f"{name}_y"]) and np.array_equal(got["dx"], z[f"{name}_dx"])
    for j in range(len(slices)):
        if f"{name}_s{j}_grad_A" in z:
            assert np.array_equal(got["grad_A"][j], z[f"{name}_s{j}_grad_A"])
            assert np.array_equal(got["grad_B"][j], z[f"{name}_s{j}_grad_B"])
        else:
            assert got["grad_A"][j] is None and got["grad_B"][j] is None
    if f"{name}_merged" in z:
        assert np.array_equal(orc.lora_merge(W, slices, w_bf16=wb), z[f"{name}_merged"])


def _random_case(rng, N, I, O, wt, specs):
    x = rng.standard_normal((N, I)).astype(np.float32)
    W = (0.3 * rng.standard_normal((O, I) if wt else (I, O))).astype(np.float32)
    slices = []
    for r, sc, c0, cols, at, bt in specs:
        A = (0.3 * rng.standard_normal((r, I) if at else (I, r))).astype(np.float32)
        B = (0.3 * rng.standard_normal((cols, r) if bt else (r, cols))).astype(np.float32)
        slices.append(dict(A=A, B=B, scale=sc, col0=c0, a_transposed=at, b_transposed=bt))
    return x, W, slices, rng.standard_normal((N, O)).astype(np.float32)


def test_oracle_matches_reference_library(orc):
    if not orc.ref_available():
        pytest.skip("oracle/_ref not built (no reference checkout here)")
    rng = np.random.default_rng(11)
    for wt, wb in ((False, False), (True, False), (False, True), (True, True)):
        x, W, slices, dy = _random_case(rng, 13, 70, 80, wt, [(4, 0.5, 0, 80, False, True), (3, 1.5, 10, 20, True,
                                                                                           False)])
        if wb:
            W = orc.round_bf16(W)
        bias = rng.standard_normal(80).astype(np.float32)
        a = orc.lora(x, W, bias, slices, w_transposed=wt, dy=dy, w_bf16=wb)
        b = orc.ref_lora(x, W, bias, slices, w_transposed=wt, dy=dy, w_bf16=wb)
        assert np.array_equal(a["y"], b["y"]) and np.array_equal(a["dx"], b["dx"]), (wt, wb)
        for j in range(2):
            assert (a["grad_A"][j] is None) == (b["grad_A"][j] is None)
            if a["grad_A"][j] is not None:
                assert np.array_equal(a["grad_A"][j], b["grad_A"][j]) and np.array_equal(a["grad_B"][j],
                                                                                         b["grad_B"][j])
        if not wt:
            assert np.array_equal(orc.lora_merge(W, slices, w_bf16=wb), orc.ref_lora_merge(W, slices, w_bf16=wb))


@pytest.mark.parametrize("wt", [False, True])
@pytest.mark.parametrize("all_grads", [False, True])
def test_oracle_matches_the_closed_form(orc, wt, all_grads):
    rng = np.random.default_rng(12)
    x, W, slices, dy = _random_case(rng, 19, 24, 30, wt, [(4, 0.5, 0, 30, False, False), (2, 2.0, 5, 12, True, True),
                                                          (3, 0.75, 0, 30, True, False)])
    bias = rng.standard_normal(30).astype(np.float32)
    got = orc.lora(x, W, bias, slices, w_transposed=wt, dy=dy, all_grads=all_grads)
    ref = closed_form(x, W, bias, slices, wt, dy, all_grads)
    assert rel(got["y"], ref["y"]) < 1e-5 and rel(got["dx"], ref["dx"]) < 1e-5
    for g, r in zip(got["grad_A"] + got["grad_B"], ref["grad_A"] + ref["grad_B"]):
        assert (g is None) == (r is None)
        if r is not None:
            assert rel(g, r) < 1e-5
    # the column-range slice is the only one without a gradient by default
    assert (got["grad_A"][1] is None) != all_grads


def test_merged_plain_layer_reproduces_the_unmerged_forward(orc):
    """nn/test_lora_linear.cpp:51-92 on the fixture's "unit" weights."""
    x, W, bias, slices, wt, wb, dy = fixture_case(_z(), "unit")
    before = orc.lora(x, W, bias, slices)["y"]
    after = orc.lora(x, orc.lora_merge(W, slices), bias, [])["y"]
    assert np.max(np.abs(before - after)) < 1e-6


def test_bf16_merge_changes_storage_and_sign_reverses_it(orc):
    """nn/test_lora_linear.cpp:94-122: a bf16 merge changes the bytes.  Undoing
    by the delta (sign -1) is exact here; the reference's unmerge restores a
    byte copy, which the GPU layer does too."""
    x, W, bias, slices, wt, wb, dy = fixture_case(_z(), "merge_bf16")
    m = orc.lora_merge(W, slices, w_bf16=True)
    assert not np.array_equal(m, W)
    assert np.array_equal(orc.round_bf16(m), m)
    assert np.array_equal(orc.lora_merge(m, slices, w_bf16=True, sign=-1.0), W)
