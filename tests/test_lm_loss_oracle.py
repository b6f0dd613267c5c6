"""The LM cross-entropy oracle (orc_lm_ce, orc_selected_ce) pinned three ways:

  * bit for bit against tests/golden/lm_loss.npz, which the REAL reference
    wrote (ops::lm_cross_entropy and ops::streaming_lm_cross_entropy with
    their Engine backward; tests/golden/make_golden.py), including the
    hand-written case of core/test_selected_token_lm_loss.cpp;
  * against oracle/_ref itself on fresh inputs where that library is built;
  * against what the mathematics fixes: uniform logits give log V, a scored
    row's gradient sums to zero and an unscored one is zero, the gradient
    matches central differences of the loss, the dense and streaming
    variants agree (the reference test's own check), and an all-ignored batch
    gives a NaN mean with zero gradients.
"""
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CASES = ("unit", "rand0", "rand1")


def _z():
    return np.load(os.path.join(HERE, "golden", "lm_loss.npz"), allow_pickle=False)


def test_fixture_was_written_by_the_reference_and_matched_the_oracle():
    assert bool(_z()["refcpu_bitwise"])


@pytest.mark.parametrize("case", CASES)
def test_oracle_matches_reference_fixture_bitwise(orc, case):
    z = _z()
    h, w, y, logits = (z[f"{case}_{k}"] for k in ("hidden", "weight", "labels", "logits"))
    for red in ("mean", "sum", "none"):
        g = z[f"{case}_dense_{red}_gout"]
        got = orc.lm_ce(logits, y, -100, red, g if red == "none" else float(g))
        assert np.array_equal(got["loss"], z[f"{case}_dense_{red}_loss"], equal_nan=True), red
        assert np.array_equal(got["grad"], z[f"{case}_dense_{red}_grad"]), red
    for red in ("mean", "sum"):
        got = orc.selected_ce(h, w, y, -100, red, 0.75)
        for k in ("loss", "grad_hidden", "grad_weight"):
            assert np.array_equal(got[k], z[f"{case}_stream_{red}_{k}"]), (red, k)


def test_oracle_matches_reference_library(orc):
    if not orc.ref_available():
        pytest.skip("oracle/_ref not built (no reference checkout here)")
    rng = np.random.default_rng(3)
    B, S, H, V = 2, 11, 7, 90
    logits = (3 * rng.standard_normal((B, S, V))).astype(np.float32)
    y = rng.integers(0, V, (B, S)).astype(np.int32)
    y[1, 3] = -100
    for red in ("mean", "sum", "none"):
        g = rng.standard_normal((B, S)).astype(np.float32) if red == "none" else 1.5
        a, b = orc.lm_ce(logits, y, -100, red, g), orc.ref_lm_ce(logits, y, -100, red, g)
        assert np.array_equal(a["loss"], b["loss"]) and np.array_equal(a["grad"], b["grad"])
    h = rng.standard_normal((B, S, H)).astype(np.float32)
    w = rng.standard_normal((V, H)).astype(np.float32)
    for red in ("mean", "sum"):
        a, b = orc.selected_ce(h, w, y, -100, red, 0.5), orc.ref_streaming_ce(h, w, y, -100, red, 0.5)
        for k in a:
            assert np.array_equal(a[k], b[k]), (red, k)


def test_uniform_logits_give_log_v(orc):
    B, S, V = 1, 6, 250
    y = np.arange(S, dtype=np.int32)[None] % V
    out = orc.lm_ce(np.full((B, S, V), 0.37, np.float32), y, -100, "mean", 1.0)
    assert abs(float(out["loss"][0]) - np.log(V)) < 1e-6
    # gradient 1/V everywhere except -(1 - 1/V) at the label, / count
    g = out["grad"][0, 0]
    assert abs(g[y[0, 1]] - (1 / V - 1) / (S - 1)) < 1e-7 and abs(g[0] - 1 / V / (S - 1)) < 1e-7


def test_gradient_rows_sum_to_zero_and_unscored_rows_are_zero(orc):
    rng = np.random.default_rng(4)
    B, S, V = 2, 8, 60
    logits = (2 * rng.standard_normal((B, S, V))).astype(np.float32)
    y = rng.integers(0, V, (B, S)).astype(np.int32)
    y[0, 4] = -100  # position (0, 3) is not scored
    g = orc.lm_ce(logits, y, -100, "sum", 1.0)["grad"]
    assert np.all(g[0, 3] == 0) and np.all(g[:, S - 1] == 0)
    scored = [(b, s) for b in range(B) for s in range(S - 1) if y[b, s + 1] != -100]
    assert max(abs(float(g[b, s].astype(np.float64).sum())) for b, s in scored) < 1e-6


def test_gradient_matches_central_differences(orc):
    rng = np.random.default_rng(5)
    B, S, V = 1, 5, 12
    logits = rng.standard_normal((B, S, V)).astype(np.float64)
    y = rng.integers(0, V, (B, S)).astype(np.int32)
    g = orc.lm_ce(logits.astype(np.float32), y, -100, "mean", 1.0)["grad"].astype(np.float64)
    h = 1e-2
    for _ in range(6):
        d = rng.standard_normal(logits.shape)
        lp = float(orc.lm_ce((logits + h * d).astype(np.float32), y)["loss"][0])
        lm = float(orc.lm_ce((logits - h * d).astype(np.float32), y)["loss"][0])
        fd, an = (lp - lm) / (2 * h), float(np.sum(g * d))
        assert abs(fd - an) <= 2e-3 * max(1.0, abs(an)), (fd, an)


def test_dense_and_streaming_agree(orc):
    """The reference test's check (core/test_selected_token_lm_loss.cpp:98-115)
    on the fixture's cases: streaming loss and gradients equal dense ones
    (logits = hidden . W^T, the dense gradient chained through it)."""
    z = _z()
    for case in CASES:
        h, w, y = (z[f"{case}_{k}"] for k in ("hidden", "weight", "labels"))
        logits = np.einsum("bsh,vh->bsv", h, w).astype(np.float32)
        for red in ("mean", "sum"):
            d = orc.lm_ce(logits, y, -100, red, 0.75)
            s = orc.selected_ce(h, w, y, -100, red, 0.75)
            assert abs(float(d["loss"][0] - s["loss"][0])) <= 1e-5 * max(1.0, abs(float(d["loss"][0])))
            gh = np.einsum("bsv,vh->bsh", d["grad"], w)
            gw = np.einsum("bsv,bsh->vh", d["grad"], h)
            assert np.max(np.abs(gh - s["grad_hidden"])) < 1e-5 and np.max(np.abs(gw - s["grad_weight"])) < 1e-5


def test_all_ignored_is_nan_with_zero_gradients(orc):
    B, S, H, V = 2, 4, 3, 5
    y = np.full((B, S), -100, np.int32)
    rng = np.random.default_rng(6)
    h, w = rng.standard_normal((B, S, H)).astype(np.float32), rng.standard_normal((V, H)).astype(np.float32)
    s = orc.selected_ce(h, w, y, -100, "mean", 1.0)
    assert np.isnan(s["loss"][0]) and np.all(s["grad_hidden"] == 0)
    d = orc.lm_ce(np.zeros((B, S, V), np.float32), y, -100, "mean", 1.0)
    assert np.isnan(d["loss"][0]) and np.all(d["grad"] == 0)


def test_out_of_range_label_raises(orc):
    y = np.array([[0, 7, 1]], np.int32)
    with pytest.raises(ValueError, match="out of range"):
        orc.lm_ce(np.zeros((1, 3, 5), np.float32), y)
