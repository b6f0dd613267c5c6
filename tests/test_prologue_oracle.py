"""The q/k prologue oracle (oracle/refcpu.cpp orc_prologue_*) pinned three ways:

  * bit for bit against tests/golden/prologue.npz, which the REAL reference
    operators wrote (ops::rms_norm / rms_norm_affine, ops::apply_rope and their
    Engine backward; tests/golden/make_golden.py);
  * against oracle/_ref itself on fresh inputs where that library is built;
  * against what the mathematics fixes, so that a dropped term, a sign or a
    swapped pair fails: RoPE is a rotation of each pair (norm-preserving, the
    identity at position 0, inverted by its backward), an unweighted RMSNorm
    row has mean square 1, and the backward matches central differences of
    the forward.
"""
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def _cases():
    z = np.load(os.path.join(HERE, "golden", "prologue.npz"), allow_pickle=False)
    i = 0
    while f"case{i}" in z:
        yield i, z
        i += 1


def test_fixture_was_written_by_the_reference_and_matched_the_oracle():
    z = np.load(os.path.join(HERE, "golden", "prologue.npz"), allow_pickle=False)
    assert bool(z["refcpu_bitwise"])


@pytest.mark.parametrize("i", range(6))
def test_oracle_matches_reference_fixture_bitwise(orc, i):
    z = np.load(os.path.join(HERE, "golden", "prologue.npz"), allow_pickle=False)
    norm_id, eps, theta = z[f"case{i}_cfg"]
    norm = {v: k for k, v in orc.NORMS.items()}[int(norm_id)]
    x, w, dy = z[f"case{i}_x"], z[f"case{i}_w"], z[f"case{i}_dy"]
    got = orc.prologue(x, w if norm != "none" else None, dy, norm, float(eps), float(theta))
    assert np.array_equal(got["y"], z[f"case{i}_y"])
    assert np.array_equal(got["dx"], z[f"case{i}_dx"])
    if norm != "none":
        assert np.array_equal(got["dw"], z[f"case{i}_dw"])


@pytest.mark.parametrize("norm,theta", [("gemma", 1e6), ("affine", 1e4), ("none", 1e4), ("gemma", 0.0)])
def test_oracle_matches_reference_library(orc, norm, theta):
    if not orc.ref_available():
        pytest.skip("oracle/_ref not built (no reference checkout here)")
    rng = np.random.default_rng(7)
    x = rng.standard_normal((2, 3, 50, 80)).astype(np.float32)
    w = (0.2 * rng.standard_normal(80)).astype(np.float32)
    dy = rng.standard_normal(x.shape).astype(np.float32)
    a = orc.prologue(x, w if norm != "none" else None, dy, norm, 1e-6, theta)
    b = orc.ref_prologue(x, w if norm != "none" else None, dy, norm, 1e-6, theta)
    for k in a:
        if a[k] is not None:
            assert np.array_equal(a[k], b[k]), k


def test_rope_rotates_pairs(orc):
    rng = np.random.default_rng(1)
    B, H, S, D = 1, 2, 300, 64
    x = rng.standard_normal((B, H, S, D)).astype(np.float32)
    y = orc.prologue(x, None, None, "none", 0.0, 10000.0)["y"]
    half = D // 2
    # each (d, d + D/2) pair keeps its length
    nx = x[..., :half] ** 2 + x[..., half:] ** 2
    ny = y[..., :half] ** 2 + y[..., half:] ** 2
    assert np.max(np.abs(ny - nx) / np.maximum(nx, 1e-3)) < 1e-5
    # position 0 is the identity (cos 0 = 1, sin 0 = 0)
    assert np.array_equal(y[:, :, 0], x[:, :, 0])
    # pair d = 0 rotates by the angle pos (freq = 1): an independent closed form
    pos = np.arange(S, dtype=np.float64)
    y0 = x[..., 0].astype(np.float64) * np.cos(pos) - x[..., half].astype(np.float64) * np.sin(pos)
    assert np.max(np.abs(y[..., 0] - y0)) < 1e-4
    # the rotation moves something at pos > 0 (a swapped or dropped sin fails)
    assert np.max(np.abs(y[:, :, 5] - x[:, :, 5])) > 0.1


def test_rope_backward_inverts_forward(orc):
    rng = np.random.default_rng(2)
    dy = rng.standard_normal((2, 1, 40, 32)).astype(np.float32)
    dx = orc.prologue(dy, None, dy, "none", 0.0, 1e6)["dx"]  # R^T dy
    back = orc.prologue(dx, None, None, "none", 0.0, 1e6)["y"]  # R R^T dy
    assert np.max(np.abs(back - dy)) < 1e-5


def test_unweighted_rmsnorm_rows_have_unit_mean_square(orc):
    rng = np.random.default_rng(3)
    x = (5.0 * rng.standard_normal((1, 2, 30, 48))).astype(np.float32)
    y = orc.prologue(x, np.zeros(48, np.float32), None, "gemma", 1e-6, 0.0)["y"]  # (1 + 0) weight
    ms = np.mean(y.astype(np.float64) ** 2, axis=-1)
    assert np.max(np.abs(ms - 1.0)) < 1e-5
    y2 = orc.prologue(x, np.full(48, 2.0, np.float32), None, "affine", 1e-6, 0.0)["y"]
    assert np.max(np.abs(np.mean(y2.astype(np.float64) ** 2, axis=-1) - 4.0)) < 1e-4


@pytest.mark.parametrize("norm,theta", [("gemma", 1e4), ("affine", 1e6), ("none", 1e4)])
def test_backward_matches_central_differences(orc, norm, theta):
    rng = np.random.default_rng(4)
    B, H, S, D = 1, 1, 6, 16
    x = rng.standard_normal((B, H, S, D)).astype(np.float32)
    w = (0.5 * rng.standard_normal(D)).astype(np.float32)
    dy = rng.standard_normal(x.shape).astype(np.float32)
    wn = w if norm != "none" else None
    g = orc.prologue(x, wn, dy, norm, 1e-6, theta)

    def loss(xx, ww):
        y = orc.prologue(xx.astype(np.float32), None if ww is None else ww.astype(np.float32), None, norm, 1e-6,
                         theta)["y"]
        return float(np.sum(y.astype(np.float64) * dy))

    h = 1e-2
    for _ in range(6):
        v = rng.standard_normal(x.shape)
        fd = (loss(x + h * v, wn) - loss(x - h * v, wn)) / (2 * h)
        an = float(np.sum(g["dx"].astype(np.float64) * v))
        assert abs(fd - an) <= 2e-3 * max(1.0, abs(an)), (fd, an)
    if norm != "none":
        for _ in range(4):
            u = rng.standard_normal(D)
            fd = (loss(x, w + h * u) - loss(x, w - h * u)) / (2 * h)
            an = float(np.sum(g["dw"].astype(np.float64) * u))
            assert abs(fd - an) <= 2e-3 * max(1.0, abs(an)), (fd, an)
