"""The CPU oracle (oracle/refcpu.cpp) pinned before it is trusted.

Each check is chosen so that a plausible mistake in the restatement (a dropped
term, a wrong sign or index, a transposed operand, a wrong rounding) fails at
least one of them:

  * golden vectors written by the REAL reference operators (oracle/_ref,
    compiled from the reference sources by tests/golden/make_golden.py):
    the fills and shapes of the reference's four hot-path unit tests plus
    seeded GQA cases (full tensors, bit-exact), and sampled outputs and
    checksums of the BASELINE.json configs;
  * the live reference build where it exists (bit-exact, fresh shapes);
  * an independent float64 brute force and closed-form invariants.
"""
import math

import numpy as np
import pytest

GOLD = __import__("os").path.join(__import__("os").path.dirname(__file__), "golden")


def _load(name):
    return np.load(f"{GOLD}/{name}.npz", allow_pickle=False)


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


# ------------------------------------------------------------ golden: tiny
def test_tiny_fixtures_bit_exact(orc):
    """Reference unit-test fills (optim/test_qkt_softmax_grad.cpp:28-59,
    optim/test_repeat_kv_softmax_grad.cpp:26-79,
    optim/test_attention_single_layer_backward.cpp:50-108,
    core/test_memory_efficient_attention_grad.cpp:61-87) and seeded GQA
    cases: the restatement reproduces the reference's O, dQ, dK, dV bits."""
    z = _load("tiny")
    names = [str(n) for n in z["names"]]
    assert len(names) == 8
    for n in names:
        r = orc.composite(z[f"{n}/q"], z[f"{n}/k"], z[f"{n}/v"], z[f"{n}/dO"],
                          scale=float(z[f"{n}/scale"]), causal=bool(z[f"{n}/causal"]))
        for t in ("o", "dq", "dk", "dv"):
            assert np.array_equal(_bits(r[t]), _bits(z[f"{n}/{t}"])), f"{n}/{t}"


def test_tiny_fill_generator_matches_fixture(orc):
    """fill_mod restates the reference tests' a*((i % m) - o) fills."""
    z = _load("tiny")
    q = z["memory_efficient_attention_grad/q"]
    assert np.array_equal(orc.fill_mod(q.size, 0.07, 11, 5).reshape(q.shape), q)


# --------------------------------------------------------- golden: configs
@pytest.mark.parametrize("cfg", ["c1", "c2", "c3", "c4", "c5", "c5f32"])
def test_config_inputs_match_fixture(orc, cfg):
    """Seeded generator (splitmix64 -> 53-bit uniform -> Box-Muller, RNE bf16,
    K-row stress for c4): first values and checksums of every stream."""
    z = _load(cfg)
    q, k, v, dO = orc.config_inputs(cfg)
    for name, arr in (("q", q), ("k", k), ("v", v), ("dO", dO)):
        flat = arr.reshape(-1)
        assert np.array_equal(flat[:8], z[f"in_{name}_head"]), name
        assert np.sum(flat, dtype=np.float64) == z[f"in_{name}_sum"], name
        assert np.sum(np.abs(flat), dtype=np.float64) == z[f"in_{name}_abssum"], name


@pytest.mark.parametrize("cfg", ["c1", "c2"])
def test_config_outputs_bit_exact(orc, cfg):
    """Full composite fwd+bwd at the config size: 2048 sampled outputs per
    tensor equal the reference's bits, and the checksums agree."""
    z = _load(cfg)
    c = orc.CONFIGS[cfg]
    q, k, v, dO = orc.config_inputs(cfg)
    r = orc.composite(q, k, v, dO, scale=c["scale"], causal=True)
    for t in ("o", "dq", "dk", "dv"):
        flat = r[t].reshape(-1)
        assert np.array_equal(_bits(flat[z[f"{t}_idx"]]), _bits(z[f"{t}_val"])), t
        assert math.isclose(float(np.sqrt(np.sum(flat.astype(np.float64) ** 2))), float(z[f"{t}_l2"]),
                            rel_tol=1e-12), t


def test_fixtures_record_refcpu_bitwise():
    """When the fixtures were written, the restatement was bit-identical to
    the reference on every config (including c3/c4/c5, too slow to rerun here)."""
    for cfg in ("c1", "c2", "c3", "c4", "c5", "c5f32"):
        assert int(_load(cfg)["refcpu_bitwise"]) == 1, cfg
    z = _load("tiny")
    for n in z["names"]:
        assert int(z[f"{n}/refcpu_bitwise"]) == 1, n


@pytest.mark.parametrize("shape,causal", [((2, 4, 1, 37, 16), True), ((1, 6, 2, 64, 32), False),
                                          ((2, 3, 3, 20, 8), True), ((1, 7, 1, 33, 64), True)])
def test_sliced_composite_is_bit_identical(orc, shape, causal):
    """composite_sliced (one (batch, head) per thread, kv gradients summed in
    head order) gives the whole-tensor composite's bits, so the full-config
    GPU parity compares against exactly the restated reference."""
    B, Hq, Hkv, S, D = shape
    q, k, v, dO = orc.make_inputs(B, Hq, Hkv, S, D, 9 + S, "f32", 0.5)
    a = orc.composite(q, k, v, dO, scale=0.3, causal=causal, want_lse=True)
    b = orc.composite_sliced(q, k, v, dO, scale=0.3, causal=causal, threads=4)
    for t in ("o", "lse", "dq", "dk", "dv"):
        assert np.array_equal(_bits(a[t]), _bits(b[t])), t


# ------------------------------------------------------- live reference
def _need_ref(orc):
    if not orc.ref_available():
        pytest.skip("oracle/_ref not built (reference checkout absent)")


@pytest.mark.parametrize("shape,causal", [((2, 6, 3, 37, 24), True), ((1, 4, 4, 29, 64), False),
                                          ((1, 4, 1, 70, 256), True)])
def test_refcpu_equals_live_reference(orc, shape, causal):
    _need_ref(orc)
    B, Hq, Hkv, S, D = shape
    q, k, v, dO = orc.make_inputs(B, Hq, Hkv, S, D, 31 + S, "f32", 0.3)
    a = orc.composite(q, k, v, dO, scale=1 / math.sqrt(D), causal=causal)
    b = orc.ref_composite(q, k, v, dO, scale=1 / math.sqrt(D), causal=causal)
    for t in ("o", "dq", "dk", "dv"):
        assert np.array_equal(_bits(a[t]), _bits(b[t])), t


def test_streaming_equals_live_reference(orc):
    """memory_efficient_attention no-grad path (core/memory_efficient_attention.cpp:110-200)."""
    _need_ref(orc)
    q, k, v, _ = orc.make_inputs(1, 3, 3, 45, 40, 7, "f32")
    for causal in (True, False):
        assert np.array_equal(_bits(orc.streaming(q, k, v, 0.2, causal)),
                              _bits(orc.ref_memeff_nograd(q, k, v, 0.2, causal)))


def test_repeat_kv_equals_live_reference(orc):
    """repeat_kv_heads and RepeatKVHeadsBackward (core/ops.cpp:2260-2335,
    core/backward_functions.cpp:693-726)."""
    _need_ref(orc)
    kv = orc.normal(2 * 3 * 9 * 16, 3, 0).reshape(2, 3, 9, 16)
    g = orc.normal(2 * 12 * 9 * 16, 3, 1).reshape(2, 12, 9, 16)
    out, dkv = orc.ref_repeat_kv(kv, 4, g)
    assert np.array_equal(orc.repeat_kv(kv, 4), out)
    assert np.array_equal(_bits(orc.repeat_kv_backward(g, 4)), _bits(dkv))


def test_bf16_rounding_equals_live_reference(orc):
    """float32_to_bf16_bits (core/dtype.h:114-128) on specials and ties."""
    _need_ref(orc)
    import ctypes
    R = orc.ref()
    R.mftref_f32_to_bf16_bits.restype = ctypes.c_uint16
    R.mftref_f32_to_bf16_bits.argtypes = [ctypes.c_float]
    vals = np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 1.0078125, 3.4e38, -3.4e38, 1e-40,
                     np.inf, -np.inf, 65504.0, 0.1, -2.5e-3], np.float32)
    vals = np.concatenate([vals, orc.normal(4096, 11, 0, 10.0)])
    for x in vals:
        assert orc.lib().orc_f32_to_bf16_bits(float(x)) == R.mftref_f32_to_bf16_bits(float(x)), x


# ------------------------------------------------ mathematics: independent
def _np_bf16_rne(x):
    """Round-to-nearest-even to bf16, written from the definition."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16).astype(np.uint32)
    return (r << 16).view(np.float32)


def test_bf16_rounding_is_round_to_nearest_even(orc):
    x = orc.normal(1 << 16, 5, 2, 3.0)
    assert np.array_equal(_bits(orc.round_bf16(x)), _bits(_np_bf16_rne(x)))
    # ties: 1 + 2^-8 is halfway between bf16 neighbours 1 and 1 + 2^-7 -> even (1.0)
    assert orc.round_bf16(np.array([1.00390625], np.float32))[0] == 1.0
    assert orc.round_bf16(np.array([1.01171875], np.float32))[0] == np.float32(1.015625)


@pytest.mark.parametrize("shape,causal", [((1, 4, 2, 50, 32), True), ((2, 3, 3, 17, 8), False),
                                          ((1, 2, 1, 96, 256), True)])
def test_composite_matches_float64_brute_force(orc, shape, causal):
    """A direct float64 evaluation of softmax(QK^T*scale + mask)V and of the
    five backward contractions agrees to fp32 rounding."""
    B, Hq, Hkv, S, D = shape
    q, k, v, dO = orc.make_inputs(B, Hq, Hkv, S, D, 90 + S, "f32", 0.5)
    a = orc.composite(q, k, v, dO, scale=1 / math.sqrt(D), causal=causal, want_lse=True)
    b = orc.brute_f64(q, k, v, dO, scale=1 / math.sqrt(D), causal=causal)
    for t in ("o", "dq", "dk", "dv"):
        assert orc.max_rel(a[t], b[t]) < 2e-6, t
    assert np.max(np.abs(a["lse"] - b["lse"])) < 1e-5


def _mha_reference(orc, q, k, v, dO, scale, causal):
    """GQA through the explicit repeat: MHA on repeat_kv(K), repeat_kv(V),
    then the repeat backward sums dK/dV over each group."""
    r = q.shape[1] // k.shape[1]
    m = orc.composite(q, orc.repeat_kv(k, r), orc.repeat_kv(v, r), dO, scale=scale, causal=causal)
    return m["o"], m["dq"], orc.repeat_kv_backward(m["dk"], r), orc.repeat_kv_backward(m["dv"], r)


def test_gqa_equals_repeat_kv_composite(orc):
    q, k, v, dO = orc.make_inputs(1, 8, 2, 40, 16, 12, "f32", 0.5)
    a = orc.composite(q, k, v, dO, scale=0.25, causal=True)
    o, dq, dk, dv = _mha_reference(orc, q, k, v, dO, 0.25, True)
    assert np.array_equal(a["o"], o) and np.array_equal(a["dq"], dq)
    assert orc.max_rel(a["dk"], dk) < 1e-6 and orc.max_rel(a["dv"], dv) < 1e-6


def test_invariants(orc):
    B, Hq, Hkv, S, D = 1, 4, 2, 33, 16
    q, k, v, dO = orc.make_inputs(B, Hq, Hkv, S, D, 77, "f32", 0.5)
    r = orc.composite(q, k, v, dO, scale=0.25, causal=True, want_lse=True)
    grp = Hq // Hkv
    # causal row 0 attends only to key 0: O[h, 0] = V[h // r, 0]
    for h in range(Hq):
        assert np.array_equal(r["o"][0, h, 0], v[0, h // grp, 0])
    # P rows sum to 1  =>  sum over keys of dV = sum over queries of dO (per KV group)
    for g in range(Hkv):
        lhs = r["dv"][0, g].astype(np.float64).sum(0)
        rhs = dO[0, g * grp:(g + 1) * grp].astype(np.float64).sum((0, 1))
        assert np.allclose(lhs, rhs, rtol=1e-5, atol=1e-5)
    # each row of dS sums to 0  =>  sum over keys of dK = 0
    assert np.max(np.abs(r["dk"].astype(np.float64).sum(2))) < 1e-5 * np.max(np.abs(r["dk"])) * S
    # equal K rows: uniform causal weights, O = prefix mean of V, dQ = 0
    k_eq = np.repeat(k[:, :, :1], S, axis=2)
    e = orc.composite(q, k_eq, v, dO, scale=0.25, causal=True)
    for h in range(Hq):
        pm = np.cumsum(v[0, h // grp].astype(np.float64), 0) / np.arange(1, S + 1)[:, None]
        assert np.allclose(e["o"][0, h], pm, rtol=1e-5, atol=1e-6)
    assert np.max(np.abs(e["dq"])) < 1e-6
    # scale equivariance with an exact power of two: bit-identical
    s2 = orc.composite(q * np.float32(2.0), k, v, dO, scale=0.125, causal=True)
    assert np.array_equal(s2["o"], r["o"])


def test_lse_is_log_normaliser(orc):
    """The saved LSE satisfies O = softmax(...)V with P = exp(s*scale - LSE)."""
    q, k, v, _ = orc.make_inputs(1, 1, 1, 20, 8, 4, "f32")
    r = orc.composite(q, k, v, scale=0.3, causal=True, want_lse=True)
    s = (q[0, 0].astype(np.float64) @ k[0, 0].astype(np.float64).T) * 0.3
    s[np.triu_indices(20, 1)] = -np.inf
    lse = np.log(np.exp(s - s.max(1, keepdims=True)).sum(1)) + s.max(1)
    assert np.allclose(r["lse"][0, 0], lse, atol=1e-5)
    p = np.exp(s - lse[:, None])
    assert np.allclose(p @ v[0, 0], r["o"][0, 0], atol=1e-5)


# ------------------------------------------------- masks (widened path)
@pytest.mark.parametrize("window,lengths", [(5, None), (None, [40, 23]), (16, [40, 40]), (1, None), (64, None)])
def test_masked_composite_equals_live_reference(orc, window, lengths):
    """Sliding-window (build_sliding_mask) and padding (build_padding_mask)
    masks added as the Gemma graph adds them (graph/gemma_model.cpp:494-499)."""
    _need_ref(orc)
    B, Hq, Hkv, S, D = 2, 4, 2, 40, 16
    q, k, v, dO = orc.make_inputs(B, Hq, Hkv, S, D, 71, "f32", 0.5)
    base = orc.sliding_mask(S, window) if window else orc.causal_mask(S)
    pad = orc.padding_mask(orc.lengths_attention_mask(lengths, S)) if lengths else None
    a = orc.composite_masked(q, k, v, dO, scale=0.25, base_mask=base, pad_mask=pad)
    b = orc.ref_composite_masked(q, k, v, dO, scale=0.25, base_mask=base, pad_mask=pad)
    for t in ("o", "dq", "dk", "dv"):
        assert np.array_equal(_bits(a[t]), _bits(b[t])), t


def test_mask_builders_and_invariants(orc):
    S = 12
    # the causal mask is the sliding mask with a window of S or more
    assert np.array_equal(orc.sliding_mask(S, S), orc.causal_mask(S))
    assert np.array_equal(orc.sliding_mask(S, 1000), orc.causal_mask(S))
    # float and int32 attention masks give the same padding mask
    am = orc.lengths_attention_mask([5, 12], S)
    assert np.array_equal(orc.padding_mask(am), orc.padding_mask(am.astype(np.float32)))
    assert orc.padding_mask(am)[0, 4] == 0 and orc.padding_mask(am)[0, 5] == orc.MASK_VALUE
    q, k, v, dO = orc.make_inputs(1, 2, 2, S, 8, 3, "f32", 0.5)
    # window 1: each query sees only itself, O_i = V_i
    r = orc.composite_masked(q, k, v, dO, scale=0.3, base_mask=orc.sliding_mask(S, 1))
    assert np.array_equal(r["o"], v)
    # the causal path through the masked entry point is the plain composite
    a = orc.composite_masked(q, k, v, dO, scale=0.3, base_mask=orc.causal_mask(S))
    b = orc.composite(q, k, v, dO, scale=0.3, causal=True)
    for t in ("o", "dq", "dk", "dv"):
        assert np.array_equal(a[t], b[t]), t
    # padded keys get no gradient and no weight when every row sees a real key
    pad = orc.padding_mask(orc.lengths_attention_mask([7], S))
    r = orc.composite_masked(q, k, v, dO, scale=0.3, pad_mask=pad)
    assert np.all(r["dk"][0, :, 7:] == 0) and np.all(r["dv"][0, :, 7:] == 0)
    ref7 = orc.composite(q[:, :, :7], k[:, :, :7], v[:, :, :7], dO[:, :, :7], scale=0.3, causal=True)
    assert np.allclose(r["o"][:, :, :7], ref7["o"], atol=1e-6)


# ------------------------------------ general additive masks (the mask mode)
def _general_masks(B, Hq, S, seed):
    rng = np.random.default_rng(seed)
    ss = rng.normal(size=(S, S)).astype(np.float32)
    ss[rng.random((S, S)) < 0.3] = -1e10
    ss[S // 2, :] = -1e10  # a row masked everywhere: uniform softmax
    bss = rng.normal(size=(B, 1, S, S)).astype(np.float32)
    bss[:, :, 1, :] = -1e9
    left = np.zeros((B, 1, 1, S), np.float32)
    left[:, :, :, :3] = -1e10  # left padding (not a suffix)
    head = (-0.25 * np.arange(1, Hq + 1)[None, :, None, None] * np.arange(S)[None, None, None, :]).astype(np.float32)
    return ss, bss, left, head


@pytest.mark.parametrize("which", [(0,), (1,), (2,), (3,), (0, 2), (1, 3)])
def test_general_mask_composite_equals_live_reference(orc, which):
    """orc.composite_masks (mode 0) bit-exact against the reference composite
    with the same dense masks added by its own broadcasting ops::add
    (ref_harness.cpp mftref_composite_mask4): [S,S], [B,1,S,S], [B,1,1,S] and
    [1,Hq,1,S] masks, alone and two in order."""
    _need_ref(orc)
    B, Hq, Hkv, S, D = 2, 4, 2, 41, 24
    q, k, v, dO = orc.make_inputs(B, Hq, Hkv, S, D, 83, "f32", 0.5)
    all_m = _general_masks(B, Hq, S, 5)
    masks = [all_m[i] for i in which]
    a = orc.composite_masks(q, k, v, dO, scale=0.3, mode=0, masks=masks)
    b = orc.ref_composite_mask4(q, k, v, dO, scale=0.3, masks=masks)
    for t in ("o", "dq", "dk", "dv"):
        assert np.array_equal(_bits(a[t]), _bits(b[t])), t


def test_mask_streaming_equals_live_reference(orc):
    """The no-grad operator with an [S,S] mask (core/memory_efficient_attention.cpp:
    160-172: causal replacement by -1e10, then + mask), bit-exact; the mask
    mode's composite arithmetic with the same rule (mode 1) is within 1e-6."""
    _need_ref(orc)
    B, H, S, D = 2, 3, 37, 32
    q, k, v, _ = orc.make_inputs(B, H, H, S, D, 19, "f32")
    ss = _general_masks(B, H, S, 9)[0]
    for causal in (True, False):
        a = orc.streaming_mask(q, k, v, ss, 0.2, causal)
        b = orc.ref_memeff_nograd_mask(q, k, v, ss, 0.2, causal)
        assert np.array_equal(_bits(a), _bits(b)), causal
        c = orc.composite_masks(q, k, v, None, scale=0.2, mode=1 if causal else 0, masks=[ss])["o"]
        assert orc.max_rel(c, b) <= 1e-6, causal


def test_general_mask_invariants(orc):
    """What the mathematics fixes for additive masks: a row masked everywhere
    by one value is a uniform softmax (O = mean of V); adding a constant to a
    whole row of the mask changes nothing; an all-zero mask is the unmasked
    composite; mode 2 equals mode 0 with create_causal_mask as the mask."""
    B, Hq, Hkv, S, D = 1, 2, 1, 30, 16
    q, k, v, dO = orc.make_inputs(B, Hq, Hkv, S, D, 23, "f32", 0.5)
    full = np.full((S, S), -1e10, np.float32)
    o = orc.composite_masks(q, k, v, None, scale=0.25, masks=[full])["o"]
    assert np.allclose(o[0, 0], v[0, 0].mean(axis=0), atol=1e-6)
    rng = np.random.default_rng(3)
    m = rng.normal(size=(S, S)).astype(np.float32)
    shift = (m + 3.0 * np.arange(S, dtype=np.float32)[:, None]).astype(np.float32)
    a = orc.composite_masks(q, k, v, dO, scale=0.25, masks=[m])
    b = orc.composite_masks(q, k, v, dO, scale=0.25, masks=[shift])
    for t in ("o", "dq", "dk", "dv"):
        assert orc.max_rel(a[t], b[t]) <= 1e-5, t
    z = orc.composite_masks(q, k, v, dO, scale=0.25, masks=[np.zeros((S, S), np.float32)])
    p = orc.composite(q, k, v, dO, scale=0.25, causal=False)
    for t in ("o", "dq", "dk", "dv"):
        assert np.array_equal(_bits(z[t]), _bits(p[t])), t
    c2 = orc.composite_masks(q, k, v, dO, scale=0.25, mode=2)
    c0 = orc.composite_masks(q, k, v, dO, scale=0.25, mode=0, masks=[orc.causal_mask(S)])
    for t in ("o", "dq", "dk", "dv"):
        assert np.array_equal(_bits(c2[t]), _bits(c0[t])), t
