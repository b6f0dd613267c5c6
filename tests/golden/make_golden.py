"""Write the golden fixtures of the attention path from the REAL reference.

Runs in the build container only (it needs oracle/_ref/libmftref.so, which is
compiled from /root/reference by oracle/Makefile).  Outputs, all data:

  tests/golden/prologue.npz  full tensors of the q/k prologue (rms_norm /
                             rms_norm_affine + apply_rope, fwd and bwd)
  tests/golden/lm_loss.npz   lm_cross_entropy and streaming_lm_cross_entropy
                             (loss, gradients), incl. the reference test's case
  tests/golden/tiny.npz      full tensors of small cases: the deterministic
                             fills and shapes of the reference's four hot-path
                             unit tests plus seeded GQA cases
  tests/golden/<cfg>.npz     for each BASELINE.json config: the first values
                             of every input stream, input checksums, and for
                             O, dQ, dK, dV the L2 norm, max |x| and 2048
                             sampled (flat index, value) pairs

While generating, the restatement (oracle/refcpu.cpp) is run on the same
inputs and must be bit-identical to the reference; the outcome is stored as
`refcpu_bitwise` in each fixture.

    python tests/golden/make_golden.py [cfg ...]
"""
from __future__ import annotations

import math
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
from oracle import oracle as O  # noqa: E402

NSAMPLE = 2048


def fill(shape, a, m, o):
    return O.fill_mod(int(np.prod(shape)), a, m, o).reshape(shape)


def tiny_cases():
    """(name, q, k, v, dO, scale, causal).  Fills cite the reference tests."""
    cases = []
    # optim/test_qkt_softmax_grad.cpp:28-59 (q, k fills; scale 256^-0.5; no mask).
    # That test has no V; v takes the fill of test_repeat_kv_softmax_grad.cpp:52.
    s = (1, 1, 3, 4)
    cases.append(("qkt_softmax_grad", fill(s, 0.1, 7, 3), fill(s, 0.07, 5, 2), fill(s, 0.03, 5, 2),
                  fill(s, 0.03, 11, 5), 256.0 ** -0.5, False))
    # optim/test_repeat_kv_softmax_grad.cpp:26-79: kvH=1 -> H=4, S=3, D=4, mask off.
    qs, ks = (1, 4, 3, 4), (1, 1, 3, 4)
    cases.append(("repeat_kv_softmax_grad", fill(qs, 0.05, 9, 4), fill(ks, 0.04, 7, 3),
                  fill(ks, 0.03, 5, 2), fill(qs, 0.02, 11, 5), 0.5, False))
    # optim/test_attention_single_layer_backward.cpp:50-108: B=1,H=4,S=8,D=8, kvH=1, causal.
    qs, ks = (1, 4, 8, 8), (1, 1, 8, 8)
    cases.append(("attention_single_layer_backward", fill(qs, 0.013, 17, 8), fill(ks, 0.011, 13, 6),
                  fill(ks, 0.015, 19, 9), fill(qs, 0.02, 11, 5), 256.0 ** -0.5, True))
    # core/test_memory_efficient_attention_grad.cpp:61-87: B=1,H=2,S=4,D=3, causal.
    s = (1, 2, 4, 3)
    cases.append(("memory_efficient_attention_grad", fill(s, 0.07, 11, 5), fill(s, 0.05, 9, 4),
                  fill(s, 0.03, 7, 3), fill(s, 0.02, 13, 6), 1.0 / math.sqrt(3.0), True))
    # Seeded GQA cases (groups of 4 and 7, D 64 and 256, causal on and off).
    for i, (B, Hq, Hkv, S, D, causal) in enumerate([(1, 4, 1, 64, 64, True), (1, 7, 1, 48, 64, False),
                                                    (2, 8, 2, 40, 256, True), (1, 14, 2, 33, 64, True)]):
        q, k, v, dO = O.make_inputs(B, Hq, Hkv, S, D, 500 + i, "f32", 0.5)
        cases.append((f"gqa_{B}x{Hq}x{Hkv}x{S}x{D}_{'causal' if causal else 'full'}", q, k, v, dO,
                      1.0 / math.sqrt(D), causal))
    return cases


def bitwise(a, b):
    return bool(np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                               np.asarray(b, np.float32).view(np.uint32)))


def make_tiny():
    out = {}
    names = []
    for name, q, k, v, dO, scale, causal in tiny_cases():
        r = O.ref_composite(q, k, v, dO, scale=scale, causal=causal)
        m = O.composite(q, k, v, dO, scale=scale, causal=causal)
        ok = all(bitwise(m[n], r[n]) for n in ("o", "dq", "dk", "dv"))
        print(f"[tiny] {name}: refcpu bitwise={ok}")
        names.append(name)
        for key, arr in (("q", q), ("k", k), ("v", v), ("dO", dO), ("o", r["o"]), ("dq", r["dq"]),
                         ("dk", r["dk"]), ("dv", r["dv"])):
            out[f"{name}/{key}"] = np.asarray(arr, np.float32)
        out[f"{name}/scale"] = np.float32(scale)
        out[f"{name}/causal"] = np.int32(causal)
        out[f"{name}/refcpu_bitwise"] = np.int32(ok)
    out["names"] = np.array(names)
    np.savez_compressed(os.path.join(HERE, "tiny.npz"), **out)


def make_config(cfg):
    c = O.CONFIGS[cfg]
    seed = O.SEEDS[cfg]
    q, k, v, dO = O.config_inputs(cfg)
    rng = np.random.default_rng(seed)
    t0 = time.time()
    r = O.ref_composite(q, k, v, dO, scale=c["scale"], causal=True)
    t_ref = time.time() - t0
    t0 = time.time()
    m = O.composite(q, k, v, dO, scale=c["scale"], causal=True)
    t_orc = time.time() - t0
    ok = all(bitwise(m[n], r[n]) for n in ("o", "dq", "dk", "dv"))
    print(f"[{cfg}] ref {t_ref:.1f}s (fwd {r['t_fwd']:.2f} bwd {r['t_bwd']:.2f}) refcpu {t_orc:.1f}s "
          f"bitwise={ok} held={r['held_bytes'] / 2**20:.1f} MiB")
    out = dict(cfg=cfg, seed=np.int64(seed), scale=np.float32(c["scale"]),
               refcpu_bitwise=np.int32(ok), held_bytes=np.int64(r["held_bytes"]),
               ref_t_fwd=np.float64(r["t_fwd"]), ref_t_bwd=np.float64(r["t_bwd"]))
    for name, arr in (("q", q), ("k", k), ("v", v), ("dO", dO)):
        flat = arr.reshape(-1)
        out[f"in_{name}_head"] = flat[:8].copy()
        out[f"in_{name}_sum"] = np.float64(np.sum(flat, dtype=np.float64))
        out[f"in_{name}_abssum"] = np.float64(np.sum(np.abs(flat), dtype=np.float64))
    for name in ("o", "dq", "dk", "dv"):
        flat = r[name].reshape(-1)
        idx = np.sort(rng.choice(flat.size, size=min(NSAMPLE, flat.size), replace=False)).astype(np.int64)
        out[f"{name}_idx"] = idx
        out[f"{name}_val"] = flat[idx].copy()
        out[f"{name}_l2"] = np.float64(np.sqrt(np.sum(flat.astype(np.float64) ** 2)))
        out[f"{name}_maxabs"] = np.float64(np.max(np.abs(flat)))
        out[f"{name}_sum"] = np.float64(np.sum(flat, dtype=np.float64))
    np.savez_compressed(os.path.join(HERE, f"{cfg}.npz"), **out)


# q/k prologue cases: (B, H, S, D, norm, eps, theta, seed).  Gemma-3's
# rms_norm_eps and rope thetas (1e6 global, 1e4 local layers), Qwen's RoPE
# without a norm, the affine variant, no RoPE, an odd half-dim, and positions
# up to 4095 on a narrow head.
PROLOGUE_CASES = [
    (1, 2, 33, 64, "gemma", 1e-6, 10000.0, 1),
    (2, 1, 17, 128, "gemma", 1e-6, 1000000.0, 2),
    (1, 3, 20, 256, "none", 1e-6, 1000000.0, 3),
    (1, 2, 12, 96, "affine", 1e-5, 10000.0, 4),
    (1, 1, 9, 6, "gemma", 1e-6, 0.0, 5),
    (1, 1, 4096, 4, "gemma", 1e-6, 10000.0, 6),
]


def make_prologue():
    """tests/golden/prologue.npz: full tensors (x, w, dy -> y, dx, dw) of the
    reference's rms_norm / rms_norm_affine + apply_rope and their backward."""
    out = {}
    ok = True
    for i, (B, H, S, D, norm, eps, theta, seed) in enumerate(PROLOGUE_CASES):
        n = B * H * S * D
        x = (2.0 * O.normal(n, 3000 + seed, 0)).reshape(B, H, S, D).astype(np.float32)
        w = (0.3 * O.normal(D, 3000 + seed, 1)).astype(np.float32)
        dy = O.normal(n, 3000 + seed, 2).reshape(B, H, S, D).astype(np.float32)
        r = O.ref_prologue(x, w if norm != "none" else None, dy, norm, eps, theta)
        mine = O.prologue(x, w if norm != "none" else None, dy, norm, eps, theta)
        ok = ok and all(bitwise(mine[k], r[k]) for k in r if r[k] is not None)
        out[f"case{i}"] = np.array([B, H, S, D, seed], np.int64)
        out[f"case{i}_cfg"] = np.array([O.NORMS[norm], eps, theta], np.float64)
        for k, v in (("x", x), ("w", w), ("dy", dy), ("y", r["y"]), ("dx", r["dx"])):
            out[f"case{i}_{k}"] = v
        if r["dw"] is not None:
            out[f"case{i}_dw"] = r["dw"]
    out["refcpu_bitwise"] = np.array(ok)
    path = os.path.join(HERE, "prologue.npz")
    np.savez_compressed(path, **out)
    print(f"prologue: {len(PROLOGUE_CASES)} cases, refcpu bitwise = {ok} -> {path}")


def make_lm_loss():
    """tests/golden/lm_loss.npz: the reference's lm_cross_entropy and
    streaming_lm_cross_entropy (loss and gradients) on the hand-written case of
    core/test_selected_token_lm_loss.cpp:49-76 and on seeded random cases."""
    out = {}
    ok = True
    # the reference test's own values
    hidden = np.array([0.10, -0.20, 0.30, 0.00, 0.25, -0.15, 0.40, -0.10, 0.05, -0.30, 0.20, 0.10,
                       0.05, 0.15, -0.25, 0.30, 0.10, -0.05, -0.20, 0.35, 0.25, 0.12, -0.08, 0.18],
                      np.float32).reshape(2, 4, 3)
    weight = np.array([0.20, -0.10, 0.05, -0.30, 0.25, 0.10, 0.15, 0.05, -0.20, 0.40, -0.35, 0.12,
                       -0.05, 0.18, 0.30], np.float32).reshape(5, 3)
    labels = np.array([[-100, 2, -100, 1], [-100, -100, 4, -100]], np.int32)
    cases = [("unit", hidden, weight, labels)]
    for i, (B, S, H, V) in enumerate([(2, 17, 24, 300), (1, 33, 40, 1000)]):
        h = (0.5 * O.normal(B * S * H, 5000 + i, 0)).reshape(B, S, H).astype(np.float32)
        w = (0.5 * O.normal(V * H, 5000 + i, 1)).reshape(V, H).astype(np.float32)
        u = np.array([O.uniform(5000 + i, 2, j) for j in range(B * S)])
        y = np.minimum((u * V).astype(np.int64), V - 1).astype(np.int32).reshape(B, S)
        y[u.reshape(B, S) < 0.15] = -100
        cases.append((f"rand{i}", h, w, y))
    for name, h, w, y in cases:
        logits = np.einsum("bsh,vh->bsv", h.astype(np.float64), w.astype(np.float64)).astype(np.float32)
        out[f"{name}_hidden"], out[f"{name}_weight"], out[f"{name}_labels"] = h, w, y
        out[f"{name}_logits"] = logits
        for red in ("mean", "sum", "none"):
            g = 0.75 if red != "none" else (O.normal(y.size, 5100, 0).reshape(y.shape) + 1.0)
            r = O.ref_lm_ce(logits, y, -100, red, g)
            m = O.lm_ce(logits, y, -100, red, g)
            ok = ok and bitwise(m["loss"], r["loss"]) and bitwise(m["grad"], r["grad"])
            out[f"{name}_dense_{red}_gout"] = np.asarray(g, np.float32)
            out[f"{name}_dense_{red}_loss"], out[f"{name}_dense_{red}_grad"] = r["loss"], r["grad"]
        for red in ("mean", "sum"):
            r = O.ref_streaming_ce(h, w, y, -100, red, 0.75)
            m = O.selected_ce(h, w, y, -100, red, 0.75)
            ok = ok and all(bitwise(m[k], r[k]) for k in r)
            for k in r:
                out[f"{name}_stream_{red}_{k}"] = r[k]
    out["refcpu_bitwise"] = np.array(ok)
    path = os.path.join(HERE, "lm_loss.npz")
    np.savez_compressed(path, **out)
    print(f"lm_loss: {len(cases)} cases, refcpu bitwise = {ok} -> {path}")


def lora_cases():
    """The LoRA fixture's cases: (name, x [N, in], W values, bias, slices,
    w_transposed, w_bf16, dy).  "unit" is the hand-written case of
    nn/test_lora_linear.cpp:51-92; "merge_bf16" and "clear" are the weights of
    its other two tests (:94-141), whose checks are about merging."""
    f32 = lambda a, *sh: np.array(a, np.float32).reshape(sh)
    cases = [
        ("unit", f32([1.0, -2.0, 0.5, -1.5, 0.25, 2.0], 2, 3),
         f32([0.10, -0.20, 0.30, 0.40, -0.50, 0.60, -0.70, 0.80, 0.90, -1.00, 1.10, -1.20], 3, 4), None,
         [dict(A=f32([0.10, -0.20, 0.30, 0.40, -0.50, 0.60], 3, 2), B=f32([0.70, -0.80, 0.90, 1.00], 2, 2),
               scale=0.5, col0=1)], False, False),
        ("merge_bf16", f32([0.5, -1.0], 1, 2), O.round_bf16(f32([0.10, -0.20, 0.30, 0.40, -0.50, 0.60], 2, 3)),
         None, [dict(A=f32([0.25, -0.50, 0.75, 0.125], 2, 2), B=f32([0.40, -0.30, 0.20, 0.10], 2, 2), scale=1.0,
                     col0=1)], False, True),
        ("clear", f32([1.0, 2.0], 1, 2), O.round_bf16(f32([0.1, 0.2, 0.3, 0.4], 2, 2)), None,
         [dict(A=f32([0.5, -0.25], 2, 1), B=f32([0.75, -0.5], 1, 2), scale=1.0)], False, True),
    ]
    for i, (N, I, Od, wt, wb, bias, specs) in enumerate([
            (24, 40, 36, False, False, True, [(4, 0.5, 0, 36, False, False), (2, 2.0, 8, 12, True, True)]),
            (17, 33, 48, True, True, False, [(8, 2.0, 0, 48, True, False)]),
            (40, 64, 96, False, True, True, [(8, 0.25, 0, 32, False, False), (8, 0.25, 32, 32, False, False),
                                             (8, 0.25, 64, 32, False, True)])]):
        seed = 7000 + 10 * i
        x = O.normal(N * I, seed, 0).reshape(N, I)
        W = (0.2 * O.normal(I * Od, seed, 1)).reshape((Od, I) if wt else (I, Od))
        if wb:
            W = O.round_bf16(W)
        b = O.normal(Od, seed, 2) if bias else None
        sl = []
        for j, (r, sc, c0, cols, at, bt) in enumerate(specs):
            A = (0.3 * O.normal(I * r, seed, 10 + j)).reshape((r, I) if at else (I, r))
            Bm = (0.3 * O.normal(r * cols, seed, 20 + j)).reshape((cols, r) if bt else (r, cols))
            sl.append(dict(A=A, B=Bm, scale=sc, col0=c0, a_transposed=at, b_transposed=bt))
        cases.append((f"rand{i}", x, W, b, sl, wt, wb))
    out = []
    for name, x, W, b, sl, wt, wb in cases:
        out_dim = W.shape[0] if wt else W.shape[1]
        dy = O.normal(x.shape[0] * out_dim, 7500 + len(out), 3).reshape(x.shape[0], out_dim)
        out.append((name, x, W, b, sl, wt, wb, dy))
    return out


def make_lora():
    """tests/golden/lora.npz: the reference's LoRALinear forward, Engine
    backward (dx, grad_A, grad_B) and merge_to_base, and whether the oracle
    matched each bit for bit."""
    out = {}
    ok = True
    cases = lora_cases()
    for name, x, W, b, sl, wt, wb, dy in cases:
        r = O.ref_lora(x, W, b, sl, w_transposed=wt, dy=dy, w_bf16=wb)
        m = O.lora(x, W, b, sl, w_transposed=wt, dy=dy, w_bf16=wb)
        ok = ok and bitwise(m["y"], r["y"]) and bitwise(m["dx"], r["dx"])
        out[f"{name}_x"], out[f"{name}_W"], out[f"{name}_dy"] = x, W, dy
        out[f"{name}_flags"] = np.array([int(wt), int(wb), len(sl), int(b is not None)], np.int64)
        if b is not None:
            out[f"{name}_bias"] = b
        out[f"{name}_y"], out[f"{name}_dx"] = r["y"], r["dx"]
        for j, s in enumerate(sl):
            out[f"{name}_s{j}_A"], out[f"{name}_s{j}_B"] = s["A"], s["B"]
            out[f"{name}_s{j}_meta"] = np.array([s.get("col0", 0), int(s.get("a_transposed", False)),
                                                 int(s.get("b_transposed", False))], np.int64)
            out[f"{name}_s{j}_scale"] = np.float32(s["scale"])
            has = r["grad_A"][j] is not None
            ok = ok and has == (m["grad_A"][j] is not None)
            if has:
                out[f"{name}_s{j}_grad_A"], out[f"{name}_s{j}_grad_B"] = r["grad_A"][j], r["grad_B"][j]
                ok = ok and bitwise(m["grad_A"][j], r["grad_A"][j]) and bitwise(m["grad_B"][j], r["grad_B"][j])
        if not wt:
            rm = O.ref_lora_merge(W, sl, w_bf16=wb)
            ok = ok and bitwise(O.lora_merge(W, sl, w_bf16=wb), rm)
            out[f"{name}_merged"] = rm
    out["names"] = np.array([c[0] for c in cases])
    out["refcpu_bitwise"] = np.array(ok)
    path = os.path.join(HERE, "lora.npz")
    np.savez_compressed(path, **out)
    print(f"lora: {len(cases)} cases, refcpu bitwise = {ok} -> {path}")


def main(argv):
    if not O.ref_available():
        O.build()
    if not O.ref_available():
        raise SystemExit("oracle/_ref/libmftref.so could not be built (needs /root/reference)")
    todo = argv or ["tiny", "prologue", "lm_loss", "lora", "c1", "c2", "c4", "c5", "c5f32", "c3"]
    for t in todo:
        if t == "tiny":
            make_tiny()
        elif t == "prologue":
            make_prologue()
        elif t == "lm_loss":
            make_lm_loss()
        elif t == "lora":
            make_lora()
        else:
            make_config(t)


if __name__ == "__main__":
    main(sys.argv[1:])
