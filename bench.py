#!/usr/bin/env python3
"""Benchmark of the fused causal GQA attention fwd+bwd on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c5] [--headline-only]
                    [--no-cpu-baseline] [--no-variants]

A step is one forward plus one backward of the attention over the config's
synthetic batch (inputs resident in HBM).  Prints ONE JSON line.  `value` is
the algorithmic causal throughput  7*B*H*D*S*(S+1) / step time  in TFLOP/s
(forward 2 and backward 5 products over the causal triangle with its
diagonal, per query head) of the --config workload (C5 by default).

Also on the line:
  per_config    every BASELINE config (C1-C5 and the C5 fp32 variant): step
                time, TFLOP/s, tokens/s, % of the dtype's MFMA peak, and the
                roofline object of its dominant kernel;
  saved_bytes   bytes held from forward to backward, measured on both sides:
                the reference composite graph's MemoryManager bytes, and the
                drop-in autograd node's device bytes (its allocator) and host
                bytes (MemoryManager);
  dropin_step   forward + backward through the finetune_ops drop-in with host
                tensors in and out (PCIe copies included) at C1, C2 and C5
                (C5 also with an [S,S] causal mask tensor, as GPT-2 passes
                one), beside its transfer floor: the step's host<->device
                bytes over the box's measured pinned-copy rates;
  variants      Gemma's sliding window (c5w512), right-padded batches (c4pad)
                and the [B,S,H,D] operand layout (c5bshd); their flops count
                the visible (query, key) pairs only;
  prologue / lm_loss / lora   the widened-path kernels (HBM or MFMA roofline);
  cpu_baseline  the reference's own CPU operators (oracle/_ref, compiled from
                the reference sources) over the config, one (batch, head)
                slice per host core.
The roofline objects cover the dominant kernel, timed live with HIP events
on the stream the kernels run on.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

METRIC = "causal GQA attn fwd+bwd TFLOP/s & % MFMA peak (1 GPU); saved-act bytes"
PEAK_TFLOPS = {"bf16": 2500.0, "f32": 157.3}  # MI355X dense MFMA (published)
# Warm-up floor: W warm-up steps are a minimum; warm-up continues until this
# much wall time of them has run.  A cold MI355X ramps its clocks over the
# first ~100 C5 steps (~25 ms): successive 50-step rounds from a cold start
# measured 303, 223, 217, 215, 215 ... us per step.
WARM_FLOOR_S = 0.15


def warm_up(fn, warmup):
    """Run fn untimed at least `warmup` times and for at least WARM_FLOOR_S
    (synchronizing every 10 calls, so that the wall time is the GPU's);
    returns the number of calls."""
    import torch
    n, t0 = 0, time.perf_counter()
    while n < warmup or time.perf_counter() - t0 < WARM_FLOOR_S:
        fn()
        n += 1
        if n % 10 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return n
HBM_GBS = 8000.0

# BASELINE.json configs (shapes, dtype, scale, dO sigma); all causal.
CONFIGS = {
    "c1": dict(B=4, Hq=12, Hkv=12, D=64, S=128, dtype="f32", scale=1 / 8, do_sigma=1.0,
               name="GPT-2-small attention fwd+bwd, fp32, causal MHA"),
    "c2": dict(B=4, Hq=16, Hkv=16, D=64, S=512, dtype="f32", scale=1 / 8, do_sigma=0.1,
               name="GPT-2-medium attention fwd+bwd, fp32, causal MHA"),
    "c3": dict(B=2, Hq=14, Hkv=2, D=64, S=2048, dtype="bf16", scale=1 / 8, do_sigma=0.1,
               name="Qwen2.5-0.5B-shaped GQA attention fwd+bwd, bf16 in / fp32 accumulate"),
    "c4": dict(B=4, Hq=4, Hkv=1, D=256, S=1024, dtype="bf16", scale=1 / 16, do_sigma=0.1,
               name="Gemma-3-270M-shaped GQA attention fwd+bwd, bf16"),
    "c5": dict(B=1, Hq=4, Hkv=1, D=256, S=4096, dtype="bf16", scale=1 / 16, do_sigma=0.1,
               name="Gemma-3-1B-shaped GQA attention fwd+bwd, bf16"),
    "c5f32": dict(B=1, Hq=4, Hkv=1, D=256, S=4096, dtype="f32", scale=1 / 16, do_sigma=0.1,
                  name="Gemma-3-1B-shaped GQA attention fwd+bwd, fp32 exactness variant"),
    # Mask variants of the model graphs (not BASELINE configs): Gemma-3's
    # sliding layers (sliding_window 512) at the c5 shape, and a right-padded
    # batch (lengths per sequence) at the c4 shape.
    "c5w512": dict(B=1, Hq=4, Hkv=1, D=256, S=4096, dtype="bf16", scale=1 / 16, do_sigma=0.1, window=512,
                   name="Gemma-3-1B-shaped sliding-window layer (window 512) fwd+bwd, bf16"),
    "c4pad": dict(B=4, Hq=4, Hkv=1, D=256, S=1024, dtype="bf16", scale=1 / 16, do_sigma=0.1,
                  lengths=[1024, 700, 400, 130],
                  name="Gemma-3-270M-shaped fwd+bwd with right-padded sequences, bf16"),
    # The models' [B,S,H,D] projection layout passed as strided views (no permute copies).
    "c5bshd": dict(B=1, Hq=4, Hkv=1, D=256, S=4096, dtype="bf16", scale=1 / 16, do_sigma=0.1, layout="bshd",
                   name="Gemma-3-1B-shaped GQA attention fwd+bwd on [B,S,H,D] views, bf16"),
}


def visible_pairs(S, window=0, length=None):
    """(query, key) pairs the causal mask, a sliding window and key padding
    leave visible in one (batch, head)."""
    n = S if length is None else length
    w = window if window else S
    # row i sees the keys j in [max(0, i - w + 1), min(i, n - 1)]
    tot = 0
    for i in range(S):
        lo, hi = max(0, i - w + 1), min(i, n - 1)
        tot += max(0, hi - lo + 1)
    return tot


def flop_units(c):
    """2*D flops per visible (query, key) pair per query head: D*S*(S+1) for
    the plain causal mask."""
    lengths = c.get("lengths") or [None] * c["B"]
    return c["Hq"] * c["D"] * 2 * sum(visible_pairs(c["S"], c.get("window", 0), n) for n in lengths)


def gpu_leg(cfg_id, steps, warmup):
    import torch
    from mobilefinetuner_amd import attention as A
    from mobilefinetuner_amd import capi

    c = CONFIGS[cfg_id]
    dev = torch.device("cuda:0")
    dt = torch.bfloat16 if c["dtype"] == "bf16" else torch.float32
    g = torch.Generator(device=dev)
    g.manual_seed(1000 + sum(map(ord, cfg_id)))
    B, Hq, Hkv, S, D = c["B"], c["Hq"], c["Hkv"], c["S"], c["D"]
    q = torch.randn(B, Hq, S, D, device=dev, generator=g).to(dt)
    k = torch.randn(B, Hkv, S, D, device=dev, generator=g).to(dt)
    v = torch.randn(B, Hkv, S, D, device=dev, generator=g).to(dt)
    dO = (torch.randn(B, Hq, S, D, device=dev, generator=g) * c["do_sigma"]).to(dt)
    if c.get("layout") == "bshd":  # [B,S,H,D] storage, passed as [B,H,S,D] views
        q, k, v, dO = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (q, k, v, dO))
    scale = c["scale"]
    window = c.get("window", 0)
    kv_len = torch.tensor(c["lengths"], dtype=torch.int32, device=dev) if c.get("lengths") else None
    ws = torch.empty(max(A.workspace_bytes(q, k, scale, True, window, kv_len), 1), dtype=torch.uint8, device=dev)
    fws_n = A.fwd_workspace_bytes(q, k, scale, True, window, kv_len)
    fws = torch.empty(max(fws_n, 1), dtype=torch.uint8, device=dev)
    o = torch.empty_like(q)
    lse = torch.empty(B, Hq, S, dtype=torch.float32, device=dev)
    dq = torch.empty_like(q, dtype=torch.float32)
    dk = torch.empty_like(k, dtype=torch.float32)
    dv = torch.empty_like(v, dtype=torch.float32)
    d = A._desc(q, k, scale, True, window, kv_len, dict(q=q, k=k, v=v, o=o, dO=dO, dq=dq, dk=dk, dv=dv))
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    P = [t.data_ptr() for t in (q, k, v, o, dO, lse, dq, dk, dv, ws)]

    fws_ptr = fws.data_ptr() if fws_n else None

    def fwd():
        capi.attn_fwd(d, P[0], P[1], P[2], P[3], P[5], fws_ptr, sp)

    def bwd():
        capi.attn_bwd(d, P[0], P[1], P[2], P[3], P[4], P[5], P[6], P[7], P[8], P[9], sp)

    def stage(mask):
        return lambda: capi.attn_bwd_stage(d, mask, P[0], P[1], P[2], P[3], P[4], P[5], P[6], P[7], P[8],
                                           P[9], sp)

    def timed(fn, n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n  # ms

    warm_n = warm_up(lambda: (fwd(), bwd()), warmup)
    step_ms = timed(lambda: (fwd(), bwd()), steps)
    n_phase = max(steps, 10)
    fwd_ms = timed(fwd, n_phase)
    bwd_ms = timed(bwd, n_phase)
    stage(capi.MFT_BWD_DELTA)()  # row terms for the gradient stages
    main_ms = timed(stage(capi.MFT_BWD_MAIN), n_phase)
    units = flop_units(c)
    return dict(step_ms=step_ms, fwd_ms=fwd_ms, bwd_ms=bwd_ms, main_ms=main_ms, units=units, warm_n=warm_n)


def prologue_leg(cfg_id, steps, warmup):
    """The fused q/k prologue (norm + RoPE) at a config's q and k shapes, on
    [B,S,H,D] projection outputs viewed [B,H,S,D] (Gemma-3: rms_norm with
    (1 + w), eps 1e-6, rope_theta 1e6), bf16 x/y, fp32 dy/dx.  HBM-bound:
    algorithmic bytes per element are 2 (x) + 2 (y) forward and 2 (x) + 4 (dy)
    + 4 (dx) backward, plus the [waves, D] dw partials written and re-read.
    The q and k heads run as one batch (mft_prologue_fwd_n / _bwd_n: one
    launch forward, two backward); "separate" times one call per tensor."""
    import torch
    from mobilefinetuner_amd import attention as A
    from mobilefinetuner_amd import capi

    c = CONFIGS[cfg_id]
    dev = torch.device("cuda:0")
    B, S, D = c["B"], c["S"], c["D"]
    g = torch.Generator(device=dev)
    g.manual_seed(77)
    sp = torch.cuda.current_stream().cuda_stream
    calls, fwd_bytes, bwd_bytes = [], 0, 0
    for H in (c["Hq"], c["Hkv"]):
        x = torch.randn(B, S, H, D, device=dev, generator=g).to(torch.bfloat16).transpose(1, 2)
        w = 0.3 * torch.randn(D, device=dev, generator=g)
        dy = torch.randn(B, S, H, D, device=dev, generator=g).transpose(1, 2)
        y = torch.empty(B, H, S, D, dtype=torch.bfloat16, device=dev)
        dx = torch.empty(B, H, S, D, dtype=torch.float32, device=dev)
        dw = torch.empty(D, dtype=torch.float32, device=dev)
        d = A._prologue_desc(x, "gemma", 1e-6, 1e6, dict(x=x, dy=dy))
        wsb = capi.prologue_workspace_size(d)
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
        n = B * H * S * D
        fwd_bytes += 4 * n
        bwd_bytes += 10 * n + 2 * wsb
        calls.append((d, x, w, y, dy, dx, dw, ws))

    def fwd1():
        for d, x, w, y, *_ in calls:
            capi.prologue_fwd(d, x.data_ptr(), w.data_ptr(), y.data_ptr(), sp)

    def bwd1():
        for d, x, w, y, dy, dx, dw, ws in calls:
            capi.prologue_bwd(d, x.data_ptr(), w.data_ptr(), dy.data_ptr(), dx.data_ptr(), dw.data_ptr(),
                              ws.data_ptr(), sp)

    ds = [cl[0] for cl in calls]
    ptr = lambda i: [cl[i].data_ptr() for cl in calls]
    wsn = torch.empty(max(capi.prologue_workspace_size_n(ds), 1), dtype=torch.uint8, device=dev)

    def fwd():
        capi.prologue_fwd_n(ds, ptr(1), ptr(2), ptr(3), sp)

    def bwd():
        capi.prologue_bwd_n(ds, ptr(1), ptr(2), ptr(4), ptr(5), ptr(6), wsn.data_ptr(), sp)

    def timed(fn, n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    warm_up(lambda: (fwd(), bwd(), fwd1(), bwd1()), warmup)
    f_ms, b_ms = timed(fwd, steps), timed(bwd, steps)
    f1_ms, b1_ms = timed(fwd1, steps), timed(bwd1, steps)
    return {"workload": f"q/k rms_norm(1+w) + RoPE of {cfg_id} (Hq {c['Hq']} + Hkv {c['Hkv']} heads, S {S}, D {D}), "
                        "[B,S,H,D] bf16 in, [B,H,S,D] out",
            "fwd_us": round(f_ms * 1e3, 2), "bwd_us": round(b_ms * 1e3, 2),
            "fwd_GBps": round(fwd_bytes / (f_ms * 1e-3) / 1e9, 1), "bwd_GBps": round(bwd_bytes / (b_ms * 1e-3) / 1e9, 1),
            "fwd_frac_hbm": round(fwd_bytes / (f_ms * 1e-3) / 8e12, 4),
            "bwd_frac_hbm": round(bwd_bytes / (b_ms * 1e-3) / 8e12, 4),
            "fwd_bytes": fwd_bytes, "bwd_bytes": bwd_bytes, "launches": {"fwd": 1, "bwd": 2},
            "separate": {"fwd_us": round(f1_ms * 1e3, 2), "bwd_us": round(b1_ms * 1e3, 2),
                         "launches": {"fwd": 2, "bwd": 4}}}


def lm_loss_leg(cfg_id, steps, warmup):
    """LM cross-entropy at the Gemma-3-1B head (H 1152, V 262144) over the
    config's B*S positions, bf16.  Streaming (hidden, weight): four GEMMs of
    2*N*V*H flop per step (forward logits; backward logits again, d hidden,
    d weight), MFMA roofline.  Dense (given bf16 logits [B, S, V]): HBM
    roofline, algorithmic bytes 2*N*V forward and 2*N*V + 4*N*V backward."""
    import torch
    from mobilefinetuner_amd import lm_loss as L

    c = CONFIGS[cfg_id]
    dev = torch.device("cuda:0")
    B, S, H, V = c["B"], c["S"], 1152, 262144
    N = B * S
    g = torch.Generator(device=dev)
    g.manual_seed(99)
    hidden = (0.5 * torch.randn(B, S, H, device=dev, generator=g)).to(torch.bfloat16)
    weight = (0.05 * torch.randn(V, H, device=dev, generator=g)).to(torch.bfloat16)
    labels = torch.randint(0, V, (B, S), device=dev, generator=g, dtype=torch.int32)
    one = torch.ones(1, device=dev)

    def timed(fn, n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        warm_up(fn, warmup)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    state = {}

    def s_fwd():
        state["lse"] = L.streaming_lm_cross_entropy(hidden, weight, labels, check_labels=False)[1]

    s_fwd()

    def s_bwd():
        L.streaming_lm_cross_entropy_backward(hidden, weight, labels, state["lse"], one)

    sf, sb = timed(s_fwd, steps), timed(s_bwd, steps)
    flop = 2.0 * N * V * H
    out = {"workload": f"Gemma-3-1B LM head (H {H}, V {V}) over the {cfg_id} batch ({N} positions), bf16",
           "streaming": {"fwd_ms": round(sf, 4), "bwd_ms": round(sb, 4),
                         "fwd_tflops": round(flop / (sf * 1e-3) / 1e12, 1),
                         "bwd_tflops": round(3 * flop / (sb * 1e-3) / 1e12, 1),
                         "frac_mfma_peak": round(4 * flop / ((sf + sb) * 1e-3) / 1e12 / PEAK_TFLOPS["bf16"], 4)}}
    del state["lse"]
    logits = torch.randn(B, S, V, device=dev, generator=g).to(torch.bfloat16)

    def d_fwd():
        state["lse"] = L.lm_cross_entropy(logits, labels, check_labels=False)[1]

    d_fwd()

    def d_bwd():
        L.lm_cross_entropy_backward(logits, labels, state["lse"], one)

    df, db = timed(d_fwd, steps), timed(d_bwd, steps)
    fb, bb = 2.0 * N * V, 6.0 * N * V
    out["dense"] = {"fwd_ms": round(df, 4), "bwd_ms": round(db, 4),
                    "fwd_frac_hbm": round(fb / (df * 1e-3) / (HBM_GBS * 1e9), 4),
                    "bwd_frac_hbm": round(bb / (db * 1e-3) / (HBM_GBS * 1e9), 4)}
    return out


def lora_leg(cfg_id, steps, warmup):
    """LoRA linear layers of Gemma-3-1B over the config's B*S positions, as
    the reference's injector builds them (graph/gemma_lora_injector.cpp:80-150):
    W bf16 [out, in] (frozen), x fp32, A [r, in], B [out, r] fp32, r = 8,
    scale = 2.  Forward y = x W^T + 2 (x A^T) B^T; backward dx, grad_A,
    grad_B.  The products with W run on the bf16 MFMA path: 2*N*in*out flop
    each way (MFMA roofline); the rank-8 products are fp32 and counted too."""
    import torch
    from mobilefinetuner_amd import capi

    c = CONFIGS[cfg_id]
    dev = torch.device("cuda:0")
    N, r = c["B"] * c["S"], 8
    st = torch.cuda.current_stream().cuda_stream
    g = torch.Generator(device=dev)
    g.manual_seed(7)

    def timed(fn, n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        warm_up(fn, warmup)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    out = {"workload": f"Gemma-3-1B LoRA projections (r {r}, W bf16 [out, in], x fp32) over the {cfg_id} batch "
                       f"({N} positions)"}
    for name, I, O in (("q_proj", 1152, 1024), ("gate_proj", 1152, 6912)):
        x = torch.randn(N, I, device=dev, generator=g)
        W = (0.03 * torch.randn(O, I, device=dev, generator=g)).to(torch.bfloat16)
        A = 0.02 * torch.randn(r, I, device=dev, generator=g)
        Bm = 0.02 * torch.randn(O, r, device=dev, generator=g)
        dy = torch.randn(N, O, device=dev, generator=g)
        y, u, dx = torch.empty(N, O, device=dev), torch.empty(N, r, device=dev), torch.empty_like(x)
        gA, gB = torch.empty_like(A), torch.empty_like(Bm)
        d = capi.lora_desc(N, I, O, capi.MFT_BF16, True,
                           [dict(A=A.data_ptr(), B=Bm.data_ptr(), grad_A=gA.data_ptr(), grad_B=gB.data_ptr(),
                                 scale=2.0, rank=r, col0=0, cols=O, a_transposed=True, b_transposed=True)])
        fw, bw = capi.lora_workspace_size(d)
        ws = torch.empty(max(fw, bw), dtype=torch.uint8, device=dev)
        fwd = lambda: capi.lora_fwd(d, x.data_ptr(), W.data_ptr(), None, y.data_ptr(), u.data_ptr(), ws.data_ptr(),
                                    st)
        bwd = lambda: capi.lora_bwd(d, x.data_ptr(), W.data_ptr(), dy.data_ptr(), u.data_ptr(), dx.data_ptr(),
                                    ws.data_ptr(), st)
        fwd()
        tf, tb = timed(fwd, steps), timed(bwd, steps)
        base = 2.0 * N * I * O
        low_f, low_b = 2.0 * N * r * (I + O), 2.0 * N * r * (2 * O + 2 * I)
        out[name] = {"in": I, "out": O, "fwd_ms": round(tf, 4), "bwd_ms": round(tb, 4),
                     "fwd_tflops": round((base + low_f) / (tf * 1e-3) / 1e12, 1),
                     "bwd_tflops": round((base + low_b) / (tb * 1e-3) / 1e12, 1),
                     "frac_mfma_peak": round(2 * base / ((tf + tb) * 1e-3) / 1e12 / PEAK_TFLOPS["bf16"], 4)}
    return out


COPY_BYTES = 1 << 30


def copy_calibration():
    """A plain elementwise copy (reads COPY_BYTES, writes COPY_BYTES): the
    known-size kernel that rocprofv3's FETCH_SIZE / WRITE_SIZE are scaled by."""
    import torch
    x = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda:0")
    y = torch.empty_like(x)
    for _ in range(3):
        torch.mul(x, 1.0, out=y)
    torch.cuda.synchronize()


def hbm_traffic(cfg_id, kernel):
    """HBM bytes per launch of `kernel` from the committed pmc summary
    (profiles/hbm_traffic_<config>.json, written by
    `python -m mobilefinetuner_amd.profiling traffic`), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"hbm_traffic_{cfg_id}.json")
    try:
        with open(path) as fh:
            return json.load(fh)["kernels"][kernel]["hbm_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def _cpu_share():
    """Host cores this process may use, capped at one GPU's CPU share (16)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_slice(task):
    """Worker process: one (batch, query head) slice of a config through the
    reference composite, forward + Engine backward; returns its seconds."""
    cfg_id, b, h, S, kind, rep = task
    from oracle import oracle as O
    c = CONFIGS[cfg_id]
    q, k, v, dO = O.make_inputs(1, 1, 1, S, c["D"], 4242 + 97 * b + h + 7919 * rep, c["dtype"], c["do_sigma"])
    if kind == "reference":
        r = O.ref_composite(q, k, v, dO, scale=c["scale"], causal=True)
        return r["t_fwd"] + r["t_bwd"]
    t0 = time.perf_counter()
    O.composite(q, k, v, dO, scale=c["scale"], causal=True)
    return time.perf_counter() - t0


def _cpu_saved(cfg_id):
    """Worker process: bytes the reference composite's autograd graph holds
    from forward to backward (MemoryManager::get_memory_usage() after the
    forward minus before it, core/memory_manager.h:144) for the whole config."""
    from oracle import oracle as O
    c = CONFIGS[cfg_id]
    q, k, v, _ = O.make_inputs(c["B"], c["Hq"], c["Hkv"], c["S"], c["D"], 4242, c["dtype"], c["do_sigma"])
    return O.ref_saved_bytes(q, k, v, scale=c["scale"], causal=True)


def cpu_leg(cfg_id, saved_cfgs=()):
    """The reference CPU path on the host's cores, run before the GPU is
    touched.  The reference operators are single-threaded, so the config is
    cut into (batch, query head) slices, each run by its own worker process
    (one core each) through the reference composite built from its own
    sources; value = the slices' flops / the slowest slice's seconds.  When
    the config has fewer slices than cores, whole copies of its slices (own
    seeds) fill the cores, so the figure is the host's throughput.  The
    reference's CMake links BLAS only when find_package(BLAS) finds one
    (operator/CMakeLists.txt:164-190); this image has none, so the build is
    its pure-C++ GEMM (DISABLE_BLAS_COMPLETELY, core/ops.cpp:768-794).  Also
    measures the reference's saved-activation bytes for `saved_cfgs`."""
    import multiprocessing as mp
    from oracle import oracle as O
    c = CONFIGS[cfg_id]
    B, Hq, S, D = c["B"], c["Hq"], c["S"], c["D"]
    while 7 * D * S * (S + 1) > 1.5e11:  # keep one slice within ~30 s
        S //= 2
    kind = "reference" if O.ref_available() else "port"
    cores = _cpu_share()
    slices = [(cfg_id, b, h, S, kind, 0) for b in range(B) for h in range(Hq)]
    if len(slices) > cores:  # whole rounds of one slice per worker
        slices = slices[:cores * (len(slices) // cores)]
    else:  # whole copies of the config's slices, one slice per core
        slices = [(cfg_id, b, h, S, kind, r) for r in range(cores // len(slices)) for (_, b, h, _, _, _) in slices]
    copies = 1 + max(t[5] for t in slices)
    workers = min(cores, len(slices))
    ctx = mp.get_context("spawn")
    with ctx.Pool(workers) as pool:
        t0 = time.perf_counter()
        secs = pool.map(_cpu_slice, slices, chunksize=1)
        wall = time.perf_counter() - t0
        saved = dict(zip(saved_cfgs, pool.map(_cpu_saved, saved_cfgs, chunksize=1))) if kind == "reference" else {}
    busiest = max(secs) if len(slices) <= workers else wall
    flops = 7.0 * D * S * (S + 1) * len(slices)
    return dict(value=round(flops / busiest / 1e12, 6), unit="TFLOP/s", cores=workers, kind=kind,
                seconds=round(busiest, 3), cpu_seconds=round(sum(secs), 3), wall_seconds=round(wall, 3),
                nproc=os.cpu_count(), cpu_share=cores, cpu_model=_cpu_model(), blas="none (pure C++ GEMM)",
                sample=f"{cfg_id}: {len(slices)} (batch, query head) slices of S={S}, D={D}"
                       f"{f' ({copies} copies of the config, own seeds)' if copies > 1 else ''}, one per worker "
                       f"process: fp32 reference composite fwd+bwd (transpose/matmul/mul/add-mask/softmax/"
                       f"matmul + Engine backward; a slice has one kv head, so no repeat_kv), reference "
                       f"sources built pure C++ (no BLAS in the image), 1 thread per slice"), saved


DROPIN_PROBE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "mobilefinetuner_amd", "adapter", "_dropin",
                            "dropin_probe")


def dropin_probe(mode, cfg_id, *extra):
    """Run the drop-in probe (reference API over the HIP kernels, host tensors
    in and out) as a child process; its JSON object, or None when the drop-in
    is not built."""
    import subprocess
    if not os.path.exists(DROPIN_PROBE):
        return None
    c = CONFIGS[cfg_id]
    cmd = [DROPIN_PROBE, mode, *(str(c[x]) for x in ("B", "Hq", "Hkv", "S", "D")), c["dtype"], *map(str, extra)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    if res.returncode != 0:
        raise RuntimeError(f"dropin_probe {mode} {cfg_id} failed: {res.stderr[-2000:]}")
    return json.loads(res.stdout.strip().splitlines()[-1])


def roofline_of(cfg_id, r):
    """Roofline object of a config's dominant kernel: the longer of the
    forward and the backward's main launch (dK/dV and dQ work units in one
    grid); achieved = its algorithmic flops / its measured launch time.
    Algorithmic work per launch in causal contraction units (D*S*(S+1) per
    query head): forward 2 (QK^T, PV; the forward call also holds the small
    partial-merge launch); backward main 5 (QK^T recompute, dO V^T, P^T dO,
    dS^T Q, dS K) - the dQ units' second QK^T and dO V^T recomputes are not
    counted."""
    c = CONFIGS[cfg_id]
    peak = PEAK_TFLOPS[c["dtype"]]
    kern = {"attn_fwd": (r["fwd_ms"], 2), "attn_bwd_main": (r["main_ms"], 5)}
    dom = max(kern, key=lambda k: kern[k][0])
    ach = kern[dom][1] * r["units"] / (kern[dom][0] * 1e-3) / 1e12
    traffic = hbm_traffic(cfg_id, dom)
    out = {"bound": "mfma", "kernel": dom, "achieved": round(ach, 2), "peak": peak, "unit": "TFLOP/s",
           "frac": round(ach / peak, 4), "traffic": traffic}
    if traffic:
        out["hbm_GBps"] = round(traffic / (kern[dom][0] * 1e-3) / 1e9, 1)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c5", choices=sorted(CONFIGS))
    ap.add_argument("--headline-only", action="store_true",
                    help="skip the per_config report (C1-C5, C5 fp32) and measure the --config workload only")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-variants", action="store_true", help="skip the mask and layout variants (variants key)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain copy of COPY_BYTES (for scaling rocprofv3 FETCH/WRITE_SIZE)")
    ap.add_argument("--leg", choices=("prologue", "lm_loss", "lora"),
                    help="run only this widened-path leg and print its JSON object (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the attention path is built and measured on a single "
              "MI355X (multi-GPU sharding is design-only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.leg:
        leg = {"prologue": prologue_leg, "lm_loss": lm_loss_leg, "lora": lora_leg}[args.leg]
        print(json.dumps(leg(args.config, args.steps, args.warmup)), flush=True)
        return

    c = CONFIGS[args.config]
    per_ids = () if args.headline_only else ("c1", "c2", "c3", "c4", "c5", "c5f32")
    cpu, ref_saved = None, {}
    if not args.no_cpu_baseline:  # before the GPU is touched: it spawns worker processes
        saved_ids = sorted({args.config, *(i for i in per_ids if i != "c5f32")})
        cpu, ref_saved = cpu_leg(args.config, saved_ids)
        if "c5" in ref_saved:  # the reference composite runs fp32 for either input rounding
            ref_saved.setdefault("c5f32", ref_saved["c5"])

    r = gpu_leg(args.config, args.steps, args.warmup)
    units = r["units"]
    peak = PEAK_TFLOPS[c["dtype"]]
    tflops = 7 * units / (r["step_ms"] * 1e-3) / 1e12
    fwd_tf = 2 * units / (r["fwd_ms"] * 1e-3) / 1e12
    out = {
        "metric": METRIC,
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_steps_run": r["warm_n"],  # W is a minimum; see WARM_FLOOR_S
        "ms_per_step": round(r["step_ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": c["dtype"],
        "data": "synthetic: seeded Q,K,V ~ N(0,1), dO ~ N(0,0.1) (sigma), resident in HBM",
        "config": {"workload": f"{args.config}: {c['name']}", "B": c["B"], "Hq": c["Hq"], "Hkv": c["Hkv"],
                   "S": c["S"], "D": c["D"], "causal": True, "scale": c["scale"],
                   **({"window": c["window"]} if c.get("window") else {}),
                   **({"kv_len": c["lengths"]} if c.get("lengths") else {}),
                   **({"layout": c["layout"]} if c.get("layout") else {})},
        "pct_mfma_peak": round(100 * tflops / peak, 2),
        "tokens_per_s": round(c["B"] * c["S"] / (r["step_ms"] * 1e-3), 1),
        "fwd_ms": round(r["fwd_ms"], 5),
        "bwd_ms": round(r["bwd_ms"], 5),
        "bwd_main_ms": round(r["main_ms"], 5),
        "fwd_tflops": round(fwd_tf, 2),
        "bwd_tflops": round(5 * units / (r["bwd_ms"] * 1e-3) / 1e12, 2),
        "roofline": roofline_of(args.config, r),
    }
    per = {}
    for cid in per_ids:
        cc = CONFIGS[cid]
        rr = r if cid == args.config else gpu_leg(cid, max(10, args.steps // 2), 5)
        u = rr["units"]
        tf = 7 * u / (rr["step_ms"] * 1e-3) / 1e12
        per[cid] = {"workload": cc["name"], "dtype": cc["dtype"], "ms_per_step": round(rr["step_ms"], 5),
                    "fwd_ms": round(rr["fwd_ms"], 5), "bwd_ms": round(rr["bwd_ms"], 5),
                    "bwd_main_ms": round(rr["main_ms"], 5), "tflops": round(tf, 2),
                    "pct_peak": round(100 * tf / PEAK_TFLOPS[cc["dtype"]], 2),
                    "tokens_per_s": round(cc["B"] * cc["S"] / (rr["step_ms"] * 1e-3), 1),
                    "roofline": roofline_of(cid, rr)}
    if per:
        out["per_config"] = per
    # Saved-activation bytes, measured on both sides: the reference composite
    # graph's MemoryManager bytes, and the drop-in's autograd node (device
    # bytes from its allocator, host bytes from MemoryManager).
    saved = {}
    for cid in sorted({args.config, *per_ids}):
        ent = {"reference": ref_saved.get(cid)}
        d = dropin_probe("saved", cid)
        if d is not None:
            ent.update(dropin_device=d["device_bytes"], dropin_host=d["host_bytes"])
            if ent["reference"]:
                ent["ratio"] = round(ent["reference"] / (d["device_bytes"] + d["host_bytes"]), 1)
        saved[cid] = ent
    out["saved_bytes"] = saved
    # The PCIe-inclusive step through the drop-in (host tensors in, host
    # gradients out, reference Engine), steady state with cached device memory.
    pcie = {}
    for cid, mask, iters in (("c1", "", 40), ("c2", "", 20), (args.config, "", 20), (args.config, "mask", 20)):
        d = dropin_probe("step", cid, 5, iters, *([mask] if mask else []))
        if d is not None:
            pcie[cid + ("_mask" if mask else "")] = d
    if pcie:
        out["dropin_step"] = pcie
    variants = {}
    for cid in () if args.no_variants else ("c5w512", "c4pad", "c5bshd"):
        cc = CONFIGS[cid]
        rr = gpu_leg(cid, max(10, args.steps // 2), 5)
        u = rr["units"]
        tf = 7 * u / (rr["step_ms"] * 1e-3) / 1e12
        variants[cid] = {"workload": cc["name"], "window": cc.get("window", 0), "lengths": cc.get("lengths"),
                         "layout": cc.get("layout", "bhsd"),
                         "ms_per_step": round(rr["step_ms"], 5), "fwd_ms": round(rr["fwd_ms"], 5),
                         "bwd_ms": round(rr["bwd_ms"], 5), "tflops": round(tf, 2),
                         "pct_peak": round(100 * tf / PEAK_TFLOPS[cc["dtype"]], 2),
                         "tokens_per_s": round(cc["B"] * cc["S"] / (rr["step_ms"] * 1e-3), 1)}
    if variants:
        out["variants"] = variants
    if not args.no_variants:
        out["prologue"] = prologue_leg(args.config, max(20, args.steps), 5)
        out["lm_loss"] = lm_loss_leg(args.config, 5, 2)
        out["lora"] = lora_leg(args.config, 20, 3)
    if args.copy_calibration:
        copy_calibration()
    if cpu is not None:
        out["cpu_baseline"] = cpu
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
