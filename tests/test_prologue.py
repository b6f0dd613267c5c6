"""GPU parity of the fused q/k prologue (mft_prologue_fwd / _bwd through the C
ABI) with the oracle restatement of the reference's rms_norm / rms_norm_affine
+ apply_rope and their backward (itself pinned bit for bit to the reference by
test_prologue_oracle.py).

Bars: fp32 max-rel 1e-4; bf16 2e-2 against the fp32 oracle run on the same
bf16-rounded inputs.  The layout tests require bitwise equality with the
contiguous run; dw must be deterministic.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = {"f32": 1e-4, "bf16": 2e-2}

CASES = [
    # B, H, S, D, dtype, norm, eps, theta
    (1, 4, 300, 256, "f32", "gemma", 1e-6, 1e6),   # Gemma-3 q, global layer
    (2, 1, 257, 256, "bf16", "gemma", 1e-6, 1e4),  # Gemma-3 k, local layer
    (2, 14, 64, 64, "f32", "none", 0.0, 1e6),      # Qwen2.5 RoPE only
    (1, 3, 100, 96, "f32", "affine", 1e-5, 1e4),
    (1, 2, 33, 6, "f32", "gemma", 1e-6, 1e4),      # odd half-dim
    (1, 2, 40, 512, "bf16", "affine", 1e-6, 1e4),  # widest head
    (3, 2, 50, 128, "f32", "gemma", 1e-6, 0.0),    # norm only
    (1, 2, 64, 200, "f32", "gemma", 1e-6, 1e4),    # strided lanes, 2 per half
    (1, 2, 48, 300, "bf16", "affine", 1e-6, 1e6),  # strided lanes, 4 per half
    (2, 3, 70, 128, "bf16", "gemma", 1e-6, 1e6),   # 16-byte lanes, 4 rows per wave access
]


def _id(c):
    return "B{}H{}S{}D{}-{}-{}-t{:g}".format(*c[:6], c[7])


def _dev(x, dtype, dev):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    return t.to(torch.bfloat16) if dtype == "bf16" else t


def _inputs(orc, B, H, S, D, dtype, seed):
    n = B * H * S * D
    x = (2.0 * orc.normal(n, 4000 + seed, 0)).reshape(B, H, S, D)
    if dtype == "bf16":
        x = orc.round_bf16(x)
    w = (0.3 * orc.normal(D, 4000 + seed, 1)).astype(np.float32)
    dy = orc.normal(n, 4000 + seed, 2).reshape(B, H, S, D)
    return x, w, dy


@pytest.mark.parametrize("case", CASES, ids=[_id(c) for c in CASES])
def test_prologue_matches_oracle(orc, dev, case):
    import torch
    from mobilefinetuner_amd import attention as A
    B, H, S, D, dtype, norm, eps, theta = case
    print(f"[case] {_id(case)}", flush=True)
    x, w, dy = _inputs(orc, B, H, S, D, dtype, S + D)
    wn = w if norm != "none" else None
    ref = orc.prologue(x, wn, dy, norm, eps, theta)
    xd = _dev(x, dtype, dev)
    wd = None if wn is None else torch.from_numpy(wn).to(dev)
    y = A.prologue_forward(xd, wd, norm, eps, theta)
    dx, dw = A.prologue_backward(xd, wd, torch.from_numpy(dy).to(dev), norm, eps, theta)
    torch.cuda.synchronize()
    tol = TOL[dtype]
    errs = {"y": orc.max_rel(y.float().cpu().numpy(), ref["y"]), "dx": orc.max_rel(dx.cpu().numpy(), ref["dx"])}
    if norm != "none":
        errs["dw"] = orc.max_rel(dw.cpu().numpy(), ref["dw"])
    print(f"[errs] {errs}", flush=True)
    for k, e in errs.items():
        assert e <= tol, (k, e)


def test_projection_layout_views_match_contiguous_bitwise(orc, dev):
    """x as a [B,S,H,D] projection output viewed [B,H,S,D] (no permute copy),
    dy as a [B,S,H,D] view too: same bits as the contiguous run."""
    import torch
    from mobilefinetuner_amd import attention as A
    B, H, S, D = 2, 4, 129, 256
    x, w, dy = _inputs(orc, B, H, S, D, "bf16", 11)
    xc, wd, dyc = _dev(x, "bf16", dev), torch.from_numpy(w).to(dev), torch.from_numpy(dy).to(dev)
    xs = _dev(x.transpose(0, 2, 1, 3), "bf16", dev).transpose(1, 2)
    dys = torch.from_numpy(np.ascontiguousarray(dy.transpose(0, 2, 1, 3))).to(dev).transpose(1, 2)
    assert not xs.is_contiguous() and not dys.is_contiguous()
    y1 = A.prologue_forward(xc, wd, "gemma", 1e-6, 1e4)
    y2 = A.prologue_forward(xs, wd, "gemma", 1e-6, 1e4)
    g1 = A.prologue_backward(xc, wd, dyc, "gemma", 1e-6, 1e4)
    g2 = A.prologue_backward(xs, wd, dys, "gemma", 1e-6, 1e4)
    # a strided output: y written straight into a [B,S,H,D] buffer
    ybuf = torch.empty(B, S, H, D, dtype=torch.bfloat16, device=dev)
    A.prologue_forward(xs, wd, "gemma", 1e-6, 1e4, out=ybuf.transpose(1, 2))
    torch.cuda.synchronize()
    assert torch.equal(y1, y2) and torch.equal(y1, ybuf.transpose(1, 2))
    assert torch.equal(g1[0], g2[0]) and torch.equal(g1[1], g2[1])


def test_dw_is_deterministic_and_in_place_forward(orc, dev):
    import torch
    from mobilefinetuner_amd import attention as A
    x, w, dy = _inputs(orc, 2, 8, 1000, 128, "f32", 12)
    xd, wd, dyd = _dev(x, "f32", dev), torch.from_numpy(w).to(dev), torch.from_numpy(dy).to(dev)
    a = A.prologue_backward(xd, wd, dyd, "gemma", 1e-6, 1e6)
    b = A.prologue_backward(xd, wd, dyd, "gemma", 1e-6, 1e6)
    y = A.prologue_forward(xd, wd, "gemma", 1e-6, 1e6)
    xin = xd.clone()
    A.prologue_forward(xin, wd, "gemma", 1e-6, 1e6, out=xin)  # y may overwrite x
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    assert torch.equal(xin, y)


def test_c5_shape_positions_up_to_4095(orc, dev):
    """Gemma-3-1B q rows at the headline shape (Hq 4, S 4096, D 256): RoPE
    angles up to 4095 rad, fp32 and bf16."""
    import torch
    from mobilefinetuner_amd import attention as A
    B, H, S, D = 1, 4, 4096, 256
    x, w, dy = _inputs(orc, B, H, S, D, "f32", 13)
    ref = orc.prologue(x, w, dy, "gemma", 1e-6, 1e6)
    for dtype in ("f32", "bf16"):
        xx = orc.round_bf16(x) if dtype == "bf16" else x
        r = ref if dtype == "f32" else orc.prologue(xx, w, dy, "gemma", 1e-6, 1e6)
        xd, wd = _dev(xx, dtype, dev), torch.from_numpy(w).to(dev)
        y = A.prologue_forward(xd, wd, "gemma", 1e-6, 1e6)
        dx, dw = A.prologue_backward(xd, wd, torch.from_numpy(dy).to(dev), "gemma", 1e-6, 1e6)
        torch.cuda.synchronize()
        e = (orc.max_rel(y.float().cpu().numpy(), r["y"]), orc.max_rel(dx.cpu().numpy(), r["dx"]),
             orc.max_rel(dw.cpu().numpy(), r["dw"]))
        print(f"[errs] {dtype} y/dx/dw {e}", flush=True)
        assert max(e) <= TOL[dtype], e


def test_gemma_chain_through_attention(orc, dev):
    """q/k projections -> prologue -> fused attention -> backward -> prologue
    backward, against the oracle chain (graph/gemma_model.cpp:403-505 order:
    rms_norm, apply_rope, then attention with the additive causal mask)."""
    import torch
    from mobilefinetuner_amd import attention as A
    B, Hq, Hkv, S, D = 1, 4, 1, 130, 64
    xq, wq, _ = _inputs(orc, B, Hq, S, D, "f32", 21)
    xk, wk, _ = _inputs(orc, B, Hkv, S, D, "f32", 22)
    v = orc.normal(B * Hkv * S * D, 23, 0).reshape(B, Hkv, S, D)
    dO = orc.normal(B * Hq * S * D, 23, 1, 0.5).reshape(B, Hq, S, D)
    eps, theta, scale = 1e-6, 1e4, 1.0 / 8
    # oracle chain
    q = orc.prologue(xq, wq, None, "gemma", eps, theta)["y"]
    k = orc.prologue(xk, wk, None, "gemma", eps, theta)["y"]
    att = orc.composite(q, k, v, dO, scale=scale, causal=True)
    rq = orc.prologue(xq, wq, att["dq"], "gemma", eps, theta)
    rk = orc.prologue(xk, wk, att["dk"], "gemma", eps, theta)
    # GPU chain
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    qd = A.prologue_forward(d(xq), d(wq), "gemma", eps, theta)
    kd = A.prologue_forward(d(xk), d(wk), "gemma", eps, theta)
    o, lse = A.attention_forward(qd, kd, d(v), scale, True)
    dq, dk, dv = A.attention_backward(qd, kd, d(v), o, d(dO), lse, scale, True)
    gq = A.prologue_backward(d(xq), d(wq), dq, "gemma", eps, theta)
    gk = A.prologue_backward(d(xk), d(wk), dk, "gemma", eps, theta)
    torch.cuda.synchronize()
    errs = dict(o=orc.max_rel(o.cpu().numpy(), att["o"]), dxq=orc.max_rel(gq[0].cpu().numpy(), rq["dx"]),
                dwq=orc.max_rel(gq[1].cpu().numpy(), rq["dw"]), dxk=orc.max_rel(gk[0].cpu().numpy(), rk["dx"]),
                dwk=orc.max_rel(gk[1].cpu().numpy(), rk["dw"]), dv=orc.max_rel(dv.cpu().numpy(), att["dv"]))
    print(f"[errs] {errs}", flush=True)
    for n, e in errs.items():
        assert e <= 1e-4, (n, e)


def test_autograd_nodes_compose(orc, dev):
    """QKPrologue -> FusedAttention under torch autograd gives the same
    gradients as the explicit calls (the nodes save x, w and q, k, v, o, lse)."""
    import torch
    from mobilefinetuner_amd import attention as A
    B, Hq, Hkv, S, D = 1, 2, 1, 70, 64
    xq, wq, _ = _inputs(orc, B, Hq, S, D, "f32", 31)
    xk, wk, _ = _inputs(orc, B, Hkv, S, D, "f32", 32)
    v = orc.normal(B * Hkv * S * D, 33, 0).reshape(B, Hkv, S, D)
    dO = orc.normal(B * Hq * S * D, 33, 1).reshape(B, Hq, S, D)
    d = lambda a, g=False: torch.from_numpy(np.ascontiguousarray(a)).to(dev).requires_grad_(g)
    tq, tk, tv, twq, twk = d(xq, True), d(xk, True), d(v, True), d(wq, True), d(wk, True)
    q = A.QKPrologue.apply(tq, twq, "gemma", 1e-6, 1e4)
    k = A.QKPrologue.apply(tk, twk, "gemma", 1e-6, 1e4)
    o = A.FusedAttention.apply(q, k, tv, 0.125, True)
    o.backward(d(dO))
    qd = A.prologue_forward(d(xq), d(wq), "gemma", 1e-6, 1e4)
    kd = A.prologue_forward(d(xk), d(wk), "gemma", 1e-6, 1e4)
    o2, lse = A.attention_forward(qd, kd, d(v), 0.125, True)
    dq, dk, dv = A.attention_backward(qd, kd, d(v), o2, d(dO), lse, 0.125, True)
    gq = A.prologue_backward(d(xq), d(wq), dq, "gemma", 1e-6, 1e4)
    torch.cuda.synchronize()
    assert torch.equal(o.detach(), o2)
    assert torch.equal(tq.grad, gq[0]) and torch.equal(twq.grad, gq[1]) and torch.equal(tv.grad, dv)


def test_unaligned_rows_take_the_scalar_path(orc, dev):
    """Rows that start off the vector boundary (a view one element into a
    padded buffer) are read element by element, with the same results."""
    import torch
    from mobilefinetuner_amd import attention as A
    B, H, S, D = 1, 2, 77, 256
    x, w, dy = _inputs(orc, B, H, S, D, "bf16", 41)
    ref = orc.prologue(x, w, dy, "gemma", 1e-6, 1e4)
    buf = torch.zeros(B, H, S, D + 8, dtype=torch.bfloat16, device=dev)
    xv = buf[..., 1:D + 1]
    xv.copy_(_dev(x, "bf16", dev))
    gbuf = torch.zeros(B, H, S, D + 4, dtype=torch.float32, device=dev)
    dyv = gbuf[..., 1:D + 1]
    dyv.copy_(torch.from_numpy(dy).to(dev))
    wd = torch.from_numpy(w).to(dev)
    y = A.prologue_forward(xv, wd, "gemma", 1e-6, 1e4)
    dx, dw = A.prologue_backward(xv, wd, dyv, "gemma", 1e-6, 1e4)
    torch.cuda.synchronize()
    e = (orc.max_rel(y.float().cpu().numpy(), ref["y"]), orc.max_rel(dx.cpu().numpy(), ref["dx"]),
         orc.max_rel(dw.cpu().numpy(), ref["dw"]))
    print(f"[errs] {e}", flush=True)
    assert max(e) <= TOL["bf16"], e



BATCH_CASES = [
    # (B, S, [(H, D, dtype, layout)], norm): q and k heads of one layer
    (1, 4096, [(4, 256, "bf16", "bshd"), (1, 256, "bf16", "bshd")], "gemma"),  # Gemma-3-1B, one launch
    (2, 257, [(3, 128, "f32", "bhsd"), (1, 128, "f32", "bshd")], "affine"),     # one launch, mixed layouts
    (1, 100, [(2, 512, "bf16", "bhsd"), (2, 512, "bf16", "bhsd")], "none"),     # RoPE only
    (2, 70, [(14, 64, "f32", "bhsd"), (2, 64, "f32", "bhsd")], "gemma"),        # head dim 64: a launch each
    (1, 33, [(2, 96, "f32", "bhsd")], "gemma"),                                 # n = 1, strided lanes
]


@pytest.mark.parametrize("case", BATCH_CASES, ids=[f"b{i}" for i in range(len(BATCH_CASES))])
def test_batched_prologue_equals_separate_calls_bitwise(orc, dev, case):
    """mft_prologue_fwd_n / _bwd_n on the q and k heads give the bits of one
    mft_prologue_fwd / _bwd call per tensor (y, dx and dw)."""
    import torch
    from mobilefinetuner_amd import attention as A
    B, S, tensors, norm = case
    xs, ws, dys = [], [], []
    for i, (H, D, dtype, layout) in enumerate(tensors):
        x, w, dy = _inputs(orc, B, H, S, D, dtype, 50 + 7 * i)
        if layout == "bshd":
            xd = _dev(x.transpose(0, 2, 1, 3), dtype, dev).transpose(1, 2)
        else:
            xd = _dev(x, dtype, dev)
        xs.append(xd)
        ws.append(torch.from_numpy(w).to(dev) if norm != "none" else None)
        dys.append(torch.from_numpy(dy).to(dev))
    print(f"[case] B{B} S{S} {tensors} {norm}", flush=True)
    ys = A.prologue_forward_n(xs, ws, norm, 1e-6, 1e4)
    gs = A.prologue_backward_n(xs, ws, dys, norm, 1e-6, 1e4)
    for i in range(len(xs)):
        y1 = A.prologue_forward(xs[i], ws[i], norm, 1e-6, 1e4)
        dx1, dw1 = A.prologue_backward(xs[i], ws[i], dys[i], norm, 1e-6, 1e4)
        torch.cuda.synchronize()
        assert torch.equal(ys[i], y1), i
        assert torch.equal(gs[i][0], dx1), i
        if norm != "none":
            assert torch.equal(gs[i][1], dw1), i
        else:
            assert gs[i][1] is None and dw1 is None


def test_batched_prologue_rejects_bad_batches(dev):
    import torch
    from mobilefinetuner_amd import capi
    a = torch.zeros(1, 2, 8, 64, dtype=torch.float32, device=dev)
    b = torch.zeros(1, 2, 8, 64, dtype=torch.bfloat16, device=dev)
    d32 = capi.prologue_desc(1, 2, 8, 64, capi.MFT_F32, capi.MFT_NORM_NONE, 0.0, 1e4)
    d16 = capi.prologue_desc(1, 2, 8, 64, capi.MFT_BF16, capi.MFT_NORM_NONE, 0.0, 1e4)
    s = torch.cuda.current_stream().cuda_stream
    with pytest.raises(capi.MftError):  # one dtype per batch
        capi.prologue_fwd_n([d32, d16], [a.data_ptr(), b.data_ptr()], [0, 0], [a.data_ptr(), b.data_ptr()], s)
    with pytest.raises(capi.MftError):  # at most two tensors
        capi.prologue_fwd_n([d32] * 3, [a.data_ptr()] * 3, [0] * 3, [a.data_ptr()] * 3, s)
