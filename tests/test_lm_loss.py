"""GPU parity of the LM cross-entropy (mft_lm_ce_* through the C ABI) with the
oracle restatement of ops::lm_cross_entropy / ops::streaming_lm_cross_entropy
(pinned bit for bit to the reference by test_lm_loss_oracle.py).

Bars: fp32 max-rel 1e-4 (loss, gradients); bf16 2e-2 against the fp32 oracle
run on the same bf16-rounded inputs.  The streaming variant is held to the
same bars, and to the dense one (the reference test's own check).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = {"f32": 1e-4, "bf16": 2e-2}


def _labels(orc, B, S, V, seed, ignore_frac=0.15):
    u = np.array([orc.uniform(seed, 7, j) for j in range(B * S)]).reshape(B, S)
    y = np.minimum((u * V).astype(np.int64), V - 1).astype(np.int32)
    y[u < ignore_frac] = -100
    return y


def _dev(x, dtype, dev):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    return t.to(torch.bfloat16) if dtype == "bf16" else t


def _rel(orc, got, ref):
    return orc.max_rel(np.asarray(got, np.float32), np.asarray(ref, np.float32))


DENSE = [
    # B, S, V, dtype, reduction
    (2, 17, 300, "f32", "mean"),
    (1, 64, 5000, "f32", "sum"),
    (2, 9, 1000, "f32", "none"),
    (1, 8, 50000, "bf16", "mean"),
    (3, 5, 777, "bf16", "none"),
]


@pytest.mark.parametrize("case", DENSE, ids=lambda c: "B{}S{}V{}-{}-{}".format(*c))
def test_dense_matches_oracle(orc, dev, case):
    import torch
    from mobilefinetuner_amd import lm_loss as L
    B, S, V, dtype, red = case
    print(f"[case] dense {case}", flush=True)
    logits = (3.0 * orc.normal(B * S * V, 6000 + V, 0)).reshape(B, S, V)
    if dtype == "bf16":
        logits = orc.round_bf16(logits)
    y = _labels(orc, B, S, V, 6000 + V)
    g = (orc.normal(B * S, 6100, 0).reshape(B, S) + 1.0) if red == "none" else 0.75
    ref = orc.lm_ce(logits, y, -100, red, g)
    lt, yt = _dev(logits, dtype, dev), torch.from_numpy(y).to(dev)
    loss, lse = L.lm_cross_entropy(lt, yt, -100, red)
    gl = torch.from_numpy(np.asarray(g, np.float32).reshape(-1) if red == "none" else np.array([g], np.float32))
    grad = L.lm_cross_entropy_backward(lt, yt, lse, gl.to(dev).reshape(loss.shape), -100, red)
    torch.cuda.synchronize()
    e = (_rel(orc, loss.cpu().numpy(), ref["loss"]), _rel(orc, grad.cpu().numpy(), ref["grad"]))
    print(f"[errs] loss {e[0]:.2e} grad {e[1]:.2e}", flush=True)
    assert max(e) <= TOL[dtype], e


STREAM = [
    # B, S, H, V, dtype, reduction, chunk
    (2, 17, 24, 300, "f32", "mean", 0),
    (1, 33, 64, 1000, "f32", "sum", 128),     # chunks that split V unevenly
    (2, 40, 128, 5000, "bf16", "mean", 1024),
    (1, 64, 1152, 4096, "bf16", "mean", 0),   # Gemma-3-1B hidden size
    (1, 20, 40, 999, "f32", "mean", 250),     # rows off the 16-byte grid: element-wise passes
]


@pytest.mark.parametrize("case", STREAM, ids=lambda c: "B{}S{}H{}V{}-{}-{}-c{}".format(*c))
def test_streaming_matches_oracle(orc, dev, case):
    import torch
    from mobilefinetuner_amd import lm_loss as L
    B, S, H, V, dtype, red, chunk = case
    print(f"[case] streaming {case}", flush=True)
    h = (0.5 * orc.normal(B * S * H, 6200 + V, 0)).reshape(B, S, H)
    w = (0.5 * orc.normal(V * H, 6200 + V, 1)).reshape(V, H)
    if dtype == "bf16":
        h, w = orc.round_bf16(h), orc.round_bf16(w)
    y = _labels(orc, B, S, V, 6200 + V)
    ref = orc.selected_ce(h, w, y, -100, red, 0.75)
    ht, wt, yt = _dev(h, dtype, dev), _dev(w, dtype, dev), torch.from_numpy(y).to(dev)
    loss, lse = L.streaming_lm_cross_entropy(ht, wt, yt, -100, red, chunk)
    gh, gw = L.streaming_lm_cross_entropy_backward(ht, wt, yt, lse, torch.full((1,), 0.75, device=dev), -100, red,
                                                   chunk)
    torch.cuda.synchronize()
    e = (_rel(orc, loss.cpu().numpy(), ref["loss"]), _rel(orc, gh.cpu().numpy(), ref["grad_hidden"]),
         _rel(orc, gw.cpu().numpy(), ref["grad_weight"]))
    print(f"[errs] loss {e[0]:.2e} gh {e[1]:.2e} gw {e[2]:.2e}", flush=True)
    assert max(e) <= TOL[dtype], e


@pytest.mark.parametrize("shape", [(1, 2048, 256, 32768), (3, 500, 128, 20000), (2, 300, 64, 2999)],
                         ids=lambda c: "B{}S{}H{}V{}".format(*c))
def test_fused_forward_placements(orc, dev, shape):
    """The fused bf16 forward at shapes whose workgroups are placed as XCD
    rectangles of vocabulary ranges x position blocks (4 x 8 and 5 x 6 here,
    the second and third with partial position and vocabulary tiles; the third
    is range-major), against a torch fp32 reference on the same bf16 inputs:
    LSE of every position and the mean NLL to 1e-5 relative."""
    import torch
    from mobilefinetuner_amd import lm_loss as L
    B, S, H, V = shape
    print(f"[case] fused forward {shape}", flush=True)
    g = torch.Generator(device=dev)
    g.manual_seed(B * S + V)
    h = (0.5 * torch.randn(B, S, H, device=dev, generator=g)).to(torch.bfloat16)
    w = (0.2 * torch.randn(V, H, device=dev, generator=g)).to(torch.bfloat16)
    y = torch.randint(0, V, (B, S), device=dev, generator=g, dtype=torch.int32)
    y[:, ::7] = -100
    loss, lse = L.streaming_lm_cross_entropy(h, w, y)
    z = h.float().reshape(B * S, H) @ w.float().t()
    ref_lse = torch.logsumexp(z.double(), dim=1).reshape(B, S)
    nxt = y[:, 1:].reshape(-1).long()
    keep = nxt != -100
    zz = z.reshape(B, S, V)[:, :-1].reshape(-1, V)[keep]
    got = lse[:, :-1].reshape(-1)
    ref = ref_lse[:, :-1].reshape(-1)
    nll = ref[keep] - zz.double().gather(1, nxt[keep].unsqueeze(1)).squeeze(1)
    torch.cuda.synchronize()
    # the LSE is kept for scored positions; the others hold 0 (as the reference's)
    e_lse = float(((got[keep].double() - ref[keep]).abs() / ref[keep].abs().clamp_min(1.0)).max())
    e_loss = abs(float(loss) - float(nll.mean())) / abs(float(nll.mean()))
    print(f"[errs] lse {e_lse:.2e} loss {e_loss:.2e}", flush=True)
    assert e_lse <= 1e-5 and e_loss <= 1e-5, (e_lse, e_loss)
    assert float(got[~keep].abs().max()) == 0.0 and float(lse[:, -1].abs().max()) == 0.0


@pytest.mark.parametrize("shape", [(1, 2048, 256, 32768, 0), (3, 500, 128, 20000, 4999), (2, 300, 64, 2999, 1000)],
                         ids=lambda c: "B{}S{}H{}V{}-c{}".format(*c))
def test_fused_backward_placements(orc, dev, shape):
    """The fused bf16 backward (G from the recomputed logits, then the two
    GEMMs) at the placement shapes above, with chunks that split V unevenly
    and rows of G off the 8-element grid, against torch fp32 on the same bf16
    inputs: max |error| over max |value| of grad_hidden and grad_weight within
    the bf16 bar (G is rounded to bf16 before the GEMMs, as the reference's
    bf16 path rounds it)."""
    import torch
    from mobilefinetuner_amd import lm_loss as L
    B, S, H, V, chunk = shape
    print(f"[case] fused backward {shape}", flush=True)
    g = torch.Generator(device=dev)
    g.manual_seed(B * S + V + 1)
    h = (0.5 * torch.randn(B, S, H, device=dev, generator=g)).to(torch.bfloat16)
    w = (0.2 * torch.randn(V, H, device=dev, generator=g)).to(torch.bfloat16)
    y = torch.randint(0, V, (B, S), device=dev, generator=g, dtype=torch.int32)
    y[:, ::5] = -100
    loss, lse = L.streaming_lm_cross_entropy(h, w, y, chunk=chunk)
    gl = torch.full((1,), 0.75, device=dev)
    gh, gw = L.streaming_lm_cross_entropy_backward(h, w, y, lse, gl, chunk=chunk)
    hf, wf = h.float().reshape(B * S, H), w.float()
    z = hf @ wf.t()
    nxt = torch.full((B, S), -100, dtype=torch.long, device=dev)
    nxt[:, :-1] = y[:, 1:].long()
    nxt = nxt.reshape(-1)
    keep = nxt != -100
    G = torch.softmax(z, dim=1)
    G[torch.arange(B * S, device=dev)[keep], nxt[keep]] -= 1.0
    G = G * keep.unsqueeze(1).float() * (0.75 / float(keep.sum()))
    ref_h = (G @ wf).reshape(B, S, H)
    ref_w = G.t().contiguous() @ hf
    torch.cuda.synchronize()
    e_h = float((gh - ref_h).abs().max() / ref_h.abs().max())
    e_w = float((gw - ref_w).abs().max() / ref_w.abs().max())
    print(f"[errs] gh {e_h:.2e} gw {e_w:.2e}", flush=True)
    assert e_h <= TOL["bf16"] and e_w <= TOL["bf16"], (e_h, e_w)


def test_streaming_equals_dense_on_the_gpu(orc, dev):
    """The reference test's check (core/test_selected_token_lm_loss.cpp:98-115):
    streaming loss and gradients equal the dense ones chained through
    logits = hidden . W^T."""
    import torch
    from mobilefinetuner_amd import lm_loss as L
    B, S, H, V = 2, 30, 48, 2000
    h = torch.from_numpy((0.5 * orc.normal(B * S * H, 6300, 0)).reshape(B, S, H)).to(dev)
    w = torch.from_numpy((0.5 * orc.normal(V * H, 6300, 1)).reshape(V, H)).to(dev)
    y = torch.from_numpy(_labels(orc, B, S, V, 6300)).to(dev)
    logits = (h @ w.t()).contiguous()
    dl, dlse = L.lm_cross_entropy(logits, y)
    dg = L.lm_cross_entropy_backward(logits, y, dlse, torch.ones(1, device=dev))
    sl, slse = L.streaming_lm_cross_entropy(h, w, y, chunk=300)
    gh, gw = L.streaming_lm_cross_entropy_backward(h, w, y, slse, torch.ones(1, device=dev), chunk=300)
    torch.cuda.synchronize()
    assert abs(float(dl) - float(sl)) <= 1e-5 * abs(float(dl))
    assert torch.allclose(gh, torch.einsum("bsv,vh->bsh", dg, w), atol=1e-5, rtol=1e-4)
    assert torch.allclose(gw, torch.einsum("bsv,bsh->vh", dg, h), atol=1e-5, rtol=1e-4)


def test_all_ignored_and_out_of_range_labels(orc, dev):
    import torch
    from mobilefinetuner_amd import lm_loss as L
    B, S, H, V = 2, 4, 3, 5
    h = torch.randn(B, S, H, device=dev)
    w = torch.randn(V, H, device=dev)
    y = torch.full((B, S), -100, dtype=torch.int32, device=dev)
    loss, lse = L.streaming_lm_cross_entropy(h, w, y)
    gh, gw = L.streaming_lm_cross_entropy_backward(h, w, y, lse, torch.ones(1, device=dev))
    dl, _ = L.lm_cross_entropy(torch.randn(B, S, V, device=dev), y)
    torch.cuda.synchronize()
    assert torch.isnan(loss).all() and torch.isnan(dl).all()
    assert torch.count_nonzero(gh) == 0 and torch.count_nonzero(gw) == 0
    y[0, 2] = V  # out of range: the reference throws
    with pytest.raises(ValueError, match="out of range"):
        L.lm_cross_entropy(torch.randn(B, S, V, device=dev), y)
    with pytest.raises(ValueError, match="out of range"):
        L.streaming_lm_cross_entropy(h, w, y)


def test_fused_all_ignored_and_out_of_range_labels(dev):
    """The same edge cases on the fused bf16 kernels (H a multiple of 64):
    all labels ignored gives a NaN mean with zero gradients; an out-of-range
    label raises from the forward, and the backward (which the reference never
    reaches) leaves that position's gradient row zero and the rest equal to a
    run where the label is ignored."""
    import torch
    from mobilefinetuner_amd import lm_loss as L
    B, S, H, V = 2, 300, 64, 700
    g = torch.Generator(device=dev)
    g.manual_seed(77)
    h = (0.5 * torch.randn(B, S, H, device=dev, generator=g)).to(torch.bfloat16)
    w = (0.3 * torch.randn(V, H, device=dev, generator=g)).to(torch.bfloat16)
    y = torch.full((B, S), -100, dtype=torch.int32, device=dev)
    loss, lse = L.streaming_lm_cross_entropy(h, w, y)
    gh, gw = L.streaming_lm_cross_entropy_backward(h, w, y, lse, torch.ones(1, device=dev))
    torch.cuda.synchronize()
    assert torch.isnan(loss).all() and torch.count_nonzero(lse) == 0
    assert torch.count_nonzero(gh) == 0 and torch.count_nonzero(gw) == 0
    y = torch.randint(0, V, (B, S), device=dev, generator=g, dtype=torch.int32)
    y_ign = y.clone()
    y[1, 7] = V + 3
    y_ign[1, 7] = -100
    with pytest.raises(ValueError, match="out of range"):
        L.streaming_lm_cross_entropy(h, w, y)
    loss_i, lse_i = L.streaming_lm_cross_entropy(h, w, y_ign)
    one = torch.ones(1, device=dev)
    # the count of scored positions differs (the out-of-range one is counted
    # as scored, as the reference's forward would before throwing), so
    # compare with reduction "sum", where the coefficient is the same
    gh, gw = L.streaming_lm_cross_entropy_backward(h, w, y, lse_i, one, reduction="sum")
    gh_i, gw_i = L.streaming_lm_cross_entropy_backward(h, w, y_ign, lse_i, one, reduction="sum")
    torch.cuda.synchronize()
    assert torch.count_nonzero(gh[1, 6]) == 0  # position 6 scores label [1, 7]
    assert torch.equal(gh, gh_i) and torch.equal(gw, gw_i)


def test_autograd_node(orc, dev):
    import torch
    from mobilefinetuner_amd import lm_loss as L
    B, S, H, V = 1, 20, 32, 700
    h = torch.from_numpy((0.5 * orc.normal(B * S * H, 6400, 0)).reshape(B, S, H)).to(dev).requires_grad_(True)
    w = torch.from_numpy((0.5 * orc.normal(V * H, 6400, 1)).reshape(V, H)).to(dev).requires_grad_(True)
    y = torch.from_numpy(_labels(orc, B, S, V, 6400)).to(dev)
    loss = L.StreamingLMCrossEntropy.apply(h, w, y)
    (2.0 * loss).sum().backward()
    ref = orc.selected_ce(h.detach().cpu().numpy(), w.detach().cpu().numpy(), y.cpu().numpy(), -100, "mean", 2.0)
    assert _rel(orc, h.grad.cpu().numpy(), ref["grad_hidden"]) <= 1e-4
    assert _rel(orc, w.grad.cpu().numpy(), ref["grad_weight"]) <= 1e-4
