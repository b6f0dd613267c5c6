"""GPU parity of the LoRA linear layer (LoRALinear over the mft_lora_* C ABI)
with the oracle restatement of ops::LoRALinear (pinned bit for bit to the
reference by test_lora_oracle.py), and the reference test's merge checks
(nn/test_lora_linear.cpp).

Bars: W fp32, every GEMM fp32: max-rel 1e-4 (y, dx, grad_A, grad_B).  W bf16:
the products with W run on the bf16 MFMA path with x (dy) rounded to bf16,
held to 2e-2 against the oracle on the same bf16 W values.  merge_to_base is
bit-exact (double rank sums, one fp32 add, bf16 rounding as the reference).
"""
import numpy as np
import pytest

from test_lora_oracle import _random_case, _z, fixture_case

pytestmark = pytest.mark.gpu

TOL = {False: 1e-4, True: 2e-2}


def _rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(1e-30, np.max(np.abs(ref))))


def _t(a, dev, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t.to(dtype) if dtype is not None else t


def _layer(dev, W, bias, slices, wb, all_grads=False):
    import torch
    from mobilefinetuner_amd.lora import LoRALinear
    layer = LoRALinear(_t(W, dev, torch.bfloat16 if wb else torch.float32),
                       None if bias is None else _t(bias, dev), grads_for_column_slices=all_grads)
    for s in slices:
        A, B = _t(s["A"], dev), _t(s["B"], dev)
        out_cols = (s["B"].shape[0] if s.get("b_transposed") else s["B"].shape[1])
        layer.attach_lora(A, B, s["scale"], s.get("col0", 0), out_cols)
    return layer


def _run(dev, x, W, bias, slices, wb, dy, all_grads=False):
    import torch
    layer = _layer(dev, W, bias, slices, wb, all_grads)
    xt = _t(x, dev).requires_grad_(True)
    y = layer.forward(xt)
    y.backward(_t(dy, dev))
    torch.cuda.synchronize()
    grads_A = [None if s.A.grad is None else s.A.grad.cpu().numpy() for s in layer.slices()]
    grads_B = [None if s.B.grad is None else s.B.grad.cpu().numpy() for s in layer.slices()]
    return dict(y=y.detach().cpu().numpy(), dx=xt.grad.cpu().numpy(), grad_A=grads_A, grad_B=grads_B)


def _check(got, ref, tol, tag):
    errs = [_rel(got["y"], ref["y"]), _rel(got["dx"], ref["dx"])]
    for g, r in zip(got["grad_A"] + got["grad_B"], ref["grad_A"] + ref["grad_B"]):
        assert (g is None) == (r is None), tag
        if r is not None:
            errs.append(_rel(g, r))
    print(f"[errs] {tag} " + " ".join(f"{e:.2e}" for e in errs), flush=True)
    assert max(errs) <= tol, (tag, errs)


@pytest.mark.parametrize("name", ["unit", "merge_bf16", "clear", "rand0", "rand1", "rand2"])
def test_reference_fixture(dev, name):
    """The reference's own outputs (tests/golden/lora.npz)."""
    print(f"[case] fixture {name}", flush=True)
    z = _z()
    x, W, bias, slices, wt, wb, dy = fixture_case(z, name)
    if wt:
        W = np.ascontiguousarray(W)
    got = _run(dev, x, W, bias, slices, wb, dy)
    ref = dict(y=z[f"{name}_y"], dx=z[f"{name}_dx"],
               grad_A=[z[f"{name}_s{j}_grad_A"] if f"{name}_s{j}_grad_A" in z else None for j in range(len(slices))],
               grad_B=[z[f"{name}_s{j}_grad_B"] if f"{name}_s{j}_grad_B" in z else None for j in range(len(slices))])
    _check(got, ref, TOL[wb], name)


CASES = [
    # N, in, out, w_transposed, w_bf16, bias, slices (rank, scale, col0, cols, a_t, b_t), all_grads
    (256, 512, 384, False, False, True, [(8, 2.0, 0, 384, False, False)], False),
    (200, 320, 192, True, False, False, [(16, 0.5, 0, 192, True, True), (4, 1.0, 64, 64, False, False)], True),
    (512, 1152, 1024, False, True, False, [(16, 2.0, 0, 1024, False, False)], False),
    (300, 256, 768, False, True, True, [(8, 2.0, 0, 256, False, False), (8, 2.0, 256, 256, True, False),
                                        (8, 2.0, 512, 256, False, True)], True),
    (64, 96, 112, True, True, True, [(4, 0.25, 0, 112, False, False)], False),
    (33, 17, 29, False, False, True, [(3, 1.0, 0, 29, True, False), (2, 3.0, 7, 9, False, True)], False),
    # bf16 W with in and out not multiples of 4 (scalar loads and bf16 stores in the staging rowdot)
    (45, 35, 50, False, True, False, [(3, 1.5, 0, 50, False, False)], False),
    # bf16 W whose only slice is a column range without gradients (dy staged by lora_round_bf16)
    (64, 128, 96, False, True, True, [(4, 1.0, 32, 32, False, False)], False),
    # bf16 W [out, in] with outputs large enough for the fused forward (GEMM, rank-r update and
    # bias in one kernel): whole tiles; partial position and output tiles with B [rank, cols]
    # and rank 16; and a plain layer (no slice) with a bias
    (1024, 64, 16384, True, True, True, [(8, 2.0, 0, 16384, True, True)], False),
    (1000, 128, 16500, True, True, False, [(16, 0.5, 0, 16500, False, False)], False),
    (1024, 64, 16384, True, True, True, [], False),
]


# A square W is always taken as [in, out], as the reference's matmul takes it
# (it transposes W only when the inner dimensions disagree, core/ops.cpp:649-654).
@pytest.mark.parametrize("case", CASES, ids=lambda c: "N{}i{}o{}-wt{:d}-bf{:d}-s{}-g{:d}".format(
    c[0], c[1], c[2], c[3], c[4], len(c[6]), c[7]))
def test_matches_oracle(orc, dev, case):
    N, I, O, wt, wb, has_bias, specs, all_grads = case
    print(f"[case] lora {case}", flush=True)
    rng = np.random.default_rng(N * 7 + I)
    x, W, slices, dy = _random_case(rng, N, I, O, wt, specs)
    if wb:
        W = orc.round_bf16(W)
    bias = rng.standard_normal(O).astype(np.float32) if has_bias else None
    ref = orc.lora(x, W, bias, slices, w_transposed=wt, dy=dy, all_grads=all_grads, w_bf16=wb)
    got = _run(dev, x, W, bias, slices, wb, dy, all_grads)
    _check(got, ref, TOL[wb], str(case))


@pytest.mark.parametrize("wb", [False, True])
def test_merge_is_bit_exact_and_unmerge_restores_bytes(orc, dev, wb):
    """nn/test_lora_linear.cpp:51-122: merging then running the plain layer
    reproduces the unmerged forward; a bf16 merge changes the stored bytes and
    unmerge_from_base restores them exactly; merge_to_base equals the
    reference's apply_lora_delta_to_base bit for bit."""
    import torch
    rng = np.random.default_rng(21 + wb)
    x, W, slices, _ = _random_case(rng, 40, 96, 160, False, [(8, 0.5, 0, 160, False, False),
                                                             (4, 2.0, 32, 64, True, True)])
    if wb:
        W = orc.round_bf16(W)
    layer = _layer(dev, W, None, slices, wb)
    xt = _t(x, dev)
    before = layer.forward(xt).detach()
    original = layer.W.detach().clone()
    layer.merge_to_base()
    assert layer.is_merged()
    torch.cuda.synchronize()
    merged = layer.W.float().cpu().numpy()
    assert np.array_equal(merged, orc.lora_merge(W, slices, w_bf16=wb))
    after = layer.forward(xt).detach()
    assert _rel(after.cpu().numpy(), before.cpu().numpy().astype(np.float64)) <= TOL[wb]
    layer.unmerge_from_base()
    assert not layer.is_merged()
    assert torch.equal(layer.W, original)


def test_merge_sign_minus_one_matches_oracle(orc, dev):
    """mft_lora_merge with sign -1 (the reference's unmerge without a backup)."""
    import torch
    from mobilefinetuner_amd import capi
    rng = np.random.default_rng(5)
    x, W, slices, _ = _random_case(rng, 8, 64, 80, False, [(6, 1.5, 8, 40, False, False)])
    W = orc.round_bf16(W)
    Wt = _t(W, dev, torch.bfloat16)
    At, Bt = _t(slices[0]["A"], dev), _t(slices[0]["B"], dev)
    d = capi.lora_desc(1, 64, 80, capi.MFT_BF16, False,
                       [dict(A=At.data_ptr(), B=Bt.data_ptr(), scale=1.5, rank=6, col0=8, cols=40)])
    capi.lora_merge(d, Wt.data_ptr(), -1.0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(Wt.float().cpu().numpy(), orc.lora_merge(W, slices, w_bf16=True, sign=-1.0))


def test_clear_lora_unmerges_first(dev):
    """nn/test_lora_linear.cpp:124-141."""
    import torch
    z = _z()
    x, W, bias, slices, wt, wb, dy = fixture_case(z, "clear")
    layer = _layer(dev, W, None, slices, True)
    original = layer.W.detach().clone()
    layer.merge_to_base()
    layer.clear_lora()
    assert not layer.is_merged() and not layer.slices()
    assert torch.equal(layer.W, original)


def test_reference_errors(dev):
    import torch
    from mobilefinetuner_amd.lora import LoRALinear
    layer = LoRALinear(torch.zeros(8, 6, device=dev))
    with pytest.raises(RuntimeError, match="left operand must be float32"):
        layer.forward(torch.zeros(2, 8, device=dev, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="must be 2D"):
        layer.attach_lora(torch.zeros(8, device=dev), torch.zeros(2, 6, device=dev), 1.0)
    with pytest.raises(RuntimeError, match="FP32"):
        layer.attach_lora(torch.zeros(8, 2, device=dev, dtype=torch.bfloat16), torch.zeros(2, 6, device=dev), 1.0)
    layer.attach_lora(torch.zeros(8, 2, device=dev), torch.zeros(2, 4, device=dev), 1.0, 4, 4)
    with pytest.raises(RuntimeError, match="exceeds base weight width"):
        layer.forward(torch.zeros(3, 8, device=dev))
