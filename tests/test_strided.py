"""Strided operands: the models' [B, S, H, D] projection layout
(graph/gemma_model.cpp:403-409, 506-508; graph/qwen_model.cpp:290-299 permute
it to [B, H, S, D] with a copy) passed as [B, H, S, D] views, for inputs, O
and the gradients.  The kernels do the same arithmetic whatever the layout, so
every output must equal the contiguous run's bit for bit; the contiguous run
itself is held to the oracle by test_attn_parity.py / test_attn_masks.py."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CASES = [
    # B, Hq, Hkv, S, D, dtype, causal, window, lengths
    (2, 4, 1, 300, 256, "bf16", True, 0, None),      # fast path, split tiles
    (1, 8, 2, 520, 128, "bf16", True, 64, None),     # window geometry
    (2, 4, 2, 200, 64, "bf16", True, 0, [200, 77]),  # padding
    (1, 4, 4, 130, 96, "f32", True, 0, None),        # fp32 fast path, partial tiles
    (1, 4, 1, 256, 256, "f32", True, 0, None),       # fp32 fast path, whole tiles (direct-load offsets)
    (2, 2, 2, 100, 20, "f32", True, 0, [100, 37]),   # general fp32 path (D <= 32), padding
    (2, 2, 1, 96, 40, "bf16", False, 0, [96, 0]),    # general bf16 path, rows with no key
]


def _bshd(x, dev, dtype):
    """[B,H,S,D] array -> a [B,H,S,D] view of [B,S,H,D] device storage."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x.transpose(0, 2, 1, 3))).to(dev)
    t = t.to(torch.bfloat16) if dtype == "bf16" else t
    return t.transpose(1, 2)


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}H{}KV{}S{}D{}-{}-{}-W{}-L{}".format(*c[:8], c[8]))
def test_bshd_views_match_contiguous_bitwise(orc, dev, case):
    import torch
    from gpu_util import to_dev
    from mobilefinetuner_amd import attention as A
    B, Hq, Hkv, S, D, dtype, causal, window, lengths = case
    print(f"[case] {case}", flush=True)
    q, k, v, dO = orc.make_inputs(B, Hq, Hkv, S, D, 900 + S, dtype, do_sigma=0.5)
    kv_len = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=dev)
    kw = dict(window=window, kv_len=kv_len)
    scale = 1.0 / np.sqrt(D)

    cq, ck, cv, cg = (to_dev(x, dtype, dev) for x in (q, k, v, dO))
    o1, l1 = A.attention_forward(cq, ck, cv, scale, causal, **kw)
    g1 = A.attention_backward(cq, ck, cv, o1, cg, l1, scale, causal, **kw)

    sq, sk, sv, sg = (_bshd(x, dev, dtype) for x in (q, k, v, dO))
    assert not sq.is_contiguous() and sq.stride(3) == 1
    o2, l2 = A.attention_forward(sq, sk, sv, scale, causal, **kw)
    assert o2.stride() == sq.stride()  # O written in q's [B,S,H,D] layout
    g2 = A.attention_backward(sq, sk, sv, o2, sg, l2, scale, causal, **kw)
    assert g2[0].stride() == sq.stride() and g2[1].stride() == sk.stride()
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    for a, b, n in zip(g1, g2, ("dq", "dk", "dv")):
        assert torch.equal(a, b), n


def test_fused_qkv_slices(orc, dev):
    """q, k, v as slices of one fused [B, S, Hq + 2*Hkv, D] projection (no copy)."""
    import torch
    from gpu_util import to_dev
    from mobilefinetuner_amd import attention as A
    B, Hq, Hkv, S, D = 2, 4, 1, 257, 128
    q, k, v, dO = orc.make_inputs(B, Hq, Hkv, S, D, 5, "bf16", do_sigma=0.5)
    qkv = torch.cat([to_dev(x, "bf16", dev).transpose(1, 2) for x in (q, k, v)], dim=2).contiguous()
    fq, fk, fv = qkv[:, :, :Hq].transpose(1, 2), qkv[:, :, Hq:Hq + Hkv].transpose(1, 2), qkv[:, :, Hq + Hkv:].transpose(1, 2)
    cq, ck, cv, cg = (to_dev(x, "bf16", dev) for x in (q, k, v, dO))
    o1, l1 = A.attention_forward(cq, ck, cv, 0.1, True)
    o2, l2 = A.attention_forward(fq, fk, fv, 0.1, True)
    g1 = A.attention_backward(cq, ck, cv, o1, cg, l1, 0.1, True)
    g2 = A.attention_backward(fq, fk, fv, o2.contiguous(), cg, l2, 0.1, True)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2.contiguous()) and torch.equal(l1, l2)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b.contiguous())


@pytest.mark.parametrize("which", ["k", "v"])
def test_kv_with_different_sequence_strides(orc, dev, which):
    """k and v with different sequence strides (one a [B,S,Hkv,D] view, the
    other contiguous): the bf16 backward then runs the general kernels (the
    fast ones take one K/V sequence stride); held to the fp32 reference."""
    import torch
    from gpu_util import TOL, to_dev
    from mobilefinetuner_amd import attention as A
    B, Hq, Hkv, S, D = 2, 4, 2, 260, 128
    print(f"[case] strided {which} only", flush=True)
    q, k, v, dO = orc.make_inputs(B, Hq, Hkv, S, D, 77, "bf16", do_sigma=0.5)
    scale = 1.0 / np.sqrt(D)
    ref = orc.composite(q, k, v, dO, scale=scale, causal=True, want_lse=True)
    cq, ck, cv, cg = (to_dev(x, "bf16", dev) for x in (q, k, v, dO))
    if which == "k":
        ck = _bshd(k, dev, "bf16")
    else:
        cv = _bshd(v, dev, "bf16")
    assert ck.stride(2) != cv.stride(2)
    o, lse = A.attention_forward(cq, ck, cv, scale, True)
    dq, dk, dv = A.attention_backward(cq, ck, cv, o, cg, lse, scale, True)
    torch.cuda.synchronize()
    got = dict(o=o.float(), dq=dq, dk=dk, dv=dv)
    for n in ("o", "dq", "dk", "dv"):
        e = orc.max_rel(got[n].contiguous().cpu().numpy(), ref[n])
        print(f"[errs] {n} {e:.2e}", flush=True)
        assert e <= TOL["bf16"], (n, e)
