"""torch-tensor plumbing over the C ABI (device memory and streams only).

The arithmetic is entirely in libmft_attn.so.  These helpers allocate the
outputs and the workspace as torch tensors on the current device and enqueue
the C-ABI calls on torch's current stream, so tests and the benchmark can drive
the kernels without writing HIP host code.  There is no fallback: a missing
library or a non-GPU tensor raises.
"""
from __future__ import annotations

import torch

from . import capi

_DT = {torch.float32: capi.MFT_F32, torch.bfloat16: capi.MFT_BF16}


def _check(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (the fused attention has no CPU path)")
    if t.dim() != 4:
        raise ValueError(f"{name} must be 4D [B,H,S,D]")
    if t.stride(3) != 1:
        raise ValueError(f"{name} must have a contiguous head dim (any [B,H,S] strides, e.g. a [B,S,H,D] view)")


def _strides(**ops):
    """Element strides (b, h, s) of each non-contiguous operand for the
    descriptor (contiguous operands take the descriptor's default)."""
    return {n: (t.stride(0), t.stride(1), t.stride(2)) for n, t in ops.items()
            if t is not None and not t.is_contiguous()}


def _mask_spec(m, B, Hq, S):
    """(device address, (sb, sh, si, sj)) of an additive fp32 mask: [S, S] or
    4-D [1|B, 1|Hq, 1|S, S] (size-1 dims broadcast)."""
    if not isinstance(m, torch.Tensor) or not m.is_cuda or m.dtype != torch.float32:
        raise ValueError("masks must be float32 GPU tensors")
    if m.dim() == 2:
        m = m.view(1, 1, *m.shape)
    if m.dim() != 4 or m.shape[3] != S or any(m.shape[i] not in (1, n) for i, n in enumerate((B, Hq, S))):
        raise ValueError(f"a mask must be [S,S] or [1|B, 1|Hq, 1|S, S] (S={S}), got {tuple(m.shape)}")
    st = tuple(0 if m.shape[i] == 1 else m.stride(i) for i in range(4))
    return m.data_ptr(), st


def _desc(q, k, scale, causal, window=0, kv_len=None, layouts=None, masks=()):
    """kv_len: None or an int32 [B] GPU tensor of valid keys per batch (key padding).
    layouts: {name: tensor} of operands (q, k, v, o, dO, dq, dk, dv) whose strides
    go into the descriptor (the others are contiguous).  masks: up to two
    additive fp32 masks (mask mode; see attention_forward)."""
    if q.dtype not in _DT:
        raise ValueError(f"unsupported dtype {q.dtype}")
    B, Hq, S, D = q.shape
    lp = None
    if kv_len is not None:
        if not kv_len.is_cuda or kv_len.dtype != torch.int32 or kv_len.shape != (B,) or not kv_len.is_contiguous():
            raise ValueError("kv_len must be a contiguous int32 GPU tensor of shape [B]")
        lp = kv_len.data_ptr()
    return capi.desc(B, Hq, k.shape[1], S, D, scale, causal, _DT[q.dtype], window, lp,
                     _strides(**(layouts or {})), [_mask_spec(m, B, Hq, S) for m in masks])


def _stream():
    return torch.cuda.current_stream().cuda_stream


def workspace_bytes(q, k, scale=-1.0, causal=True, window=0, kv_len=None):
    """Backward workspace bytes."""
    return capi.workspace_size(_desc(q, k, scale, causal, window, kv_len))[1]


def fwd_workspace_bytes(q, k, scale=-1.0, causal=True, window=0, kv_len=None):
    """Forward workspace bytes (0 when the forward needs none)."""
    return capi.workspace_size(_desc(q, k, scale, causal, window, kv_len))[0]


def attention_forward(q, k, v, scale: float = -1.0, causal: bool = True, want_lse: bool = True,
                      workspace=None, balanced: bool = True, window: int = 0, kv_len=None, out=None,
                      masks=()):
    """o, lse = fused attention forward (lse None when want_lse is False).

    balanced=True passes the forward workspace (allocated here unless given),
    which selects the launch that splits long query tiles across work units;
    balanced=False passes none (one workgroup per query tile).  window > 0:
    causal sliding window of that many keys; kv_len: int32 [B] GPU tensor of
    valid (unpadded) keys per batch.  q, k, v (and out, the output buffer)
    may be any [B,H,S,D] views with a contiguous head dim, e.g. transposed
    [B,S,H,D] projections; by default o takes q's layout.

    masks: up to two additive fp32 masks ([S,S] or [1|B, 1|Hq, 1|S, S]), added
    to the scaled scores in order (mask mode, mft_mask: every key is visited;
    causal=True replaces the scores above the diagonal by -1e10 first, the
    reference's no-grad rule).  lse is then [B, Hq, S, 2]: (row max, ln sum)."""
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _check(t, n)
    if k.dtype != q.dtype or v.dtype != q.dtype or k.shape != v.shape:
        raise ValueError("q, k, v must share dtype and k, v must have equal shapes")
    if k.shape[0] != q.shape[0] or k.shape[2:] != q.shape[2:]:
        raise ValueError("k/v must be [B, Hkv, S, D] with q's B, S, D")
    o = torch.empty_like(q) if out is None else out
    if o.shape != q.shape or o.dtype != q.dtype:
        raise ValueError("out must have q's shape and dtype")
    _check(o, "out")
    d = _desc(q, k, scale, causal, window, kv_len, dict(q=q, k=k, v=v, o=o), masks)
    lse_shape = tuple(q.shape[:3]) + ((2,) if masks else ())
    lse = torch.empty(lse_shape, dtype=torch.float32, device=q.device) if want_lse else None
    ws_ptr = None
    if balanced:
        nbytes = capi.workspace_size(d)[0]
        if nbytes:
            if workspace is None or workspace.numel() < nbytes:
                workspace = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
            ws_ptr = workspace.data_ptr()
    capi.attn_fwd(d, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                  lse.data_ptr() if lse is not None else None, ws_ptr, _stream())
    return o, lse


def attention_backward(q, k, v, o, dO, lse, scale: float = -1.0, causal: bool = True, workspace=None,
                       window: int = 0, kv_len=None, masks=()):
    """dq, dk, dv (fp32; dk, dv already summed over the GQA group), each in the
    layout of q, k, v respectively (operands may be views as in attention_forward)."""
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (o, "o"), (dO, "dO")):
        _check(t, n)
    if not lse.is_cuda or not lse.is_contiguous():
        raise ValueError("lse must be a contiguous GPU tensor")
    if dO.dtype != q.dtype or o.dtype != q.dtype or lse.dtype != torch.float32:
        raise ValueError("o and dO must have q's dtype; lse must be float32")
    dq = torch.empty_like(q, dtype=torch.float32)
    dk = torch.empty_like(k, dtype=torch.float32)
    dv = torch.empty_like(v, dtype=torch.float32)
    d = _desc(q, k, scale, causal, window, kv_len, dict(q=q, k=k, v=v, o=o, dO=dO, dq=dq, dk=dk, dv=dv), masks)
    nbytes = capi.workspace_size(d)[1]
    if workspace is None or workspace.numel() < nbytes:
        workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    capi.attn_bwd(d, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), dO.data_ptr(),
                  lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                  workspace.data_ptr(), _stream())
    return dq, dk, dv


def repeat_kv(kv: torch.Tensor, r: int) -> torch.Tensor:
    _check(kv, "kv")
    B, H, S, D = kv.shape
    out = torch.empty((B, H * r, S, D), dtype=kv.dtype, device=kv.device)
    capi.repeat_kv_fwd(kv.data_ptr(), out.data_ptr(), B, H, S, D, r, _DT[kv.dtype], _stream())
    return out


def repeat_kv_backward(g: torch.Tensor, r: int) -> torch.Tensor:
    _check(g, "g")
    if g.dtype != torch.float32:
        raise ValueError("repeat_kv backward takes fp32 gradients")
    B, Hr, S, D = g.shape
    if Hr % r:
        raise ValueError("repeat_factor does not divide head dimension")
    out = torch.empty((B, Hr // r, S, D), dtype=torch.float32, device=g.device)
    capi.repeat_kv_bwd(g.data_ptr(), out.data_ptr(), B, Hr // r, S, D, r, _stream())
    return out


class FusedAttention(torch.autograd.Function):
    """Autograd node that saves only q, k, v, o and the row log-sum-exp."""

    @staticmethod
    def forward(ctx, q, k, v, scale=-1.0, causal=True, window=0, kv_len=None):
        o, lse = attention_forward(q, k, v, scale, causal, window=window, kv_len=kv_len)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.scale, ctx.causal, ctx.window, ctx.kv_len = scale, causal, window, kv_len
        return o

    @staticmethod
    def backward(ctx, dO):
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = attention_backward(q, k, v, o, dO.contiguous().to(q.dtype), lse, ctx.scale, ctx.causal,
                                        window=ctx.window, kv_len=ctx.kv_len)
        return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), None, None, None, None


# ------------------------------------------------------------ q/k prologue
_NORMS = {"none": capi.MFT_NORM_NONE, "gemma": capi.MFT_NORM_GEMMA, "affine": capi.MFT_NORM_AFFINE}


def _prologue_desc(x, norm, eps, theta, layouts):
    if x.dtype not in _DT:
        raise ValueError(f"unsupported dtype {x.dtype}")
    if norm not in _NORMS:
        raise ValueError(f"norm must be one of {sorted(_NORMS)}")
    B, H, S, D = x.shape
    return capi.prologue_desc(B, H, S, D, _DT[x.dtype], _NORMS[norm], eps, theta, _strides(**layouts))


def prologue_forward(x, w=None, norm="gemma", eps=1e-6, theta=10000.0, out=None):
    """y = rope(norm(x)) for x [B, H, S, D] (any [B, H, S] strides with a
    contiguous head dim, e.g. the [B, S, H, D] projection output viewed as
    [B, H, S, D]).  y is a new contiguous [B, H, S, D] tensor of x's dtype
    unless `out` is given.  norm: "gemma" (ops::rms_norm, x / rms * (1 + w)),
    "affine" (ops::rms_norm_affine) or "none"; theta 0 = no RoPE."""
    _check(x, "x")
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device) if out is None else out
    _check(y, "y")
    if w is not None and (not w.is_cuda or w.dtype != torch.float32 or not w.is_contiguous()):
        raise ValueError("w must be a contiguous fp32 GPU tensor [D]")
    d = _prologue_desc(x, norm, eps, theta, dict(x=x, y=y))
    capi.prologue_fwd(d, x.data_ptr(), None if w is None else w.data_ptr(), y.data_ptr(), _stream())
    return y


def prologue_backward(x, w, dy, norm="gemma", eps=1e-6, theta=10000.0, want_dw=True):
    """(dx, dw) for y = rope(norm(x)): dx fp32 contiguous [B, H, S, D], dw fp32
    [D] (None without a norm or when want_dw is False)."""
    _check(x, "x")
    _check(dy, "dy")
    if dy.dtype != torch.float32:
        raise ValueError("dy must be fp32")
    dx = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    d = _prologue_desc(x, norm, eps, theta, dict(x=x, dy=dy))
    dw = ws = None
    if norm != "none" and want_dw:
        dw = torch.empty(x.shape[3], dtype=torch.float32, device=x.device)
        ws = torch.empty(max(capi.prologue_workspace_size(d), 1), dtype=torch.uint8, device=x.device)
    capi.prologue_bwd(d, x.data_ptr(), None if w is None else w.data_ptr(), dy.data_ptr(), dx.data_ptr(),
                      None if dw is None else dw.data_ptr(), None if ws is None else ws.data_ptr(), _stream())
    return dx, dw


def prologue_forward_n(xs, ws, norm="gemma", eps=1e-6, theta=10000.0):
    """prologue_forward of up to two tensors (a layer's q and k heads) in one
    launch (mft_prologue_fwd_n): xs, ws lists; returns the list of y."""
    ys, ds = [], []
    for x, w in zip(xs, ws):
        _check(x, "x")
        if w is not None and (not w.is_cuda or w.dtype != torch.float32 or not w.is_contiguous()):
            raise ValueError("w must be a contiguous fp32 GPU tensor [D]")
        y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        ys.append(y)
        ds.append(_prologue_desc(x, norm, eps, theta, dict(x=x, y=y)))
    capi.prologue_fwd_n(ds, [x.data_ptr() for x in xs], [0 if w is None else w.data_ptr() for w in ws],
                        [y.data_ptr() for y in ys], _stream())
    return ys


def prologue_backward_n(xs, ws, dys, norm="gemma", eps=1e-6, theta=10000.0, want_dw=True):
    """prologue_backward of up to two tensors in one launch per kernel
    (mft_prologue_bwd_n): returns the list of (dx, dw)."""
    ds, dxs, dws = [], [], []
    for x, dy in zip(xs, dys):
        _check(x, "x")
        _check(dy, "dy")
        if dy.dtype != torch.float32:
            raise ValueError("dy must be fp32")
        dxs.append(torch.empty(x.shape, dtype=torch.float32, device=x.device))
        dws.append(torch.empty(x.shape[3], dtype=torch.float32, device=x.device)
                   if norm != "none" and want_dw else None)
        ds.append(_prologue_desc(x, norm, eps, theta, dict(x=x, dy=dy)))
    ws_bytes = capi.prologue_workspace_size_n(ds)
    wsp = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=xs[0].device)
    capi.prologue_bwd_n(ds, [x.data_ptr() for x in xs], [0 if w is None else w.data_ptr() for w in ws],
                        [dy.data_ptr() for dy in dys], [dx.data_ptr() for dx in dxs],
                        [0 if dw is None else dw.data_ptr() for dw in dws], wsp.data_ptr() if ws_bytes else None,
                        _stream())
    return list(zip(dxs, dws))


class QKPrologue(torch.autograd.Function):
    """Autograd node of y = rope(norm(x)); saves x and w only (the row norms
    are recomputed in the backward, as the reference's RMSNormBackward does)."""

    @staticmethod
    def forward(ctx, x, w=None, norm="gemma", eps=1e-6, theta=10000.0):
        y = prologue_forward(x, w, norm, eps, theta)
        ctx.save_for_backward(x, w)
        ctx.cfg = (norm, eps, theta)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        norm, eps, theta = ctx.cfg
        dx, dw = prologue_backward(x, w, dy.float(), norm, eps, theta,
                                   want_dw=w is not None and ctx.needs_input_grad[1])
        return dx.to(x.dtype), dw, None, None, None
