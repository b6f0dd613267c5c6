"""torch-tensor plumbing over the LM cross-entropy C ABI (include/mft/lm_loss.h).

The arithmetic is in libmft_attn.so (HIP kernels, rocBLAS for the streaming
variant's chunk GEMMs).  These helpers allocate outputs and workspace as torch
tensors on the current device and enqueue on torch's current stream; there is
no CPU path.  Semantics are ops::lm_cross_entropy /
ops::streaming_lm_cross_entropy (core/lm_loss.h): labels[b, s + 1] scores
position s, ignore_index is skipped, "mean" divides by the scored count.
"""
from __future__ import annotations

import torch

from . import capi

_DT = {torch.float32: capi.MFT_F32, torch.bfloat16: capi.MFT_BF16}
_RED = {"mean": capi.MFT_REDUCE_MEAN, "sum": capi.MFT_REDUCE_SUM, "none": capi.MFT_REDUCE_NONE}


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _check(t, name, dims):
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (the LM loss has no CPU path)")
    if t.dim() != dims or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous {dims}-D tensor")


def _labels(labels, B, S):
    _check(labels, "labels", 2)
    if labels.dtype != torch.int32 or tuple(labels.shape) != (B, S):
        raise ValueError("labels must be int32 [B, S]")


def _workspace(d, dev):
    f, b = capi.lm_ce_workspace_size(d)
    return torch.empty(max(f, b, 1), dtype=torch.uint8, device=dev)


def _raise_on_status(status):
    if int(status.item()) != 0:
        raise ValueError("lm_cross_entropy: label out of range")


def lm_cross_entropy(logits, labels, ignore_index=-100, reduction="mean", check_labels=True):
    """(loss, lse) for logits [B, S, V] (fp32 or bf16).  loss is [1] or [B, S]
    ("none"); lse [B, S] is kept for the backward.  check_labels synchronises
    and raises on a label outside [0, V), as the reference does."""
    _check(logits, "logits", 3)
    B, S, V = logits.shape
    _labels(labels, B, S)
    d = capi.lm_loss_desc(B, S, V, 0, _DT[logits.dtype], ignore_index, _RED[reduction])
    ws = _workspace(d, logits.device)
    loss = torch.empty((B, S) if reduction == "none" else (1,), dtype=torch.float32, device=logits.device)
    lse = torch.empty(B, S, dtype=torch.float32, device=logits.device)
    status = torch.zeros(1, dtype=torch.int32, device=logits.device)
    capi.lm_ce_fwd(d, logits.data_ptr(), labels.data_ptr(), loss.data_ptr(), lse.data_ptr(), status.data_ptr(),
                   ws.data_ptr(), _stream())
    if check_labels:
        _raise_on_status(status)
    return loss, lse


def lm_cross_entropy_backward(logits, labels, lse, grad_loss, ignore_index=-100, reduction="mean"):
    """grad_logits [B, S, V] fp32 for grad_loss ([1] or [B, S] fp32)."""
    B, S, V = logits.shape
    d = capi.lm_loss_desc(B, S, V, 0, _DT[logits.dtype], ignore_index, _RED[reduction])
    ws = _workspace(d, logits.device)
    g = torch.empty(B, S, V, dtype=torch.float32, device=logits.device)
    gl = grad_loss.float().contiguous()
    capi.lm_ce_bwd(d, logits.data_ptr(), labels.data_ptr(), lse.data_ptr(), gl.data_ptr(), g.data_ptr(),
                   ws.data_ptr(), _stream())
    return g


def streaming_lm_cross_entropy(hidden, weight, labels, ignore_index=-100, reduction="mean", chunk=0,
                               check_labels=True):
    """(loss [1], lse [B, S]) from hidden [B, S, H] and weight [V, H] (both fp32
    or both bf16), without materialising the [B, S, V] logits."""
    _check(hidden, "hidden", 3)
    _check(weight, "weight", 2)
    B, S, H = hidden.shape
    V = weight.shape[0]
    if weight.shape[1] != H or weight.dtype != hidden.dtype:
        raise ValueError("selected_token_lm_cross_entropy: hidden H and weight H mismatch (or dtypes differ)")
    _labels(labels, B, S)
    d = capi.lm_loss_desc(B, S, V, H, _DT[hidden.dtype], ignore_index, _RED[reduction], chunk)
    ws = _workspace(d, hidden.device)
    loss = torch.empty(1, dtype=torch.float32, device=hidden.device)
    lse = torch.empty(B, S, dtype=torch.float32, device=hidden.device)
    status = torch.zeros(1, dtype=torch.int32, device=hidden.device)
    capi.lm_ce_streaming_fwd(d, hidden.data_ptr(), weight.data_ptr(), labels.data_ptr(), loss.data_ptr(),
                             lse.data_ptr(), status.data_ptr(), ws.data_ptr(), _stream())
    if check_labels:
        _raise_on_status(status)
    return loss, lse


def streaming_lm_cross_entropy_backward(hidden, weight, labels, lse, grad_loss, ignore_index=-100, reduction="mean",
                                        chunk=0, want_hidden=True, want_weight=True):
    """(grad_hidden [B, S, H], grad_weight [V, H]) fp32 (None where not wanted)."""
    B, S, H = hidden.shape
    V = weight.shape[0]
    d = capi.lm_loss_desc(B, S, V, H, _DT[hidden.dtype], ignore_index, _RED[reduction], chunk)
    ws = _workspace(d, hidden.device)
    gh = torch.empty(B, S, H, dtype=torch.float32, device=hidden.device) if want_hidden else None
    gw = torch.empty(V, H, dtype=torch.float32, device=hidden.device) if want_weight else None
    gl = grad_loss.float().contiguous()
    capi.lm_ce_streaming_bwd(d, hidden.data_ptr(), weight.data_ptr(), labels.data_ptr(), lse.data_ptr(),
                             gl.data_ptr(), None if gh is None else gh.data_ptr(),
                             None if gw is None else gw.data_ptr(), ws.data_ptr(), _stream())
    return gh, gw


class StreamingLMCrossEntropy(torch.autograd.Function):
    """Autograd node of streaming_lm_cross_entropy; saves hidden, weight and
    the row log-sum-exp."""

    @staticmethod
    def forward(ctx, hidden, weight, labels, ignore_index=-100, reduction="mean", chunk=0):
        loss, lse = streaming_lm_cross_entropy(hidden, weight, labels, ignore_index, reduction, chunk)
        ctx.save_for_backward(hidden, weight, labels, lse)
        ctx.cfg = (ignore_index, reduction, chunk)
        return loss

    @staticmethod
    def backward(ctx, grad_loss):
        hidden, weight, labels, lse = ctx.saved_tensors
        ignore_index, reduction, chunk = ctx.cfg
        gh, gw = streaming_lm_cross_entropy_backward(hidden, weight, labels, lse, grad_loss, ignore_index, reduction,
                                                     chunk, ctx.needs_input_grad[0], ctx.needs_input_grad[1])
        return (None if gh is None else gh.to(hidden.dtype), None if gw is None else gw.to(weight.dtype),
                None, None, None, None)
