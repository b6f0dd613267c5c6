"""LoRA-augmented linear layer on the GPU: the host-side mirror of
ops::LoRALinear (nn/lora_linear.h:36-95, nn/lora_linear.cpp) over device
tensors, computed by the mft_lora_* C ABI (include/mft/lora.h).

Same names, argument meaning and errors as the reference:

  layer = LoRALinear(W, b)                 W [in, out] or [out, in], frozen
  layer.attach_lora(A, B, scale, col0, cols)
  y = layer.forward(x)                     y = x @ W + b + sum scale * (x @ A) @ B
  layer.merge_to_base() / unmerge_from_base() / clear_lora()
  layer.trainable_parameters()             [A0, B0, A1, B1, ...]

x, b, A, B are fp32 (the reference's matmul needs an fp32 left operand and
keeps trainable weights fp32, core/ops.cpp:634-642); W is fp32 or bf16.
A slice over a column range gets no gradient, as in the reference
(nn/lora_linear.cpp:417-434), unless grads_for_column_slices is set.
"""
from __future__ import annotations

import torch

from . import capi


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


def _w_dtype(W):
    if W.dtype == torch.float32:
        return capi.MFT_F32
    if W.dtype == torch.bfloat16:
        return capi.MFT_BF16
    raise TypeError(f"matmul: unsupported right operand dtype {W.dtype}")


def _effective_shape(A, B, in_dim):
    """(rank, out, a_transposed, b_transposed) as infer_effective_lora_shape
    (nn/lora_linear.cpp:52-88) decides them."""
    if A.dim() != 2 or B.dim() != 2:
        raise RuntimeError("LoRALinear: LoRA A/B must be 2D tensors")
    if A.shape[0] == in_dim:
        rank, at = A.shape[1], False
    elif A.shape[1] == in_dim:
        rank, at = A.shape[0], True
    else:
        raise RuntimeError("LoRALinear: LoRA A shape is incompatible with input dimension")
    if B.shape[0] == rank:
        out, bt = B.shape[1], False
    elif B.shape[1] == rank:
        out, bt = B.shape[0], True
    else:
        raise RuntimeError("LoRALinear: LoRA B shape is incompatible with rank")
    return int(rank), int(out), at, bt


class _Slice:
    def __init__(self, A, B, scale, col0, cols):
        self.A, self.B, self.scale, self.col0, self.cols = A, B, float(scale), int(col0), int(cols)


class _LoRALinearFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, W, bias, layer, *ab):
        in_dim = x.shape[-1]
        N = x.numel() // in_dim
        w_t = W.shape[0] != in_dim and W.shape[1] == in_dim
        out = W.shape[0] if w_t else W.shape[1]
        if not w_t and W.shape[0] != in_dim:
            raise RuntimeError("matmul dimension mismatch: A K dimension=%d, B K dimension=%d" % (in_dim, W.shape[0]))
        slices = []
        for i, s in enumerate(layer._active_slices()):
            A, B = ab[2 * i], ab[2 * i + 1]
            rank, cols, at, bt = _effective_shape(A, B, in_dim)
            if s.col0 < 0 or s.col0 + cols > out:
                raise RuntimeError("LoRALinear: LoRA slice range exceeds base weight width")
            slices.append(dict(A=A.data_ptr(), B=B.data_ptr(), scale=s.scale, rank=rank, col0=s.col0, cols=cols,
                               a_transposed=at, b_transposed=bt))
        d = capi.lora_desc(N, in_dim, out, _w_dtype(W), w_t, slices, layer.grads_for_column_slices)
        fwd_ws, _ = capi.lora_workspace_size(d)
        dev = x.device
        R = sum(s["rank"] for s in slices)
        y = torch.empty(*x.shape[:-1], out, dtype=torch.float32, device=dev)
        u = torch.empty(N, max(R, 1), dtype=torch.float32, device=dev)
        ws = torch.empty(fwd_ws, dtype=torch.uint8, device=dev)
        capi.lora_fwd(d, x.data_ptr(), W.data_ptr(), _ptr(bias), y.data_ptr(), u.data_ptr(), ws.data_ptr(),
                      _stream(dev))
        ctx.save_for_backward(x, W, u, *ab)
        ctx.meta = (N, in_dim, out, w_t, slices, layer.grads_for_column_slices)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, W, u, *ab = ctx.saved_tensors
        N, in_dim, out, w_t, slices, all_grads = ctx.meta
        dev = x.device
        dy = dy.contiguous().float()
        grads = []
        for i, s in enumerate(slices):
            full = s["col0"] == 0 and s["cols"] == out
            if full or all_grads:
                gA, gB = torch.empty_like(ab[2 * i]), torch.empty_like(ab[2 * i + 1])
                s = dict(s, grad_A=gA.data_ptr(), grad_B=gB.data_ptr())
            else:
                gA = gB = None
            slices[i] = s
            grads += [gA, gB]
        d = capi.lora_desc(N, in_dim, out, _w_dtype(W), w_t, slices, all_grads)
        _, bwd_ws = capi.lora_workspace_size(d)
        dx = torch.empty_like(x) if ctx.needs_input_grad[0] else None
        ws = torch.empty(bwd_ws, dtype=torch.uint8, device=dev)
        capi.lora_bwd(d, x.data_ptr(), W.data_ptr(), dy.data_ptr(), u.data_ptr(), _ptr(dx), ws.data_ptr(),
                      _stream(dev))
        return (dx, None, None, None, *grads)


class LoRALinear:
    """ops::LoRALinear over device tensors (nn/lora_linear.h:36-95)."""

    def __init__(self, W_base, b_base=None, grads_for_column_slices=False):
        self._W, self._b = W_base, b_base
        self._slices = []
        self._merged = False
        self._backup = None
        self.grads_for_column_slices = bool(grads_for_column_slices)

    # -- reference interface ------------------------------------------------
    def attach_lora(self, A, B, scale, col0=0, cols=-1):
        """nn/lora_linear.cpp:299-322."""
        if A is None or B is None:
            raise RuntimeError("LoRALinear::attach_lora: A and B must not be null")
        if A.dim() != 2 or B.dim() != 2:
            raise RuntimeError("LoRALinear::attach_lora: A and B must be 2D")
        if A.dtype != torch.float32 or B.dtype != torch.float32:
            raise RuntimeError("matmul: low-precision trainable right operand is not supported; "
                               "keep trainable weights FP32")
        out_cols = int(cols)
        if out_cols <= 0:
            base_in = self._W.shape[0] if self._W.dim() == 2 else A.shape[0]
            try:
                out_cols = _effective_shape(A, B, base_in)[1]
            except RuntimeError:
                out_cols = _effective_shape(A, B, self._W.shape[1])[1]
        A.requires_grad_(True)
        B.requires_grad_(True)
        self._slices.append(_Slice(A, B, scale, col0, out_cols))

    def clear_lora(self):
        if self._merged:
            self.unmerge_from_base()
        self._slices = []
        self._merged = False
        self._backup = None

    def merge_to_base(self):
        """Bake each slice's scale * A . B into W (apply_lora_delta_to_base), keeping a
        byte copy of W for unmerge_from_base, as the reference does."""
        if self._merged or not self._slices:
            return
        self._backup = self._W.detach().clone()
        self._merge(+1.0)
        self._merged = True

    def unmerge_from_base(self):
        if not self._merged or not self._slices:
            return
        with torch.no_grad():
            if self._backup is not None:
                self._W.copy_(self._backup)
                self._backup = None
                self._merged = False
                return
        self._merge(-1.0)
        self._merged = False

    def forward(self, x):
        if x.dtype != torch.float32:
            raise RuntimeError("matmul: left operand must be float32 for mixed-precision CPU kernels")
        _w_dtype(self._W)
        if self._b is not None and self._b.dtype != torch.float32:
            raise TypeError("LoRALinear: bias must be fp32")
        ab = []
        for s in self._active_slices():
            ab += [s.A.contiguous(), s.B.contiguous()]
        return _LoRALinearFn.apply(x.contiguous(), self._W.detach().contiguous(),
                                   None if self._b is None else self._b.detach().contiguous(), self, *ab)

    __call__ = forward

    def trainable_parameters(self):
        out = []
        for s in self._slices:
            out += [s.A, s.B]
        return out

    @property
    def W(self):
        return self._W

    @property
    def b(self):
        return self._b

    def slices(self):
        return list(self._slices)

    def is_merged(self):
        return self._merged

    # -- internals ----------------------------------------------------------
    def _active_slices(self):
        return [] if self._merged else self._slices

    def _merge(self, sign):
        W = self._W
        in_dim = W.shape[0]
        slices, keep = [], []  # keep: the contiguous operands stay alive until the launch is enqueued
        for s in self._slices:
            rank, cols, at, bt = _effective_shape(s.A, s.B, in_dim)
            if s.cols != cols:
                raise RuntimeError("LoRALinear: LoRA slice cols do not match B output dimension")
            if s.col0 < 0 or s.col0 + cols > W.shape[1]:
                raise RuntimeError("LoRALinear: LoRA slice range exceeds base weight width")
            A, B = s.A.detach().contiguous(), s.B.detach().contiguous()
            keep += [A, B]
            slices.append(dict(A=A.data_ptr(), B=B.data_ptr(), scale=s.scale, rank=rank, col0=s.col0, cols=cols,
                               a_transposed=at, b_transposed=bt))
        d = capi.lora_desc(1, in_dim, W.shape[1], _w_dtype(W), False, slices)
        capi.lora_merge(d, W.data_ptr(), sign, _stream(W.device))
        del keep  # the caching allocator reuses this memory only after the merge on this stream
