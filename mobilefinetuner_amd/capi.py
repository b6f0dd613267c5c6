"""ctypes binding of the C ABI in ``include/mft/attention.h``,
``include/mft/prologue.h`` and ``include/mft/lm_loss.h``.

This is the binding a Python caller would use (the C++ finetune_ops adapter
links the same library directly).  It raises when the library is missing: the
HIP path is the only implementation, there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "lib", "libmft_attn.so")

MFT_OK, MFT_ERR_INVALID_ARG, MFT_ERR_UNSUPPORTED, MFT_ERR_HIP = 0, 1, 2, 3
MFT_F32, MFT_BF16 = 0, 2
NOALLOC_SCRATCH_BYTES = 128 << 20  # device scratch of mft_attn_bwd_noalloc, per GPU
MFT_BWD_DELTA, MFT_BWD_DKDV, MFT_BWD_REDUCE, MFT_BWD_DQ = 1, 2, 4, 8
MFT_BWD_MAIN, MFT_BWD_ALL = 10, 15

MFT_NORM_NONE, MFT_NORM_GEMMA, MFT_NORM_AFFINE = 0, 1, 2

# Every symbol the headers declare (checked by tests/test_capi.py).
EXPORTS = (
    "mft_attn_workspace_size", "mft_attn_fwd", "mft_attn_bwd", "mft_attn_bwd_stage", "mft_attn_bwd_noalloc",
    "mft_repeat_kv_fwd", "mft_repeat_kv_bwd", "mft_convert", "mft_last_error", "mft_version",
    "mft_prologue_fwd", "mft_prologue_workspace_size", "mft_prologue_bwd",
    "mft_prologue_fwd_n", "mft_prologue_workspace_size_n", "mft_prologue_bwd_n",
    "mft_lm_ce_workspace_size", "mft_lm_ce_fwd", "mft_lm_ce_bwd", "mft_lm_ce_streaming_fwd",
    "mft_lm_ce_streaming_bwd",
    "mft_lora_workspace_size", "mft_lora_fwd", "mft_lora_bwd", "mft_lora_merge",
)
MFT_REDUCE_MEAN, MFT_REDUCE_SUM, MFT_REDUCE_NONE = 0, 1, 2


class Strides(C.Structure):
    """mft_strides: element strides of the batch, head and sequence dims (0,0,0 = contiguous)."""
    _fields_ = [("b", C.c_int64), ("h", C.c_int64), ("s", C.c_int64)]


LAYOUTS = ("q", "k", "v", "o", "dO", "dq", "dk", "dv")


class Mask(C.Structure):
    """mft_mask: an additive fp32 mask, element (b, h, i, j) at
    ptr[b*sb + h*sh + i*si + j*sj] (zero strides broadcast); ptr NULL = none."""
    _fields_ = [("ptr", C.c_void_p), ("sb", C.c_int64), ("sh", C.c_int64), ("si", C.c_int64), ("sj", C.c_int64)]


class AttnDesc(C.Structure):
    _fields_ = [
        ("B", C.c_int64), ("Hq", C.c_int64), ("Hkv", C.c_int64), ("S", C.c_int64), ("D", C.c_int64),
        ("scale", C.c_float), ("causal", C.c_int32), ("dtype", C.c_int32),
        ("window", C.c_int32), ("kv_len", C.c_void_p),
    ] + [(n, Strides) for n in LAYOUTS] + [("mask0", Mask), ("mask1", Mask)]


class PrologueDesc(C.Structure):
    _fields_ = [
        ("B", C.c_int64), ("H", C.c_int64), ("S", C.c_int64), ("D", C.c_int64),
        ("dtype", C.c_int32), ("norm", C.c_int32), ("eps", C.c_float), ("theta", C.c_float),
    ] + [(n, Strides) for n in ("x", "y", "dy", "dx")]


class LmLossDesc(C.Structure):
    _fields_ = [("B", C.c_int64), ("S", C.c_int64), ("V", C.c_int64), ("H", C.c_int64),
                ("dtype", C.c_int32), ("ignore_index", C.c_int32), ("reduction", C.c_int32), ("chunk", C.c_int32)]


class LoraSlice(C.Structure):
    _fields_ = [("A", C.c_void_p), ("B", C.c_void_p), ("grad_A", C.c_void_p), ("grad_B", C.c_void_p),
                ("scale", C.c_float), ("a_transposed", C.c_int32), ("b_transposed", C.c_int32),
                ("rank", C.c_int64), ("col0", C.c_int64), ("cols", C.c_int64)]


class LoraDesc(C.Structure):
    _fields_ = [("N", C.c_int64), ("in_dim", C.c_int64), ("out_dim", C.c_int64), ("w_dtype", C.c_int32),
                ("w_transposed", C.c_int32), ("n_slices", C.c_int32), ("grads_for_column_slices", C.c_int32),
                ("slices", C.POINTER(LoraSlice))]


class MftError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"[mft status {status}] {msg}")
        self.status = status


_lib = None


def lib():
    """Load libmft_attn.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m mobilefinetuner_amd.build`")
    L = C.CDLL(LIB_PATH)
    vp, i64 = C.c_void_p, C.c_int64
    L.mft_version.restype = C.c_int
    L.mft_last_error.restype = C.c_char_p
    L.mft_attn_workspace_size.restype = C.c_int
    L.mft_attn_workspace_size.argtypes = [C.POINTER(AttnDesc), C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
    L.mft_attn_fwd.restype = C.c_int
    L.mft_attn_fwd.argtypes = [C.POINTER(AttnDesc), vp, vp, vp, vp, vp, vp, vp]
    L.mft_attn_bwd.restype = C.c_int
    L.mft_attn_bwd.argtypes = [C.POINTER(AttnDesc), vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    L.mft_attn_bwd_stage.restype = C.c_int
    L.mft_attn_bwd_stage.argtypes = [C.POINTER(AttnDesc), C.c_int, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    L.mft_attn_bwd_noalloc.restype = C.c_int
    L.mft_attn_bwd_noalloc.argtypes = [C.POINTER(AttnDesc), vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    L.mft_repeat_kv_fwd.restype = C.c_int
    L.mft_repeat_kv_fwd.argtypes = [vp, vp, i64, i64, i64, i64, i64, C.c_int32, vp]
    L.mft_repeat_kv_bwd.restype = C.c_int
    L.mft_repeat_kv_bwd.argtypes = [vp, vp, i64, i64, i64, i64, i64, vp]
    L.mft_convert.restype = C.c_int
    L.mft_convert.argtypes = [vp, C.c_int, vp, C.c_int, i64, vp]
    L.mft_prologue_fwd.restype = C.c_int
    L.mft_prologue_fwd.argtypes = [C.POINTER(PrologueDesc), vp, vp, vp, vp]
    L.mft_prologue_workspace_size.restype = C.c_int
    L.mft_prologue_workspace_size.argtypes = [C.POINTER(PrologueDesc), C.POINTER(C.c_size_t)]
    L.mft_prologue_bwd.restype = C.c_int
    L.mft_prologue_bwd.argtypes = [C.POINTER(PrologueDesc), vp, vp, vp, vp, vp, vp, vp]
    L.mft_prologue_fwd_n.restype = C.c_int
    L.mft_prologue_fwd_n.argtypes = [C.c_int, C.POINTER(PrologueDesc), vp, vp, vp, vp]
    L.mft_prologue_workspace_size_n.restype = C.c_int
    L.mft_prologue_workspace_size_n.argtypes = [C.c_int, C.POINTER(PrologueDesc), C.POINTER(C.c_size_t)]
    L.mft_prologue_bwd_n.restype = C.c_int
    L.mft_prologue_bwd_n.argtypes = [C.c_int, C.POINTER(PrologueDesc)] + [vp] * 7
    L.mft_lm_ce_workspace_size.restype = C.c_int
    L.mft_lm_ce_workspace_size.argtypes = [C.POINTER(LmLossDesc), C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
    L.mft_lm_ce_fwd.restype = C.c_int
    L.mft_lm_ce_fwd.argtypes = [C.POINTER(LmLossDesc)] + [vp] * 7
    L.mft_lm_ce_bwd.restype = C.c_int
    L.mft_lm_ce_bwd.argtypes = [C.POINTER(LmLossDesc)] + [vp] * 7
    L.mft_lm_ce_streaming_fwd.restype = C.c_int
    L.mft_lm_ce_streaming_fwd.argtypes = [C.POINTER(LmLossDesc)] + [vp] * 8
    L.mft_lm_ce_streaming_bwd.restype = C.c_int
    L.mft_lm_ce_streaming_bwd.argtypes = [C.POINTER(LmLossDesc)] + [vp] * 9
    L.mft_lora_workspace_size.restype = C.c_int
    L.mft_lora_workspace_size.argtypes = [C.POINTER(LoraDesc), C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
    L.mft_lora_fwd.restype = C.c_int
    L.mft_lora_fwd.argtypes = [C.POINTER(LoraDesc)] + [vp] * 7
    L.mft_lora_bwd.restype = C.c_int
    L.mft_lora_bwd.argtypes = [C.POINTER(LoraDesc)] + [vp] * 7
    L.mft_lora_merge.restype = C.c_int
    L.mft_lora_merge.argtypes = [C.POINTER(LoraDesc), vp, C.c_float, vp]
    if L.mft_version() != 7:
        raise RuntimeError("libmft_attn.so version mismatch")
    _lib = L
    return L


def check(status: int) -> None:
    if status != MFT_OK:
        raise MftError(status, lib().mft_last_error().decode())


def desc(B, Hq, Hkv, S, D, scale=-1.0, causal=True, dtype=MFT_BF16, window=0, kv_len=None,
         strides=None, masks=()) -> AttnDesc:
    """kv_len: device address of an int32 [B] array of valid keys per batch, or None.
    strides: {name: (b, h, s)} element strides per operand (names in LAYOUTS);
    missing operands are contiguous [B, H, S, D].
    masks: up to two (device address, (sb, sh, si, sj)) additive fp32 masks
    (mask mode, see mft_mask; lse then holds two floats per row)."""
    d = AttnDesc(int(B), int(Hq), int(Hkv), int(S), int(D), float(scale), int(bool(causal)), int(dtype),
                 int(window), kv_len)
    for name, st in (strides or {}).items():
        if name not in LAYOUTS:
            raise ValueError(f"unknown operand {name!r}")
        setattr(d, name, Strides(*(int(x) for x in st)))
    if len(masks) > 2:
        raise ValueError("at most two masks")
    for i, (ptr, st) in enumerate(masks):
        setattr(d, f"mask{i}", Mask(ptr, *(int(x) for x in st)))
    return d


def workspace_size(d: AttnDesc):
    f, b = C.c_size_t(), C.c_size_t()
    check(lib().mft_attn_workspace_size(C.byref(d), C.byref(f), C.byref(b)))
    return f.value, b.value


def attn_fwd(d: AttnDesc, q, k, v, o, lse, workspace, stream) -> None:
    check(lib().mft_attn_fwd(C.byref(d), q, k, v, o, lse, workspace, stream))


def attn_bwd(d: AttnDesc, q, k, v, o, dO, lse, dq, dk, dv, workspace, stream) -> None:
    check(lib().mft_attn_bwd(C.byref(d), q, k, v, o, dO, lse, dq, dk, dv, workspace, stream))


def attn_bwd_stage(d: AttnDesc, stages: int, q, k, v, o, dO, lse, dq, dk, dv, workspace, stream) -> None:
    check(lib().mft_attn_bwd_stage(C.byref(d), int(stages), q, k, v, o, dO, lse, dq, dk, dv, workspace, stream))


def attn_bwd_noalloc(d: AttnDesc, q, k, v, o, dO, lse, dq, dk, dv, stream) -> None:
    check(lib().mft_attn_bwd_noalloc(C.byref(d), q, k, v, o, dO, lse, dq, dk, dv, stream))


def repeat_kv_fwd(kv, out, B, Hkv, S, D, r, dtype, stream) -> None:
    check(lib().mft_repeat_kv_fwd(kv, out, B, Hkv, S, D, r, dtype, stream))


def repeat_kv_bwd(g, dkv, B, Hkv, S, D, r, stream) -> None:
    check(lib().mft_repeat_kv_bwd(g, dkv, B, Hkv, S, D, r, stream))


def prologue_desc(B, H, S, D, dtype=MFT_BF16, norm=MFT_NORM_GEMMA, eps=1e-6, theta=10000.0,
                  strides=None) -> PrologueDesc:
    """strides: {name: (b, h, s)} element strides of x, y, dy, dx (missing = contiguous [B, H, S, D])."""
    d = PrologueDesc(int(B), int(H), int(S), int(D), int(dtype), int(norm), float(eps), float(theta))
    for name, st in (strides or {}).items():
        if name not in ("x", "y", "dy", "dx"):
            raise ValueError(f"unknown operand {name!r}")
        setattr(d, name, Strides(*(int(v) for v in st)))
    return d


def prologue_workspace_size(d: PrologueDesc) -> int:
    n = C.c_size_t()
    check(lib().mft_prologue_workspace_size(C.byref(d), C.byref(n)))
    return n.value


def prologue_fwd(d: PrologueDesc, x, w, y, stream) -> None:
    check(lib().mft_prologue_fwd(C.byref(d), x, w, y, stream))


def prologue_bwd(d: PrologueDesc, x, w, dy, dx, dw, workspace, stream) -> None:
    check(lib().mft_prologue_bwd(C.byref(d), x, w, dy, dx, dw, workspace, stream))


def _descs(ds):
    arr = (PrologueDesc * len(ds))(*ds)
    return len(ds), arr


def _ptrs(ps):
    return (C.c_void_p * len(ps))(*[p if p else None for p in ps])


def prologue_workspace_size_n(ds) -> int:
    """mft_prologue_workspace_size_n over a list of descriptors."""
    n, arr = _descs(ds)
    out = C.c_size_t()
    check(lib().mft_prologue_workspace_size_n(n, arr, C.byref(out)))
    return out.value


def prologue_fwd_n(ds, x, w, y, stream) -> None:
    """mft_prologue_fwd_n: ds a list of descriptors, x / w / y lists of device pointers."""
    n, arr = _descs(ds)
    check(lib().mft_prologue_fwd_n(n, arr, _ptrs(x), _ptrs(w), _ptrs(y), stream))


def prologue_bwd_n(ds, x, w, dy, dx, dw, workspace, stream) -> None:
    """mft_prologue_bwd_n: lists of device pointers per operand (dw entries may be 0)."""
    n, arr = _descs(ds)
    check(lib().mft_prologue_bwd_n(n, arr, _ptrs(x), _ptrs(w), _ptrs(dy), _ptrs(dx), _ptrs(dw), workspace, stream))


def lm_loss_desc(B, S, V, H=0, dtype=MFT_F32, ignore_index=-100, reduction=MFT_REDUCE_MEAN, chunk=0) -> LmLossDesc:
    return LmLossDesc(int(B), int(S), int(V), int(H), int(dtype), int(ignore_index), int(reduction), int(chunk))


def lm_ce_workspace_size(d: LmLossDesc):
    f, b = C.c_size_t(), C.c_size_t()
    check(lib().mft_lm_ce_workspace_size(C.byref(d), C.byref(f), C.byref(b)))
    return f.value, b.value


def lm_ce_fwd(d, logits, labels, loss, lse, status, workspace, stream) -> None:
    check(lib().mft_lm_ce_fwd(C.byref(d), logits, labels, loss, lse, status, workspace, stream))


def lm_ce_bwd(d, logits, labels, lse, grad_loss, grad_logits, workspace, stream) -> None:
    check(lib().mft_lm_ce_bwd(C.byref(d), logits, labels, lse, grad_loss, grad_logits, workspace, stream))


def lm_ce_streaming_fwd(d, hidden, weight, labels, loss, lse, status, workspace, stream) -> None:
    check(lib().mft_lm_ce_streaming_fwd(C.byref(d), hidden, weight, labels, loss, lse, status, workspace, stream))


def lm_ce_streaming_bwd(d, hidden, weight, labels, lse, grad_loss, grad_hidden, grad_weight, workspace,
                        stream) -> None:
    check(lib().mft_lm_ce_streaming_bwd(C.byref(d), hidden, weight, labels, lse, grad_loss, grad_hidden,
                                        grad_weight, workspace, stream))


def lora_desc(N, in_dim, out_dim, w_dtype=MFT_F32, w_transposed=False, slices=(), grads_for_column_slices=False):
    """slices: sequence of dicts with A, B, grad_A, grad_B (device pointers or None), scale, rank, col0, cols,
    a_transposed, b_transposed.  The returned desc keeps its slice array alive."""
    arr = (LoraSlice * max(1, len(slices)))()
    for i, s in enumerate(slices):
        arr[i] = LoraSlice(s["A"], s["B"], s.get("grad_A"), s.get("grad_B"), float(s["scale"]),
                           int(bool(s.get("a_transposed", False))), int(bool(s.get("b_transposed", False))),
                           int(s["rank"]), int(s.get("col0", 0)), int(s["cols"]))
    d = LoraDesc(int(N), int(in_dim), int(out_dim), int(w_dtype), int(bool(w_transposed)), len(slices),
                 int(bool(grads_for_column_slices)), C.cast(arr, C.POINTER(LoraSlice)))
    d._slices = arr
    return d


def lora_workspace_size(d: LoraDesc):
    f, b = C.c_size_t(), C.c_size_t()
    check(lib().mft_lora_workspace_size(C.byref(d), C.byref(f), C.byref(b)))
    return f.value, b.value


def lora_fwd(d, x, W, bias, y, u, workspace, stream) -> None:
    check(lib().mft_lora_fwd(C.byref(d), x, W, bias, y, u, workspace, stream))


def lora_bwd(d, x, W, dy, u, dx, workspace, stream) -> None:
    check(lib().mft_lora_bwd(C.byref(d), x, W, dy, u, dx, workspace, stream))


def lora_merge(d, W, sign, stream) -> None:
    check(lib().mft_lora_merge(C.byref(d), W, float(sign), stream))


def convert(src, src_dtype, dst, dst_dtype, n, stream) -> None:
    """mft_convert: bf16 -> fp32 (exact) or fp32 -> bf16 (the reference's RNE) on the device."""
    check(lib().mft_convert(src, int(src_dtype), dst, int(dst_dtype), int(n), stream))
