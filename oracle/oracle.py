"""ctypes bindings for the CPU oracle (TEST INFRASTRUCTURE ONLY).

Loads ``oracle/librefcpu.so`` (this repository's C++ restatement of the
reference attention composite) and, where it was built, ``oracle/_ref/
libmftref.so`` (the reference's own operators compiled from its sources).
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg import this module; the product path never does.

Each wrapper names the reference function it restates; the C files carry the
file:line citations.
"""
from __future__ import annotations

import ctypes as C
import math
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librefcpu.so")
REF_PATH = os.path.join(HERE, "_ref", "libmftref.so")

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i64 = C.c_int64

_lib = None
_ref = None


def build() -> None:
    """Compile the oracle (and the reference CPU path where its sources exist)."""
    subprocess.run(["make", "-s", "-C", HERE, "-j8"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run make -C oracle)")
        L = C.CDLL(LIB_PATH)
        L.orc_uniform.restype = C.c_double
        L.orc_uniform.argtypes = [C.c_uint64, C.c_uint32, C.c_uint64]
        L.orc_fill_normal.argtypes = [_f32p, _i64, C.c_uint64, C.c_uint32, C.c_float]
        L.orc_fill_mod.argtypes = [_f32p, _i64, C.c_float, C.c_int, C.c_int]
        L.orc_stress_rows.argtypes = [_f32p, _i64, _i64, _i64, _i64, _i64, C.c_float, C.c_uint64]
        L.orc_f32_to_bf16_bits.restype = C.c_uint16
        L.orc_f32_to_bf16_bits.argtypes = [C.c_float]
        L.orc_round_bf16.argtypes = [_f32p, _i64]
        L.orc_to_bf16_bits.argtypes = [_f32p, _u16p, _i64]
        L.orc_from_bf16_bits.argtypes = [_u16p, _f32p, _i64]
        opt_f32 = C.c_void_p
        L.orc_attn_composite.restype = C.c_int
        L.orc_attn_composite.argtypes = [_f32p, _f32p, _f32p, opt_f32,
                                         _i64, _i64, _i64, _i64, _i64, C.c_float, C.c_int,
                                         opt_f32, opt_f32, opt_f32, opt_f32, opt_f32]
        L.orc_attn_composite_masked.restype = C.c_int
        L.orc_attn_composite_masked.argtypes = [_f32p, _f32p, _f32p, opt_f32,
                                                _i64, _i64, _i64, _i64, _i64, C.c_float, C.c_int,
                                                opt_f32, opt_f32,
                                                opt_f32, opt_f32, opt_f32, opt_f32, opt_f32]
        L.orc_attn_streaming.restype = C.c_int
        L.orc_attn_streaming.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64,
                                         C.c_float, C.c_int, _f32p]
        L.orc_attn_streaming_mask.restype = C.c_int
        L.orc_attn_streaming_mask.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64,
                                              C.c_float, C.c_int, opt_f32, _f32p]
        L.orc_attn_composite_masks.restype = C.c_int
        L.orc_attn_composite_masks.argtypes = [_f32p, _f32p, _f32p, opt_f32,
                                               _i64, _i64, _i64, _i64, _i64, C.c_float, C.c_int,
                                               opt_f32, opt_f32, opt_f32, opt_f32,
                                               opt_f32, opt_f32, opt_f32, opt_f32, opt_f32, opt_f32]
        L.orc_attn_f64.restype = C.c_int
        L.orc_attn_f64.argtypes = [_f32p, _f32p, _f32p, opt_f32,
                                   _i64, _i64, _i64, _i64, _i64, C.c_double, C.c_int,
                                   opt_f32, opt_f32, opt_f32, opt_f32, opt_f32]
        L.orc_repeat_kv.argtypes = [_f32p, _f32p, _i64, _i64, _i64, _i64, _i64]
        L.orc_repeat_kv_backward.argtypes = [_f32p, _f32p, _i64, _i64, _i64, _i64, _i64]
        L.orc_lm_ce.restype = C.c_int
        L.orc_lm_ce.argtypes = [_f32p, C.c_void_p, _i64, _i64, _i64, C.c_int, C.c_int, C.c_void_p, _f32p, C.c_void_p]
        L.orc_selected_ce.restype = C.c_int
        L.orc_selected_ce.argtypes = [_f32p, _f32p, C.c_void_p, _i64, _i64, _i64, _i64, C.c_int, C.c_int, C.c_float,
                                      _f32p, C.c_void_p, C.c_void_p]
        L.orc_prologue_fwd.argtypes = [_f32p, C.c_void_p, _i64, _i64, _i64, _i64, C.c_int, C.c_float, C.c_float,
                                       _f32p]
        L.orc_lora.argtypes = [_f32p, _f32p, C.c_void_p, _i64, _i64, _i64, C.c_int, C.c_int, C.c_int, C.c_void_p, _f32p,
                               _f32p, _f32p, C.c_int, C.c_void_p, _f32p, C.c_void_p, _f32p, _f32p, C.c_void_p]
        L.orc_lora_merge.argtypes = [_f32p, C.c_int, _i64, _i64, C.c_int, C.c_void_p, _f32p, _f32p, _f32p,
                                     C.c_float]
        L.orc_prologue_bwd.argtypes = [_f32p, C.c_void_p, _f32p, _i64, _i64, _i64, _i64, C.c_int, C.c_float,
                                       C.c_float, _f32p, C.c_void_p]
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref():
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError(f"reference CPU library missing: {REF_PATH}")
        R = C.CDLL(REF_PATH)
        opt = C.c_void_p
        R.mftref_composite.restype = C.c_int
        R.mftref_composite.argtypes = [_f32p, _f32p, _f32p, opt, _i64, _i64, _i64, _i64, _i64,
                                       C.c_float, C.c_int, opt, opt, opt, opt,
                                       C.POINTER(C.c_double), C.POINTER(C.c_double),
                                       C.POINTER(C.c_int64)]
        R.mftref_composite_saved.restype = C.c_int
        R.mftref_composite_saved.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _i64,
                                             C.c_float, C.c_int, _f32p, C.POINTER(C.c_int64)]
        R.mftref_memeff_nograd.restype = C.c_int
        R.mftref_memeff_nograd.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64,
                                           C.c_float, C.c_int, _f32p]
        R.mftref_memeff_grad.restype = C.c_int
        R.mftref_memeff_grad.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, _i64,
                                         C.c_float, C.c_int, _f32p, _f32p, _f32p, _f32p]
        R.mftref_repeat_kv.restype = C.c_int
        R.mftref_repeat_kv.argtypes = [_f32p, opt, _i64, _i64, _i64, _i64, _i64, _f32p, opt]
        R.mftref_lm_ce.restype = C.c_int
        R.mftref_lm_ce.argtypes = [_f32p, opt, _i64, _i64, _i64, C.c_int, C.c_int, opt, _f32p, opt]
        R.mftref_streaming_ce.restype = C.c_int
        R.mftref_streaming_ce.argtypes = [_f32p, _f32p, opt, _i64, _i64, _i64, _i64, C.c_int, C.c_int, C.c_float,
                                          _f32p, opt, opt]
        R.mftref_prologue.restype = C.c_int
        R.mftref_prologue.argtypes = [_f32p, opt, opt, _i64, _i64, _i64, _i64, C.c_int, C.c_float, C.c_float,
                                      _f32p, opt, opt]
        R.mftref_f32_to_bf16_bits.restype = C.c_uint16
        R.mftref_lora.argtypes = [_f32p, _f32p, C.c_void_p, _i64, _i64, _i64, C.c_int, C.c_int, C.c_int,
                                  C.c_void_p, _f32p, _f32p, _f32p, C.c_void_p, _f32p, C.c_void_p, _f32p, _f32p,
                                  C.c_void_p]
        R.mftref_lora_merge.argtypes = [_f32p, C.c_int, _i64, _i64, C.c_int, C.c_void_p, _f32p, _f32p, _f32p]
        R.mftref_f32_to_bf16_bits.argtypes = [C.c_float]
        _ref = R
    return _ref


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- generator
def uniform(seed: int, stream: int, counter: int) -> float:
    """The generator's 53-bit uniform in (0, 1) (splitmix64 of seed, stream, counter)."""
    return float(lib().orc_uniform(seed, stream, counter))


def normal(n: int, seed: int, stream: int, sigma: float = 1.0) -> np.ndarray:
    x = np.empty(n, dtype=np.float32)
    lib().orc_fill_normal(x, n, seed, stream, sigma)
    return x


def fill_mod(n: int, a: float, m: int, o: int) -> np.ndarray:
    x = np.empty(n, dtype=np.float32)
    lib().orc_fill_mod(x, n, a, m, o)
    return x


def round_bf16(x: np.ndarray) -> np.ndarray:
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    lib().orc_round_bf16(y.reshape(-1), y.size)
    return y


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_to_bf16_bits(x.reshape(-1), out.reshape(-1), x.size)
    return out


# ------------------------------------------------------------------ configs
# BASELINE.json configs; seed = 1000 + config number, streams Q=0 K=1 V=2 dO=3.
CONFIGS = {
    "c1": dict(B=4, Hq=12, Hkv=12, D=64, S=128, dtype="f32", scale=1 / 8, do_sigma=1.0, stress=False,
               name="GPT-2-small MHA fp32"),
    "c2": dict(B=4, Hq=16, Hkv=16, D=64, S=512, dtype="f32", scale=1 / 8, do_sigma=0.1, stress=False,
               name="GPT-2-medium MHA fp32"),
    "c3": dict(B=2, Hq=14, Hkv=2, D=64, S=2048, dtype="bf16", scale=1 / 8, do_sigma=0.1, stress=False,
               name="Qwen2.5-0.5B GQA bf16"),
    "c4": dict(B=4, Hq=4, Hkv=1, D=256, S=1024, dtype="bf16", scale=1 / 16, do_sigma=0.1, stress=True,
               name="Gemma-3-270M GQA bf16 (K-row stress)"),
    "c5": dict(B=1, Hq=4, Hkv=1, D=256, S=4096, dtype="bf16", scale=1 / 16, do_sigma=0.1, stress=False,
               name="Gemma-3-1B GQA bf16"),
    "c5f32": dict(B=1, Hq=4, Hkv=1, D=256, S=4096, dtype="f32", scale=1 / 16, do_sigma=0.1, stress=False,
                  name="Gemma-3-1B GQA fp32 exactness variant"),
}
SEEDS = {"c1": 1001, "c2": 1002, "c3": 1003, "c4": 1004, "c5": 1005, "c5f32": 1005}


def make_inputs(B, Hq, Hkv, S, D, seed, dtype="f32", do_sigma=1.0, stress=False):
    """Seeded Q, K, V, dO as float32 arrays ([B,H,S,D]).  For bf16 the values
    are rounded to bf16 (RNE), so the fp32 oracle sees exactly the kernel input."""
    q = normal(B * Hq * S * D, seed, 0).reshape(B, Hq, S, D)
    k = normal(B * Hkv * S * D, seed, 1).reshape(B, Hkv, S, D)
    v = normal(B * Hkv * S * D, seed, 2).reshape(B, Hkv, S, D)
    do = normal(B * Hq * S * D, seed, 3, do_sigma).reshape(B, Hq, S, D)
    if stress:
        cnt = int(round(0.01 * S))
        lib().orc_stress_rows(k.reshape(-1), B, Hkv, S, D, cnt, 8.0, seed)
    if dtype == "bf16":
        q, k, v, do = (round_bf16(t) for t in (q, k, v, do))
    return q, k, v, do


def config_inputs(cfg_id):
    c = CONFIGS[cfg_id]
    return make_inputs(c["B"], c["Hq"], c["Hkv"], c["S"], c["D"], SEEDS[cfg_id], c["dtype"],
                       c["do_sigma"], c["stress"])


# ---------------------------------------------------------------- composite
def composite(q, k, v, dO=None, scale=None, causal=True, want_lse=False):
    """Reference composite forward (+ Engine backward if dO is given)."""
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    q, k, v = (np.ascontiguousarray(t, dtype=np.float32) for t in (q, k, v))
    o = np.empty_like(q)
    lse = np.empty((B, Hq, S), dtype=np.float32) if want_lse else None
    dq = dk = dv = None
    if dO is not None:
        dO = np.ascontiguousarray(dO, dtype=np.float32)
        dq = np.empty_like(q)
        dk = np.empty_like(k)
        dv = np.empty_like(v)
    rc = lib().orc_attn_composite(q, k, v, _ptr(dO), B, Hq, Hkv, S, D, float(scale), int(causal),
                                  _ptr(o), _ptr(lse), _ptr(dq), _ptr(dk), _ptr(dv))
    if rc != 0:
        raise ValueError("orc_attn_composite rejected its arguments")
    return dict(o=o, lse=lse, dq=dq, dk=dk, dv=dv)


def composite_sliced(q, k, v, dO, scale=None, causal=True, threads=16):
    """composite() computed one (batch, query head) at a time on `threads`
    threads, bit-identical to composite() on the whole tensors: every head's
    arithmetic is independent of the others, and the kv-head gradients are
    summed over the query heads of their group in head order starting from 0,
    ((0 + g_0) + g_1) + ..., as RepeatKVHeadsBackward::apply does
    (core/backward_functions.cpp:693-726).  For the full config sizes."""
    from concurrent.futures import ThreadPoolExecutor
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    r = Hq // Hkv

    def one(bh):
        b, h = bh
        g = h // r
        return composite(q[b:b + 1, h:h + 1], k[b:b + 1, g:g + 1], v[b:b + 1, g:g + 1], dO[b:b + 1, h:h + 1],
                         scale=scale, causal=causal, want_lse=True)

    jobs = [(b, h) for b in range(B) for h in range(Hq)]
    with ThreadPoolExecutor(max(1, min(threads, len(jobs)))) as ex:
        parts = list(ex.map(one, jobs))
    o = np.empty_like(q, dtype=np.float32)
    lse = np.empty((B, Hq, S), np.float32)
    dq = np.empty_like(q, dtype=np.float32)
    dk = np.zeros(k.shape, np.float32)
    dv = np.zeros(v.shape, np.float32)
    for (b, h), p in zip(jobs, parts):
        g = h // r
        o[b, h], lse[b, h], dq[b, h] = p["o"][0, 0], p["lse"][0, 0], p["dq"][0, 0]
        dk[b, g] = dk[b, g] + p["dk"][0, 0]
        dv[b, g] = dv[b, g] + p["dv"][0, 0]
    return dict(o=o, lse=lse, dq=dq, dk=dk, dv=dv)


# ------------------------------------------------------------------ masks
MASK_VALUE = np.float32(-1e10)  # kMaskValue, graph/gemma_model.cpp:175


def causal_mask(S):
    """create_causal_mask (core/ops.cpp:2167-2180): -1e10 above the diagonal."""
    m = np.zeros((S, S), np.float32)
    m[np.triu_indices(S, 1)] = MASK_VALUE
    return m


def sliding_mask(S, window):
    """GemmaModel::build_sliding_mask (graph/gemma_model.cpp:272-285): key j is
    allowed for query i iff j <= i and i - j < window."""
    i = np.arange(S)[:, None]
    j = np.arange(S)[None, :]
    allow = (j <= i) & (i - j < window)
    return np.where(allow, np.float32(0), MASK_VALUE).astype(np.float32)


def padding_mask(attention_mask):
    """GemmaModel::build_padding_mask (graph/gemma_model.cpp:287-321) from a
    [B,S] attention mask (float: <= 0.5 is padding; int32: 0 is padding);
    returns the [B,S] additive mask (the [B,1,1,S] tensor without its unit dims)."""
    am = np.asarray(attention_mask)
    pad = am <= 0.5 if am.dtype.kind == "f" else am == 0
    return np.where(pad, MASK_VALUE, np.float32(0)).astype(np.float32)


def lengths_attention_mask(lengths, S):
    """[B,S] int32 attention mask with the first lengths[b] tokens real."""
    return (np.arange(S)[None, :] < np.asarray(lengths)[:, None]).astype(np.int32)


def composite_masked(q, k, v, dO=None, scale=None, base_mask=None, pad_mask=None, causal=True,
                     want_lse=False):
    """Reference composite with additive masks: base_mask [S,S] (None: the
    causal mask when causal) then pad_mask [B,S]."""
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    q, k, v = (np.ascontiguousarray(t, dtype=np.float32) for t in (q, k, v))
    bm = None if base_mask is None else np.ascontiguousarray(base_mask, np.float32)
    pm = None if pad_mask is None else np.ascontiguousarray(pad_mask, np.float32)
    o = np.empty_like(q)
    lse = np.empty((B, Hq, S), dtype=np.float32) if want_lse else None
    dq = dk = dv = None
    if dO is not None:
        dO = np.ascontiguousarray(dO, dtype=np.float32)
        dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    rc = lib().orc_attn_composite_masked(q, k, v, _ptr(dO), B, Hq, Hkv, S, D, float(scale), int(causal),
                                         _ptr(bm), _ptr(pm), _ptr(o), _ptr(lse), _ptr(dq), _ptr(dk), _ptr(dv))
    if rc != 0:
        raise ValueError("orc_attn_composite_masked rejected its arguments")
    return dict(o=o, lse=lse, dq=dq, dk=dk, dv=dv)


def mask_strides(m, B, Hq, S):
    """Element strides (sb, sh, si, sj) of an additive mask array [S,S] or
    [1|B, 1|Hq, 1|S, S] broadcast over [B, Hq, S, S] (0 for broadcast dims),
    and the array as a C-contiguous 4-D float32 array."""
    m = np.ascontiguousarray(m, dtype=np.float32)
    if m.ndim == 2:
        m = m.reshape(1, 1, *m.shape)
    if m.ndim != 4 or m.shape[3] != S or any(m.shape[i] not in (1, n) for i, n in enumerate((B, Hq, S))):
        raise ValueError(f"mask shape {m.shape} does not broadcast to [B, Hq, S, S]")
    st = [0 if m.shape[i] == 1 else m.strides[i] // 4 for i in range(4)]
    return m, np.asarray(st, dtype=np.int64)


def composite_masks(q, k, v, dO=None, scale=None, mode=0, masks=(), want_lse=False):
    """Reference composite with the mask mode of the C ABI: mode 0 (no causal
    rule), 1 (-1e10 replaces the scores above the diagonal: the no-grad
    operator's rule) or 2 (create_causal_mask added), then up to two additive
    masks ([S,S] or [1|B, 1|Hq, 1|S, S]) in order.  lse2 (want_lse): [B,Hq,S,2]
    row max and ln of the row sum."""
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    q, k, v = (np.ascontiguousarray(t, dtype=np.float32) for t in (q, k, v))
    ms = [mask_strides(m, B, Hq, S) for m in masks]
    if len(ms) > 2:
        raise ValueError("at most two masks")
    (m0, s0), (m1, s1) = (ms + [(None, None)] * 2)[:2]
    o = np.empty_like(q)
    lse2 = np.empty((B, Hq, S, 2), dtype=np.float32) if want_lse else None
    dq = dk = dv = None
    if dO is not None:
        dO = np.ascontiguousarray(dO, dtype=np.float32)
        dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    rc = lib().orc_attn_composite_masks(q, k, v, _ptr(dO), B, Hq, Hkv, S, D, float(scale), int(mode),
                                        _ptr(m0), _ptr(s0), _ptr(m1), _ptr(s1),
                                        _ptr(o), None, _ptr(lse2), _ptr(dq), _ptr(dk), _ptr(dv))
    if rc != 0:
        raise ValueError("orc_attn_composite_masks rejected its arguments")
    return dict(o=o, lse2=lse2, dq=dq, dk=dk, dv=dv)


def streaming_mask(q, k, v, mask, scale=None, causal=True):
    """The no-grad operator with its [S,S] mask (core/memory_efficient_attention.cpp:110-200)."""
    B, H, S, D = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    o = np.empty_like(q)
    m = None if mask is None else np.ascontiguousarray(mask, np.float32)
    rc = lib().orc_attn_streaming_mask(np.ascontiguousarray(q), np.ascontiguousarray(k), np.ascontiguousarray(v),
                                       B, H, S, D, float(scale), int(causal), _ptr(m), o)
    if rc != 0:
        raise ValueError("orc_attn_streaming_mask rejected its arguments")
    return o


def streaming(q, k, v, scale=None, causal=True):
    B, H, S, D = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    o = np.empty_like(q)
    rc = lib().orc_attn_streaming(np.ascontiguousarray(q), np.ascontiguousarray(k),
                                  np.ascontiguousarray(v), B, H, S, D, float(scale), int(causal), o)
    if rc != 0:
        raise ValueError("orc_attn_streaming rejected its arguments")
    return o


def brute_f64(q, k, v, dO=None, scale=None, causal=True):
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    o = np.empty(q.shape, np.float64)
    lse = np.empty((B, Hq, S), np.float64)
    dq = dk = dv = None
    if dO is not None:
        dO = np.ascontiguousarray(dO, dtype=np.float32)
        dq = np.empty(q.shape, np.float64)
        dk = np.empty(k.shape, np.float64)
        dv = np.empty(v.shape, np.float64)
    rc = lib().orc_attn_f64(np.ascontiguousarray(q), np.ascontiguousarray(k), np.ascontiguousarray(v),
                            _ptr(dO), B, Hq, Hkv, S, D, float(scale), int(causal),
                            _ptr(o), _ptr(lse), _ptr(dq), _ptr(dk), _ptr(dv))
    if rc != 0:
        raise ValueError("orc_attn_f64 rejected its arguments")
    return dict(o=o, lse=lse, dq=dq, dk=dk, dv=dv)


def repeat_kv(kv, r):
    B, H, S, D = kv.shape
    out = np.empty((B, H * r, S, D), np.float32)
    lib().orc_repeat_kv(np.ascontiguousarray(kv), out, B, H, S, D, r)
    return out


def repeat_kv_backward(g, r):
    B, Hr, S, D = g.shape
    out = np.empty((B, Hr // r, S, D), np.float32)
    lib().orc_repeat_kv_backward(np.ascontiguousarray(g), out, B, Hr // r, S, D, r)
    return out


NORMS = {"none": 0, "gemma": 1, "affine": 2}


def prologue(x, w=None, dy=None, norm="gemma", eps=1e-6, theta=10000.0):
    """y = rope(norm(x)) per row of x [B, H, S, D] (fp32), and with dy the
    backward: dict(y, dx, dw).  norm: "none", "gemma" (ops::rms_norm,
    x / rms * (1 + w)) or "affine" (ops::rms_norm_affine); theta 0 = no RoPE."""
    B, H, S, D = x.shape
    x = np.ascontiguousarray(x, np.float32)
    nm = NORMS[norm]
    wp = None if w is None else np.ascontiguousarray(w, np.float32)
    y = np.empty_like(x)
    lib().orc_prologue_fwd(x, _ptr(wp), B, H, S, D, nm, float(eps), float(theta), y)
    out = dict(y=y)
    if dy is not None:
        dx = np.empty_like(x)
        dw = np.empty(D, np.float32) if nm else None
        lib().orc_prologue_bwd(x, _ptr(wp), np.ascontiguousarray(dy, np.float32), B, H, S, D, nm, float(eps),
                               float(theta), dx, _ptr(dw))
        out.update(dx=dx, dw=dw)
    return out


REDUCTIONS = {"mean": 0, "sum": 1, "none": 2}


def _ce_dense(fn, logits, labels, ignore_index, reduction, grad_out):
    B, S, V = logits.shape
    logits = np.ascontiguousarray(logits, np.float32)
    labels = np.ascontiguousarray(labels, np.int32)
    red = REDUCTIONS[reduction]
    loss = np.zeros((B, S) if red == 2 else (1,), np.float32)
    g = None
    if grad_out is not None:
        g = np.ascontiguousarray(np.broadcast_to(np.float32(grad_out), loss.shape), np.float32)
    grad = np.zeros_like(logits) if g is not None else None
    rc = fn(logits, labels.ctypes.data, B, S, V, int(ignore_index), red, _ptr(g), loss, _ptr(grad))
    if rc != 0:
        raise ValueError("lm_cross_entropy: label out of range")
    return dict(loss=loss, grad=grad)


def lm_ce(logits, labels, ignore_index=-100, reduction="mean", grad_out=None):
    """ops::lm_cross_entropy on logits [B, S, V] (fp32) and int32 labels [B, S];
    with grad_out (scalar, or [B, S] for "none") also the logits gradient."""
    return _ce_dense(lib().orc_lm_ce, logits, labels, ignore_index, reduction, grad_out)


def _ce_stream(fn, hidden, weight, labels, ignore_index, reduction, grad_out):
    B, S, H = hidden.shape
    V = weight.shape[0]
    hidden = np.ascontiguousarray(hidden, np.float32)
    weight = np.ascontiguousarray(weight, np.float32)
    labels = np.ascontiguousarray(labels, np.int32)
    loss = np.zeros(1, np.float32)
    gh = np.zeros_like(hidden) if grad_out is not None else None
    gw = np.zeros_like(weight) if grad_out is not None else None
    rc = fn(hidden, weight, labels.ctypes.data, B, S, H, V, int(ignore_index), REDUCTIONS[reduction],
            float(1.0 if grad_out is None else grad_out), loss, _ptr(gh), _ptr(gw))
    if rc != 0:
        raise ValueError("lm_cross_entropy: label out of range")
    return dict(loss=loss, grad_hidden=gh, grad_weight=gw)


def selected_ce(hidden, weight, labels, ignore_index=-100, reduction="mean", grad_out=None):
    """ops::selected_token_lm_cross_entropy (= streaming) on fp32 hidden
    [B, S, H] and weight [V, H]; reduction "mean" or "sum"."""
    return _ce_stream(lib().orc_selected_ce, hidden, weight, labels, ignore_index, reduction, grad_out)


# ------------------------------------------------- reference (oracle/_ref)
def ref_composite(q, k, v, dO=None, scale=None, causal=True):
    """The reference's own operators (compiled from its sources)."""
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    q, k, v = (np.ascontiguousarray(t, dtype=np.float32) for t in (q, k, v))
    o = np.empty_like(q)
    dq = dk = dv = None
    if dO is not None:
        dO = np.ascontiguousarray(dO, dtype=np.float32)
        dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    tf, tb, held = C.c_double(), C.c_double(), C.c_int64()
    rc = ref().mftref_composite(q, k, v, _ptr(dO), B, Hq, Hkv, S, D, float(scale), int(causal),
                                _ptr(o), _ptr(dq), _ptr(dk), _ptr(dv),
                                C.byref(tf), C.byref(tb), C.byref(held))
    if rc != 0:
        raise RuntimeError("reference composite raised")
    return dict(o=o, dq=dq, dk=dk, dv=dv, t_fwd=tf.value, t_bwd=tb.value, held_bytes=held.value)


def ref_saved_bytes(q, k, v, scale=None, causal=True):
    """MemoryManager bytes the reference composite's autograd graph holds
    after its forward (inputs requiring grad; no backward is run)."""
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    q, k, v = (np.ascontiguousarray(t, dtype=np.float32) for t in (q, k, v))
    o = np.empty_like(q)
    held = C.c_int64()
    rc = ref().mftref_composite_saved(q, k, v, B, Hq, Hkv, S, D, float(scale), int(causal), o,
                                      C.byref(held))
    if rc != 0:
        raise RuntimeError("reference composite raised")
    return held.value


def ref_composite_masked(q, k, v, dO=None, scale=None, base_mask=None, pad_mask=None):
    """The reference's composite with additive masks (ref_harness.cpp)."""
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    q, k, v = (np.ascontiguousarray(t, dtype=np.float32) for t in (q, k, v))
    bm = None if base_mask is None else np.ascontiguousarray(base_mask, np.float32)
    pm = None if pad_mask is None else np.ascontiguousarray(pad_mask, np.float32)
    o = np.empty_like(q)
    dq = dk = dv = None
    if dO is not None:
        dO = np.ascontiguousarray(dO, dtype=np.float32)
        dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    R = ref()
    R.mftref_composite_masked.restype = C.c_int
    R.mftref_composite_masked.argtypes = [_f32p, _f32p, _f32p, C.c_void_p, _i64, _i64, _i64, _i64, _i64,
                                          C.c_float, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                          C.c_void_p, C.c_void_p]
    rc = R.mftref_composite_masked(q, k, v, _ptr(dO), B, Hq, Hkv, S, D, float(scale), _ptr(bm), _ptr(pm),
                                   _ptr(o), _ptr(dq), _ptr(dk), _ptr(dv))
    if rc != 0:
        raise RuntimeError("reference composite (masked) raised")
    return dict(o=o, dq=dq, dk=dk, dv=dv)


def ref_composite_mask4(q, k, v, dO=None, scale=None, masks=()):
    """The reference composite with up to two dense masks [1|B, 1|Hq, 1|S, S]
    added by its own broadcasting ops::add (ref_harness.cpp)."""
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    q, k, v = (np.ascontiguousarray(t, dtype=np.float32) for t in (q, k, v))
    dense = []
    for m in masks:
        m = np.ascontiguousarray(m, np.float32)
        if m.ndim == 2:
            m = m.reshape(1, 1, *m.shape)
        dense.append(m)
    dense += [None] * (2 - len(dense))
    o = np.empty_like(q)
    dq = dk = dv = None
    if dO is not None:
        dO = np.ascontiguousarray(dO, dtype=np.float32)
        dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    R = ref()
    R.mftref_composite_mask4.restype = C.c_int
    R.mftref_composite_mask4.argtypes = [_f32p, _f32p, _f32p, C.c_void_p, _i64, _i64, _i64, _i64, _i64, C.c_float,
                                         C.c_void_p, _i64, _i64, _i64, C.c_void_p, _i64, _i64, _i64,
                                         C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
    shp = [(m.shape[0], m.shape[1], m.shape[2]) if m is not None else (1, 1, 1) for m in dense]
    rc = R.mftref_composite_mask4(q, k, v, _ptr(dO), B, Hq, Hkv, S, D, float(scale),
                                  _ptr(dense[0]), *shp[0], _ptr(dense[1]), *shp[1],
                                  _ptr(o), _ptr(dq), _ptr(dk), _ptr(dv))
    if rc != 0:
        raise RuntimeError("reference composite (mask4) raised")
    return dict(o=o, dq=dq, dk=dk, dv=dv)


def ref_memeff_nograd_mask(q, k, v, mask, scale=None, causal=True):
    B, H, S, D = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    o = np.empty_like(q)
    R = ref()
    R.mftref_memeff_nograd_mask.restype = C.c_int
    R.mftref_memeff_nograd_mask.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, C.c_float, C.c_int,
                                            _f32p, _f32p]
    rc = R.mftref_memeff_nograd_mask(np.ascontiguousarray(q), np.ascontiguousarray(k), np.ascontiguousarray(v),
                                     B, H, S, D, float(scale), int(causal),
                                     np.ascontiguousarray(mask, np.float32), o)
    if rc != 0:
        raise RuntimeError("reference memory_efficient_attention (mask) raised")
    return o


def ref_memeff_nograd(q, k, v, scale=None, causal=True):
    B, H, S, D = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    o = np.empty_like(q)
    rc = ref().mftref_memeff_nograd(np.ascontiguousarray(q), np.ascontiguousarray(k),
                                    np.ascontiguousarray(v), B, H, S, D, float(scale), int(causal), o)
    if rc != 0:
        raise RuntimeError("reference memory_efficient_attention raised")
    return o


def ref_repeat_kv(kv, r, g=None):
    B, H, S, D = kv.shape
    out = np.empty((B, H * r, S, D), np.float32)
    dkv = np.empty_like(kv) if g is not None else None
    rc = ref().mftref_repeat_kv(np.ascontiguousarray(kv),
                                _ptr(None if g is None else np.ascontiguousarray(g)),
                                B, H, S, D, r, out, _ptr(dkv))
    if rc != 0:
        raise RuntimeError("reference repeat_kv_heads raised")
    return out, dkv


def ref_lm_ce(logits, labels, ignore_index=-100, reduction="mean", grad_out=None):
    """The reference's lm_cross_entropy and Engine backward (same contract as lm_ce)."""
    return _ce_dense(ref().mftref_lm_ce, logits, labels, ignore_index, reduction, grad_out)


def ref_streaming_ce(hidden, weight, labels, ignore_index=-100, reduction="mean", grad_out=None):
    """The reference's streaming_lm_cross_entropy and Engine backward."""
    return _ce_stream(ref().mftref_streaming_ce, hidden, weight, labels, ignore_index, reduction, grad_out)


def ref_prologue(x, w=None, dy=None, norm="gemma", eps=1e-6, theta=10000.0):
    """The reference's rms_norm / rms_norm_affine and apply_rope with their
    Engine backward (compiled from its sources); same contract as prologue()."""
    B, H, S, D = x.shape
    x = np.ascontiguousarray(x, np.float32)
    nm = NORMS[norm]
    wp = None if w is None else np.ascontiguousarray(w, np.float32)
    y = np.empty_like(x)
    dx = np.empty_like(x) if dy is not None else None
    dw = np.empty(D, np.float32) if (dy is not None and nm) else None
    rc = ref().mftref_prologue(x, _ptr(wp), _ptr(None if dy is None else np.ascontiguousarray(dy, np.float32)),
                               B, H, S, D, nm, float(eps), float(theta), y, _ptr(dx), _ptr(dw))
    if rc != 0:
        raise RuntimeError("reference rms_norm / apply_rope raised")
    out = dict(y=y)
    if dy is not None:
        out.update(dx=dx, dw=dw)
    return out


# ------------------------------------------------------------------ metrics
def max_rel(x, ref) -> float:
    """max_i |x_i - ref_i| / max_i |ref_i| (the tolerance measure of the build)."""
    x = np.asarray(x, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.max(np.abs(ref))
    num = np.max(np.abs(x - ref))
    return float(num / den) if den > 0 else float(num)


def rel_l2(x, ref) -> float:
    """||x - ref||_2 / ||ref||_2, the reference tests' rel_diff
    (optim/test_qkt_softmax_grad.cpp:11-24)."""
    x = np.asarray(x, np.float64)
    ref = np.asarray(ref, np.float64)
    nb = np.sum(ref * ref)
    nd = np.sum((x - ref) ** 2)
    return float(math.sqrt(nd / nb)) if nb > 0 else float(math.sqrt(nd))


# ------------------------------------------------------------- LoRA linear
def _lora_pack(slices, in_dim):
    """slices: dicts with A, B (fp32 arrays in their stored layout), scale, col0,
    a_transposed, b_transposed.  Returns (meta int64 [n, 5], scale, A_all, B_all)."""
    meta, sc, As, Bs = [], [], [], []
    for sl in slices:
        A, B = np.asarray(sl["A"], np.float32), np.asarray(sl["B"], np.float32)
        at, bt = bool(sl.get("a_transposed", False)), bool(sl.get("b_transposed", False))
        r = A.shape[0] if at else A.shape[1]
        cols = B.shape[0] if bt else B.shape[1]
        meta.append([r, int(sl.get("col0", 0)), cols, int(at), int(bt)])
        sc.append(float(sl["scale"]))
        As.append(A.ravel())
        Bs.append(B.ravel())
    meta = np.ascontiguousarray(np.array(meta, np.int64).reshape(-1, 5))
    cat = lambda xs: np.ascontiguousarray(np.concatenate(xs) if xs else np.zeros(1, np.float32), np.float32)
    return meta, np.ascontiguousarray(np.array(sc or [0.0], np.float32)), cat(As), cat(Bs)


def _lora_unpack(flat, slices, key):
    out, o = [], 0
    for sl in slices:
        n = np.asarray(sl[key]).size
        out.append(flat[o:o + n].reshape(np.asarray(sl[key]).shape))
        o += n
    return out


def _lora_prep(x, W, bias, slices, w_transposed, dy):
    x = np.ascontiguousarray(x, np.float32)
    W = np.ascontiguousarray(W, np.float32)
    N, in_dim = x.shape
    out = W.shape[0] if w_transposed else W.shape[1]
    meta, sc, A_all, B_all = _lora_pack(slices, in_dim)
    y = np.zeros((N, out), np.float32)
    dx = np.zeros_like(x) if dy is not None else None
    dA = np.full(A_all.shape, np.nan, np.float32)
    dB = np.full(B_all.shape, np.nan, np.float32)
    has = np.zeros(max(1, len(slices)), np.int32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    dyc = None if dy is None else np.ascontiguousarray(dy, np.float32)
    return x, W, N, in_dim, out, meta, sc, A_all, B_all, y, dx, dA, dB, has, b, dyc


def lora(x, W, bias=None, slices=(), w_transposed=False, dy=None, all_grads=False, w_bf16=False):
    """ops::LoRALinear forward (and, with dy, the Engine backward) on fp32 x
    [N, in]; W [in, out] (or [out, in] with w_transposed) as fp32 values,
    those of a bf16 weight with w_bf16.  Returns y, dx, grad_A / grad_B lists
    (None where the slice has no gradient)."""
    slices = list(slices)
    x, W, N, in_dim, out, meta, sc, A_all, B_all, y, dx, dA, dB, has, b, dyc = _lora_prep(
        x, W, bias, slices, w_transposed, dy)
    lib().orc_lora(x, W, _ptr(b), N, in_dim, out, int(bool(w_transposed)), int(bool(w_bf16)), len(slices), meta.ctypes.data, sc, A_all,
                   B_all, int(bool(all_grads)), _ptr(dyc), y, _ptr(dx), dA, dB, has.ctypes.data)
    return _lora_result(y, dx, dA, dB, has, slices, dy is not None)


def ref_lora(x, W, bias=None, slices=(), w_transposed=False, dy=None, w_bf16=False):
    """The real ops::LoRALinear (oracle/_ref), same arguments as lora()."""
    slices = list(slices)
    x, W, N, in_dim, out, meta, sc, A_all, B_all, y, dx, dA, dB, has, b, dyc = _lora_prep(
        x, W, bias, slices, w_transposed, dy)
    rc = ref().mftref_lora(x, W, _ptr(b), N, in_dim, out, int(bool(w_transposed)), int(bool(w_bf16)), len(slices),
                           meta.ctypes.data, sc, A_all, B_all, _ptr(dyc), y, _ptr(dx), dA, dB, has.ctypes.data)
    if rc != 0:
        raise RuntimeError("mftref_lora failed")
    return _lora_result(y, dx, dA, dB, has, slices, dy is not None)


def _lora_result(y, dx, dA, dB, has, slices, grad):
    res = dict(y=y, dx=dx, grad_A=[], grad_B=[])
    if grad:
        for i, (a, bb) in enumerate(zip(_lora_unpack(dA, slices, "A"), _lora_unpack(dB, slices, "B"))):
            res["grad_A"].append(a if has[i] else None)
            res["grad_B"].append(bb if has[i] else None)
    return res


def lora_merge(W, slices, w_bf16=False, sign=1.0):
    """apply_lora_delta_to_base of every slice on W [in, out] (values); returns the new W."""
    W = np.array(W, np.float32, copy=True)
    meta, sc, A_all, B_all = _lora_pack(list(slices), W.shape[0])
    lib().orc_lora_merge(W, int(bool(w_bf16)), W.shape[0], W.shape[1], len(slices), meta.ctypes.data, sc, A_all,
                         B_all, float(sign))
    return W


def ref_lora_merge(W, slices, w_bf16=False):
    """The real LoRALinear::merge_to_base (oracle/_ref) on W [in, out]."""
    W = np.array(W, np.float32, copy=True)
    meta, sc, A_all, B_all = _lora_pack(list(slices), W.shape[0])
    if ref().mftref_lora_merge(W, int(bool(w_bf16)), W.shape[0], W.shape[1], len(slices), meta.ctypes.data, sc,
                               A_all, B_all) != 0:
        raise RuntimeError("mftref_lora_merge failed")
    return W
