"""The C-ABI library without a GPU: it loads, exports every entry point that
include/mft/attention.h declares, and rejects bad requests the way the
reference rejects bad operator inputs (core/memory_efficient_attention.cpp:85-103)
before any device work is enqueued."""
import ctypes as C
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mft", "attention.h")
HEADERS = [HEADER] + [os.path.join(ROOT, "include", "mft", h) for h in ("prologue.h", "lm_loss.h", "lora.h")]


@pytest.fixture(scope="module")
def capi():
    from mobilefinetuner_amd import capi as M
    if not os.path.exists(M.LIB_PATH):
        from mobilefinetuner_amd import build
        build.build(verbose=False)
    M.lib()
    return M


def header_functions():
    text = "".join(open(h).read() for h in HEADERS)
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(mft_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    fns = header_functions()
    for f in ("mft_attn_workspace_size", "mft_attn_fwd", "mft_attn_bwd", "mft_repeat_kv_fwd",
              "mft_repeat_kv_bwd", "mft_last_error"):
        assert f in fns


def test_every_header_symbol_is_exported(capi):
    fns = header_functions()
    assert sorted(capi.EXPORTS) == fns
    out = subprocess.run(["nm", "-D", "--defined-only", capi.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [f for f in fns if f not in exported]
    assert not missing, missing
    L = capi.lib()
    for f in fns:
        assert hasattr(L, f)


def test_header_compiles_as_c(tmp_path):
    """The header is plain C (extern "C", C99 types, no torch types)."""
    src = tmp_path / "t.c"
    src.write_text('#include "mft/attention.h"\n#include "mft/prologue.h"\n#include "mft/lm_loss.h"\n'
                   'int main(void){return mft_version()==7?0:1;}\n')
    res = subprocess.run(["gcc", "-std=c99", "-fsyntax-only", "-D__HIP_PLATFORM_AMD__",
                          "-I", os.path.join(ROOT, "include"), "-I", "/opt/rocm/include", str(src)],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr


def test_version(capi):
    assert capi.lib().mft_version() == 7


def _err(capi, fn):
    with pytest.raises(capi.MftError) as e:
        fn()
    return e.value


@pytest.mark.parametrize("kw,status,needle", [
    (dict(B=0), 1, "positive"),
    (dict(Hq=6, Hkv=4), 1, "multiple of kv heads"),
    (dict(D=320), 2, "head_dim > 256"),
    (dict(dtype=1), 1, "dtype"),
    (dict(scale=float("nan")), 1, "scale"),
    (dict(window=-1), 1, "window"),
    (dict(window=16, causal=False), 1, "causal"),
    (dict(kv_len=2), 1, "aligned"),
])
def test_desc_validation(capi, kw, status, needle):
    args = dict(B=1, Hq=4, Hkv=1, S=64, D=64, scale=-1.0, causal=True, dtype=capi.MFT_BF16)
    args.update(kw)
    e = _err(capi, lambda: capi.workspace_size(capi.desc(**args)))
    assert e.status == status and needle in str(e)


def test_null_pointers_rejected_before_launch(capi):
    d = capi.desc(1, 4, 1, 64, 64)
    e = _err(capi, lambda: capi.attn_fwd(d, None, None, None, None, None, None, None))
    assert e.status == capi.MFT_ERR_INVALID_ARG
    e = _err(capi, lambda: capi.attn_bwd(d, 1, 1, 1, 1, 1, 1, 1, 1, 1, None, None))
    assert e.status == capi.MFT_ERR_INVALID_ARG and "workspace" in str(e)
    e = _err(capi, lambda: capi.attn_bwd_stage(d, 16, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, None))
    assert "stages" in str(e)
    e = _err(capi, lambda: capi.attn_fwd(d, 16, 32, 48, 8, None, None, None))
    assert e.status == capi.MFT_ERR_INVALID_ARG and "aligned" in str(e)
    e = _err(capi, lambda: capi.attn_bwd(d, 16, 16, 16, 16, 16, 16, 16, 16, 20, 16, None))
    assert "aligned" in str(e)
    e = _err(capi, lambda: capi.repeat_kv_fwd(None, None, 1, 1, 1, 1, 1, capi.MFT_F32, None))
    assert e.status == capi.MFT_ERR_INVALID_ARG
    e = _err(capi, lambda: capi.repeat_kv_bwd(1, 1, 1, 1, 1, 1, 0, None))
    assert e.status == capi.MFT_ERR_INVALID_ARG


def test_last_error_is_thread_local(capi):
    import threading
    _err(capi, lambda: capi.workspace_size(capi.desc(1, 3, 2, 8, 8)))
    seen = []
    t = threading.Thread(target=lambda: seen.append(capi.lib().mft_last_error()))
    t.start()
    t.join()
    assert seen == [b""]
    assert b"multiple" in capi.lib().mft_last_error()


def test_workspace_is_aligned_and_subquadratic(capi):
    """The backward workspace holds per-row statistics (O(S)) and fp32
    partial tiles of split work units (bounded by the unit count): it never
    grows like the S x S score matrices the reference keeps."""
    sizes = []
    for S in (1024, 4096, 16384):
        f, b = capi.workspace_size(capi.desc(1, 4, 1, S, 256, 1 / 16, True, capi.MFT_BF16))
        assert b % 256 == 0 and b > 0
        sizes.append(b)
        assert b < 4 * 4 * S * S * 4 or S <= 1024  # reference holds four S x S fp32 tensors per head
    assert sizes[2] < 16 * sizes[1]  # 4x longer sequence, far less than 16x the bytes


def test_window_and_padding_workspace(capi):
    """A window shrinks the backward's split-tile partials (fewer iterations
    per tile); key lengths add the per-row scratch of the rows that see no
    key (two fp32/int32 values per query row); a window >= S is no window."""
    base = capi.workspace_size(capi.desc(1, 4, 1, 4096, 256, 1 / 16, True, capi.MFT_BF16))
    same = capi.workspace_size(capi.desc(1, 4, 1, 4096, 256, 1 / 16, True, capi.MFT_BF16, window=4096))
    assert same == base
    win = capi.workspace_size(capi.desc(1, 4, 1, 4096, 256, 1 / 16, True, capi.MFT_BF16, window=512))
    assert win[1] > 0
    pad = capi.workspace_size(capi.desc(1, 4, 1, 4096, 256, 1 / 16, True, capi.MFT_BF16, kv_len=1 << 20))
    assert pad[1] == base[1] + 2 * 4 * 4 * 4096 and pad[0] == base[0]


@pytest.mark.parametrize("strides,needle", [
    ({"q": (4096 * 64, 64, 64 * 4 + 4)}, "multiples of 16 bytes"),   # sequence stride 260 bf16 = 520 B
    ({"k": (1, 0, 0)}, "multiples of 16 bytes"),
    ({"dq": (4096 * 64, 64, 32)}, "shorter than a row"),
])
def test_stride_validation(capi, strides, needle):
    """Operand layouts: every stride a positive multiple of 16 bytes, and a
    sequence stride of at least one row; all-zero means contiguous."""
    d = capi.desc(1, 4, 1, 4096, 64, 0.125, True, capi.MFT_BF16, strides=strides)
    e = _err(capi, lambda: capi.workspace_size(d))
    assert e.status == capi.MFT_ERR_INVALID_ARG and needle in str(e)


def test_strided_layout_accepted(capi):
    """[B,S,H,D] storage passed as [B,H,S,D] views (b = S*H*D, h = D, s = H*D)."""
    B, H, S, D = 2, 4, 256, 64
    st = (S * H * D, D, H * D)
    d = capi.desc(B, H, 1, S, D, 0.125, True, capi.MFT_BF16,
                  strides={n: st for n in ("q", "o", "dO")} | {"dq": st})
    f, b = capi.workspace_size(d)
    assert b == capi.workspace_size(capi.desc(B, H, 1, S, D, 0.125, True, capi.MFT_BF16))[1]


@pytest.mark.parametrize("kw,status,needle", [
    (dict(D=7), 1, "even head_dim"),
    (dict(D=514), 2, "head_dim > 512"),
    (dict(S=0), 1, "4D tensor"),
    (dict(dtype=5), 1, "dtype"),
    (dict(norm=3), 1, "norm must be"),
    (dict(eps=-1.0), 1, "eps"),
    (dict(theta=float("nan")), 1, "theta"),
])
def test_prologue_desc_validation(capi, kw, status, needle):
    args = dict(B=1, H=2, S=8, D=64, dtype=capi.MFT_BF16, norm=capi.MFT_NORM_GEMMA, eps=1e-6, theta=1e4)
    args.update(kw)
    d = capi.prologue_desc(**args)
    with pytest.raises(capi.MftError) as e:
        capi.prologue_fwd(d, 16, 16, 16, None)
    assert e.value.status == status and needle in str(e.value)


def test_prologue_pointer_rules(capi):
    d = capi.prologue_desc(1, 2, 8, 64)
    for call, needle in ((lambda: capi.prologue_fwd(d, None, 16, 16, None), "non-NULL"),
                         (lambda: capi.prologue_fwd(d, 16, None, 16, None), "weight"),
                         (lambda: capi.prologue_fwd(d, 17, 16, 16, None), "element-aligned"),
                         (lambda: capi.prologue_bwd(d, 16, 16, 32, 32, None, None, None), "alias"),
                         (lambda: capi.prologue_bwd(d, 16, 16, 32, 48, 64, None, None), "workspace")):
        with pytest.raises(capi.MftError) as e:
            call()
        assert needle in str(e.value)
    bad = capi.prologue_desc(1, 2, 8, 64, strides=dict(x=(1024, 64, 100)))
    with pytest.raises(capi.MftError) as e:
        capi.prologue_fwd(bad, 16, 16, 16, None)
    assert "multiples of 16 bytes" in str(e.value)
    # workspace: [waves, D] fp32 partials, sized by the shape alone
    assert capi.prologue_workspace_size(capi.prologue_desc(1, 4, 4096, 256)) == 16384 // 16 * 4 * 256
    assert capi.prologue_workspace_size(capi.prologue_desc(1, 4, 4096, 256, norm=capi.MFT_NORM_NONE)) == 0


def test_lm_loss_validation(capi):
    for kw, needle in ((dict(B=0), "[B,S,V]"), (dict(dtype=7), "dtype"), (dict(reduction=5), "reduction"),
                       (dict(H=3, reduction=2), "only mean and sum"), (dict(chunk=-1), "chunk")):
        args = dict(B=1, S=4, V=5)
        args.update(kw)
        with pytest.raises(capi.MftError) as e:
            capi.lm_ce_workspace_size(capi.lm_loss_desc(**args))
        assert needle in str(e.value), (kw, str(e.value))
    d = capi.lm_loss_desc(1, 4, 5)
    with pytest.raises(capi.MftError) as e:
        capi.lm_ce_fwd(d, None, 16, 16, 16, None, 16, None)
    assert "non-NULL" in str(e.value)
    # streaming workspace, fp32: one fp32 logits chunk and one G chunk plus the GEMM workspace
    f, b = capi.lm_ce_workspace_size(capi.lm_loss_desc(1, 4096, 262144, 1152, capi.MFT_F32))
    assert f == b and 4096 * 16384 * 8 < f < 4096 * 16384 * 8 + (80 << 20)
    # bf16 with H a multiple of 64 (fused kernels): no logits chunk, one bf16 G chunk
    f, b = capi.lm_ce_workspace_size(capi.lm_loss_desc(1, 4096, 262144, 1152, capi.MFT_BF16))
    assert f == b and 4096 * 16384 * 2 < f < 4096 * 16384 * 2 + (80 << 20)



def test_lora_validation(capi):
    A = dict(A=16, B=16, scale=0.5, rank=4, cols=32)
    for kw, slices, needle in ((dict(N=0), [A], "positive sizes"), (dict(w_dtype=1), [A], "w_dtype"),
                               ({}, [dict(A, col0=8)], "exceeds base weight width"),
                               ({}, [dict(A, A=None)], "must not be null"), ({}, [dict(A, rank=0)], "rank")):
        args = dict(N=8, in_dim=16, out_dim=32, w_dtype=capi.MFT_F32, slices=slices)
        args.update(kw)
        with pytest.raises(capi.MftError) as e:
            capi.lora_workspace_size(capi.lora_desc(**args))
        assert needle in str(e.value), (kw, str(e.value))
    d = capi.lora_desc(8, 16, 32, capi.MFT_BF16, slices=[A])
    with pytest.raises(capi.MftError) as e:
        capi.lora_fwd(d, None, 16, None, 16, None, 16, None)
    assert "non-NULL" in str(e.value)
    with pytest.raises(capi.MftError) as e:
        capi.lora_bwd(d, 16, 16, 16, None, None, 16, None)
    assert "non-NULL" in str(e.value)
    # workspace: bf16 staging of x (forward) / dy (backward), x . A or g [N, R] fp32, the GEMM workspace
    f, b = capi.lora_workspace_size(capi.lora_desc(4096, 1152, 1024, capi.MFT_BF16, slices=[dict(A, rank=16)]))
    # plus a k-major copy of the largest rank-r operand ([max(in, cols), r] fp32)
    pack = 1152 * 16 * 4
    assert f == 4096 * 1152 * 2 + 4096 * 16 * 4 + pack + (32 << 20)
    # backward adds the per-row-chunk partials of grad_A / grad_B ([chunks, max(in, cols), r] fp32;
    # 16-row chunks here: 5 x 256 column waves)
    assert b == 4096 * 1024 * 2 + 4096 * 16 * 4 + 4096 // 16 * 1152 * 16 * 4 + pack + (32 << 20)
