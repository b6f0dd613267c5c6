"""The closed-form work geometry of the fast kernels (attn_geometry.h: which
key tiles each query tile visits and which query blocks each key tile visits,
and where each tile's iterations start in the flattened order) against
brute-force enumeration of the tiles holding a visible (query, key) pair under
the causal mask and the causal sliding window (graph/gemma_model.cpp:272-285).
Host code only; no GPU."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_geometry_closed_forms_match_enumeration(tmp_path):
    exe = tmp_path / "geometry_check"
    subprocess.run(["/opt/rocm/bin/hipcc", "-x", "hip", "--offload-arch=gfx950", "--cuda-host-only", "-O1",
                    "-std=c++17", "-I", os.path.join(ROOT, "mobilefinetuner_amd", "csrc"),
                    os.path.join(ROOT, "tests", "native", "geometry_check.cpp"), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout.startswith("ok"), out.stdout + out.stderr
    assert int(out.stdout.split()[1]) > 600


def test_precomputed_offsets_match_swizzled_addressing(tmp_path):
    """TileDma (direct loads) and FwdLane (forward LDS reads) replace per-load
    swizzle arithmetic with loop-invariant per-lane offsets; they must address
    exactly the bytes tile_off / issue_tile_part address."""
    exe = tmp_path / "offsets_check"
    subprocess.run(["/opt/rocm/bin/hipcc", "-x", "hip", "--offload-arch=gfx950", "--cuda-host-only", "-O1",
                    "-std=c++17", "-I", os.path.join(ROOT, "include"),
                    "-I", os.path.join(ROOT, "mobilefinetuner_amd", "csrc"),
                    os.path.join(ROOT, "tests", "native", "offsets_check.cpp"), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout.startswith("ok 0"), out.stdout + out.stderr


def test_lora_coldot_grid_stays_within_launch_limits(tmp_path):
    """lora_coldot launches one grid row per chunk of rows: past ~8.4M rows the
    chunks grow so that grid.y stays within 65535 (the C ABI accepts N up to
    2^31 - 1)."""
    exe = tmp_path / "lora_grid_check"
    subprocess.run(["/opt/rocm/bin/hipcc", "-x", "hip", "--offload-arch=gfx950", "--cuda-host-only", "-O1",
                    "-std=c++17", "-I", os.path.join(ROOT, "mobilefinetuner_amd", "csrc"),
                    os.path.join(ROOT, "tests", "native", "lora_grid_check.cpp"), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout.startswith("ok"), out.stdout + out.stderr


def test_prologue_fast_division(tmp_path):
    """The prologue's 32-bit row addressing divides by H and S with a
    multiply and a shift (FastDiv); it must equal n / d for every n < 2^31."""
    exe = tmp_path / "fastdiv_check"
    subprocess.run(["/opt/rocm/bin/hipcc", "-x", "hip", "--offload-arch=gfx950", "--cuda-host-only", "-O1",
                    "-std=c++17", "-I", os.path.join(ROOT, "mobilefinetuner_amd", "csrc"),
                    os.path.join(ROOT, "tests", "native", "fastdiv_check.cpp"), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout.startswith("ok"), out.stdout + out.stderr
    assert int(out.stdout.split()[1]) > 10_000_000


def test_split_plans_stay_within_slot_limit(tmp_path):
    """The forward and backward split planners never give a tile more
    partial slots than the merge kernels hold (kSplitMaxSlots), over a sweep
    of shapes up to S = 2^20, GQA groups, windows and head dims."""
    lib = os.path.join(ROOT, "mobilefinetuner_amd", "lib")
    if not os.path.exists(os.path.join(lib, "libmft_attn.so")):
        import pytest
        pytest.skip("libmft_attn.so not built")
    exe = tmp_path / "plan_check"
    subprocess.run(["/opt/rocm/bin/hipcc", "-x", "hip", "--offload-arch=gfx950", "--cuda-host-only", "-O1",
                    "-std=c++17", "-I", os.path.join(ROOT, "include"),
                    "-I", os.path.join(ROOT, "mobilefinetuner_amd", "csrc"),
                    os.path.join(ROOT, "tests", "native", "plan_check.cpp"), "-o", str(exe),
                    "-L", lib, "-lmft_attn", f"-Wl,-rpath,{lib}"],
                   check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, env={**os.environ, "HIP_VISIBLE_DEVICES": ""})
    assert out.returncode == 0 and out.stdout.startswith("ok"), out.stdout + out.stderr


def _mfma_overlaps(asm_text):
    """MFMAs whose result registers overlap their A or B operand registers."""
    import re

    def rng(t):
        m = re.match(r"([va])\[(\d+):(\d+)\]", t) or re.match(r"([va])(\d+)()$", t)
        if not m:
            return None
        lo = int(m.group(2))
        return m.group(1), lo, int(m.group(3)) if m.group(3) else lo

    bad = []
    for line in asm_text.splitlines():
        m = re.match(r"\s+v_mfma\S*\s+(\S+),\s*(\S+),\s*(\S+),\s*(\S+)", line)
        if not m:
            continue
        d = rng(m.group(1))
        for src in (rng(m.group(2)), rng(m.group(3))):
            if d and src and d[0] == src[0] and not (src[2] < d[1] or src[1] > d[2]):
                bad.append(line.strip())
    return bad


def test_no_mfma_result_overlaps_its_operands(tmp_path):
    """The compiler (ROCm 7.2) may give an MFMA with a literal-zero
    accumulator result registers that overlap its A/B operands, which gave
    NaN gradients on gfx950; the kernels start every chain with the
    early-clobber form instead.  Compile the attention translation units and
    the fused LM cross-entropy GEMM to assembly, with the build's flags, and
    check that no MFMA does this."""
    import concurrent.futures as cf
    import sys
    sys.path.insert(0, ROOT)
    from mobilefinetuner_amd import build as B
    units = sorted(f for f in os.listdir(B.CSRC)
                   if (f.startswith("attn_") or f == "lm_loss_fused.hip") and f.endswith(".hip"))

    def asm(name):
        out = tmp_path / (name + ".s")
        cmd = [B.hipcc(), *B.HIP_FLAGS, "-I", os.path.join(ROOT, "include"), "-I", B.CSRC, "--cuda-device-only",
               "-S", os.path.join(B.CSRC, name), "-o", str(out)]
        if name in B.VGPR_FORM:
            cmd[1:1] = ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
        subprocess.run(cmd, check=True, capture_output=True, text=True)
        return out.read_text()

    with cf.ThreadPoolExecutor(len(units)) as ex:
        texts = list(ex.map(asm, units))
    bad = [b for t in texts for b in _mfma_overlaps(t)]
    assert sum(t.count("v_mfma") for t in texts) > 1000
    assert not bad, bad[:5]
