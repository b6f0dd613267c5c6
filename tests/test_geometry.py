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
