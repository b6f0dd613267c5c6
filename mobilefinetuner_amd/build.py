"""Build the gfx950 attention library in-tree.

    python -m mobilefinetuner_amd.build

compiles every source under ``csrc/`` with hipcc for gfx950 and links
``mobilefinetuner_amd/lib/libmft_attn.so`` (the C ABI of
``include/mft/attention.h``).  The library is built in the source tree so that
it travels with the repository snapshot to the GPU machine.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libmft_attn.so")
BUILD = os.path.join(PKG, "_build")

ARCH = os.environ.get("MFT_OFFLOAD_ARCH", "gfx950")
# Packed-fp32 VALU ops are disabled for all device code (the compiler would
# otherwise form v_pk_* fp32 instructions from scalar float code).
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libmft_attn.so)")


# Files whose MFMA accumulators should be allocated in VGPRs: their kernels
# keep all live state within 256 VGPRs, and the VGPR form avoids copying the
# loop-carried accumulators between AGPRs and VGPRs on every iteration.
VGPR_FORM = {"attn_fwd.hip", "attn_fwd_fast256.hip", "attn_bwd_fast64.hip"}


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC)
                  if f.endswith((".hip", ".cpp")))


def _stale(src: str, obj: str) -> bool:
    """The object is older than its source or any header of csrc/ and include/."""
    if not os.path.exists(obj):
        return True
    heads = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    inc = os.path.join(ROOT, "include", "mft")
    heads += [os.path.join(inc, f) for f in os.listdir(inc)]
    newest = max(os.path.getmtime(p) for p in heads + [src])
    return os.path.getmtime(obj) < newest


INCREMENTAL = False


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    if INCREMENTAL and not _stale(src, obj):
        return obj
    cmd = [hipcc(), *HIP_FLAGS, "-I", os.path.join(ROOT, "include"), "-I", CSRC, "-c", src, "-o", obj]
    if os.path.basename(src) in VGPR_FORM:
        cmd[1:1] = ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    noise = "is not a recognized feature for this target"
    out = "\n".join(l for l in res.stdout.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{out}")
    return obj


def build(verbose: bool = True) -> str:
    """Compile all sources and link the shared library; returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = sources()
    workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    # rocBLAS runs the plain GEMMs of the streaming LM cross-entropy.
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, "-L/opt/rocm/lib", "-lrocblas",
           "-Wl,-rpath,/opt/rocm/lib"]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"[mft build] {LIB} ({len(objs)} objects, arch {ARCH})")
    return LIB


if __name__ == "__main__":
    # --incremental: recompile only sources older than their object's inputs
    # (a development shortcut; build() with no flag compiles everything).
    INCREMENTAL = "--incremental" in sys.argv
    build()
    sys.exit(0)
