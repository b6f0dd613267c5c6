"""The drop-in: the reference's finetune_ops core with
core/memory_efficient_attention.cpp replaced by
mobilefinetuner_amd/adapter/memory_efficient_attention_hip.cpp (built by
mobilefinetuner_amd/adapter/Makefile from the reference sources, in the build
container).  On the GPU:

  * the reference's OWN unit test core/test_memory_efficient_attention_grad.cpp,
    compiled unchanged against the drop-in, passes;
  * test_fused_attention_dropin.cpp compares the fused operator (GQA, bf16,
    no-grad path, error convention) with the reference composite through the
    unchanged ops / autograd API;
  * with nn/lora_linear.cpp replaced by lora_linear_hip.cpp, the reference's
    OWN nn/test_lora_linear.cpp (merge, unmerge, clear) passes unchanged, and
    test_lora_dropin.cpp compares forward and Engine backward with the graph
    of the reference's operators;
  * with core/lm_loss.cpp replaced by lm_loss_hip.cpp, the reference's OWN
    core/test_selected_token_lm_loss.cpp (dense vs selected vs streaming,
    all-ignored NaN, out-of-range label) passes unchanged, and
    test_lm_loss_dropin.cpp checks every reduction and both weight dtypes
    against the reference formulas on a multi-chunk vocabulary.
"""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
OUT = os.path.join(ROOT, "mobilefinetuner_amd", "adapter", "_dropin")


def _run(name):
    exe = os.path.join(OUT, name)
    if not os.path.exists(exe):
        pytest.skip(f"{exe} not built (needs the reference checkout at build time)")
    print(f"[dropin] running {name}", flush=True)
    res = subprocess.run([exe], capture_output=True, text=True, timeout=100)
    print(res.stdout[-4000:], res.stderr[-2000:], flush=True)
    return res


def test_reference_unit_test_passes_on_dropin(dev):
    res = _run("test_memory_efficient_attention_grad")
    assert res.returncode == 0 and "[PASS]" in res.stdout


def test_fused_attention_dropin_parity(dev):
    res = _run("test_fused_attention_dropin")
    assert res.returncode == 0 and "[PASS]" in res.stdout


def test_reference_lora_unit_test_passes_on_dropin(dev):
    res = _run("test_lora_linear")
    assert res.returncode == 0, res.stdout + res.stderr


def test_lora_dropin_parity(dev):
    res = _run("test_lora_dropin")
    assert res.returncode == 0 and "[PASS]" in res.stdout


def test_reference_lm_loss_unit_test_passes_on_dropin(dev):
    res = _run("test_selected_token_lm_loss")
    assert res.returncode == 0 and "[PASS]" in res.stdout


def test_lm_loss_dropin_parity(dev):
    res = _run("test_lm_loss_dropin")
    assert res.returncode == 0 and "[PASS]" in res.stdout
