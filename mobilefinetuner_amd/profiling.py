"""Summaries of rocprofv3 output for the attention kernels.

    python -m mobilefinetuner_amd.profiling stats <dir> [--command "..."] [--only attn_,prologue_]
    python -m mobilefinetuner_amd.profiling traffic <fetch_dir> <write_dir> --config c5 \
        --copy-bytes N [--out profiles/hbm_traffic_c5.json] [--command "..."]
    python -m mobilefinetuner_amd.profiling counters <dir> [--command "..."]

``stats`` prints the per-kernel table of a ``rocprofv3 --kernel-trace --stats
--output-format csv`` run.  ``traffic`` reads two ``--pmc`` runs (FETCH_SIZE,
then WRITE_SIZE, both in KiB per dispatch) of ``bench.py --copy-calibration``
and converts them to HBM bytes per launch of each attention kernel.  Each
counter is scaled by bytes/counter measured on the calibration copy (an
elementwise kernel reading N bytes and writing N bytes), so the figures do not
depend on what unit the counter reports in.
"""
from __future__ import annotations

import argparse
import collections
import csv
import glob
import json
import os
import sys

# Kernel-name fragments -> short names used in bench.py's roofline object.
KERNELS = {
    "attn_fwd_masked_rows": "attn_fwd_masked_rows",
    "attn_bwd_masked_dq": "attn_bwd_masked_dq",
    "attn_bwd_masked_dkdv": "attn_bwd_masked_dkdv",
    "attn_fwd_combine": "attn_fwd_combine",
    "attn_fwd": "attn_fwd",
    "attn_bwd_main": "attn_bwd_main",
    "attn_bwd_dkdv": "attn_bwd_dkdv",
    "attn_bwd_dq": "attn_bwd_dq",
    "attn_bwd_stats": "attn_bwd_stats",
    "attn_bwd_fast_reduce": "attn_bwd_reduce",
    "attn_bwd_reduce": "attn_bwd_reduce",
    "prologue_fwd_vec": "prologue_fwd_vec",
    "prologue_bwd_vec": "prologue_bwd_vec",
    "prologue_fwd_kernel": "prologue_fwd",
    "prologue_bwd_kernel": "prologue_bwd",
    "prologue_dw_reduce": "prologue_dw_reduce",
    "ce_fused_kernel<true, 1>": "ce_fused_grad",
    "ce_fused_kernel<false, 1>": "ce_fused_grad",
    "ce_fused_kernelILb1ELi1E": "ce_fused_grad",
    "ce_fused_kernelILb0ELi1E": "ce_fused_grad",
    "ce_fused_kernel<true, 2>": "lora_fused_fwd",
    "ce_fused_kernel<false, 2>": "lora_fused_fwd",
    "ce_fused_kernelILb1ELi2E": "lora_fused_fwd",
    "ce_fused_kernelILb0ELi2E": "lora_fused_fwd",
    "ce_fused_kernel": "ce_fused_fwd",
    "ce_fused_merge": "ce_fused_merge",
    "ce_row_stats": "ce_row_stats",
    "ce_grad": "ce_grad",
    "ce_finalize": "ce_finalize",
    "ce_reduce": "ce_reduce",
    "lora_round_bf16": "lora_round_bf16",
    "lora_fill_bias": "lora_fill_bias",
    "lora_rowdot": "lora_rowdot",
    "lora_coldot_reduce": "lora_coldot_reduce",
    "lora_coldot_kernel": "lora_coldot",
    "lora_merge": "lora_merge",
    "Cijk_": "rocblas_gemm",
}
COPY_TAG = "MulFunctor"  # torch.mul(x, 1.0, out=y): the calibration copy


def short_name(full: str) -> str:
    for frag, short in KERNELS.items():
        if frag in full:
            if short == "rocblas_gemm":  # keep the Tensile tile name: the GEMMs differ
                if "_UserArgs_" in full:
                    return "rocblas_" + full.split("_UserArgs_")[-1][:24]
                mt = full.find("_MT")
                return "rocblas_f32_" + full[mt + 1:].split("_")[0] if mt >= 0 else short
            return short
    if COPY_TAG in full:
        return "copy_calibration"
    return full.split("(")[0][:60]


def _csvs(d: str, suffix: str):
    return sorted(glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True))


def kernel_stats(d: str):
    rows = []
    for f in _csvs(d, "kernel_stats.csv"):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                rows.append(r)
    return rows


def pmc_per_kernel(d: str, counter: str):
    """Mean counter value per dispatch, by short kernel name.  Of the torch
    multiply dispatches only the largest grid (the calibration copy) is kept:
    bench.py also scales dO with a small multiply."""
    acc = collections.defaultdict(list)
    for f in _csvs(d, "counter_collection.csv"):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                if r.get("Counter_Name") != counter:
                    continue
                acc[(short_name(r["Kernel_Name"]), int(r["Grid_Size"]))].append(float(r["Counter_Value"]))
    out = {}
    for (k, grid), v in sorted(acc.items(), key=lambda kv: kv[0][1]):
        out[k] = (sum(v) / len(v), len(v))  # largest grid last, so it wins for the copy
    return out


def cmd_stats(args):
    rows = kernel_stats(args.dir)
    if not rows:
        sys.exit(f"no *kernel_stats.csv under {args.dir}")
    if args.command:
        print(f"command: {args.command}\n")
    if args.only:
        keep = tuple(args.only.split(","))
        rows = [r for r in rows if short_name(r["Name"]).startswith(keep)]
    print(f"{'kernel':40s} {'calls':>6s} {'avg_us':>10s} {'min_us':>10s} {'max_us':>10s} {'pct':>6s}")
    for r in rows:
        print(f"{short_name(r['Name']):40s} {int(r['Calls']):6d} {float(r['AverageNs']) / 1e3:10.2f} "
              f"{float(r['MinNs']) / 1e3:10.2f} {float(r['MaxNs']) / 1e3:10.2f} {float(r['Percentage']):6.2f}")


def cmd_counters(args):
    """Mean SQ/GRBM counters per dispatch of each attention kernel, with the
    MFMA-busy fraction SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE/XCDs *
    CUs * 4 SIMDs) (GRBM_GUI_ACTIVE is summed over the XCDs)."""
    acc = collections.defaultdict(lambda: collections.defaultdict(list))
    for f in _csvs(args.dir, "counter_collection.csv"):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                acc[short_name(r["Kernel_Name"])][r["Counter_Name"]].append(float(r["Counter_Value"]))
    if args.command:
        print(f"command: {args.command}\n")
    for k in sorted(acc):
        if not k.startswith("attn"):
            continue
        m = {c: sum(v) / len(v) for c, v in acc[k].items()}
        print(k)
        for c in sorted(m):
            print(f"    {c:28s} {m[c]:16.1f}")
        if "SQ_VALU_MFMA_BUSY_CYCLES" in m and "GRBM_GUI_ACTIVE" in m:
            busy = m["SQ_VALU_MFMA_BUSY_CYCLES"] / (m["GRBM_GUI_ACTIVE"] / args.xcds * args.cus * 4)
            print(f"    {'=> MFMA busy fraction':28s} {busy:16.4f}")
        if "SQ_WAVES" in m and m["SQ_WAVES"]:
            for c in ("SQ_INSTS_MFMA", "SQ_INSTS_VALU", "SQ_INSTS_LDS"):
                if c in m:
                    print(f"    {'=> ' + c + ' per wave':28s} {m[c] / m['SQ_WAVES']:16.1f}")


def cmd_traffic(args):
    fetch = pmc_per_kernel(args.fetch_dir, "FETCH_SIZE")
    write = pmc_per_kernel(args.write_dir, "WRITE_SIZE")
    if "copy_calibration" not in fetch or "copy_calibration" not in write:
        sys.exit("calibration copy kernel not found in the pmc runs")
    f_scale = args.copy_bytes / fetch["copy_calibration"][0]
    w_scale = args.copy_bytes / write["copy_calibration"][0]
    out = {"config": args.config, "copy_bytes": args.copy_bytes,
           "bytes_per_fetch_unit": f_scale, "bytes_per_write_unit": w_scale,
           "command": args.command, "kernels": {}}
    for k in sorted(set(fetch) & set(write)):
        if k == "copy_calibration":
            continue
        fb, wb = fetch[k][0] * f_scale, write[k][0] * w_scale
        out["kernels"][k] = {"fetch_bytes": round(fb), "write_bytes": round(wb), "hbm_bytes": round(fb + wb),
                             "dispatches": fetch[k][1]}
    text = json.dumps(out, indent=1)
    print(text)
    if args.out:
        with open(args.out, "w") as fh:
            fh.write(text + "\n")


def main():
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    a = sub.add_parser("stats")
    a.add_argument("dir")
    a.add_argument("--command", default="")
    a.add_argument("--only", default="", help="comma-separated short-name prefixes to keep")
    b = sub.add_parser("traffic")
    b.add_argument("fetch_dir")
    b.add_argument("write_dir")
    b.add_argument("--config", required=True)
    b.add_argument("--copy-bytes", type=int, required=True)
    b.add_argument("--out")
    b.add_argument("--command", default="")
    c = sub.add_parser("counters")
    c.add_argument("dir")
    c.add_argument("--cus", type=int, default=256)
    c.add_argument("--xcds", type=int, default=8)
    c.add_argument("--command", default="")
    args = ap.parse_args()
    {"stats": cmd_stats, "traffic": cmd_traffic, "counters": cmd_counters}[args.cmd](args)


if __name__ == "__main__":
    main()
