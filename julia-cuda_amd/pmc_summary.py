"""Per-kernel summary of rocprofv3 counter runs (--pmc, CSV output): for each kernel name
substring, the median over its dispatches of every counter the runs collected (a counter's
instances within one dispatch summed, as rocprofv3 reports them).

    rocprofv3 --pmc MfmaUtil MfmaFlopsF16 SQ_BUSY_CYCLES -f csv -d OUT/mfma -o pmc -- \\
        python3 julia-cuda_amd/kernel_bench.py --step qkv --tokens 18752 --spec ...
    python julia-cuda_amd/pmc_summary.py OUT/mfma --kernel "gemm_big<256, 20>" --kernel gemm_lat1

Prints one JSON object: {kernel: {"dispatches": n, counter: median, ...}}. With --duration-us
KERNEL=US (the kernel's average duration from a --kernel-trace --stats run), MfmaFlopsF16 is
also given as TFLOP/s over that duration.
"""

import argparse
import csv
import glob
import json
import os
import statistics


def counter_rows(path):
    files = [path] if os.path.isfile(path) else sorted(
        glob.glob(os.path.join(path, "**", "*counter_collection*.csv"), recursive=True))
    if not files:
        raise SystemExit(f"no counter_collection CSV under {path}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def summarize(rows, name_part):
    by = {}
    for r in rows:
        if name_part not in r.get("Kernel_Name", ""):
            continue
        key = r.get("Dispatch_Id") or r.get("Correlation_Id")
        c = by.setdefault(r["Counter_Name"], {})
        c[key] = c.get(key, 0.0) + float(r["Counter_Value"])
    if not by:
        raise SystemExit(f"no counter values for kernels matching {name_part!r}")
    out = {"dispatches": max(len(v) for v in by.values())}
    for name, per in sorted(by.items()):
        out[name] = statistics.median(per.values())
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("dirs", nargs="+", help="rocprofv3 output directories or CSV files")
    ap.add_argument("--kernel", action="append", required=True,
                    help="substring of a kernel's name (repeatable)")
    ap.add_argument("--duration-us", action="append", default=[],
                    help="KERNEL=US: the kernel's average duration, for TFLOP/s")
    args = ap.parse_args()
    rows = []
    for d in args.dirs:
        rows.extend(counter_rows(d))
    dur = dict(x.split("=", 1) for x in args.duration_us)
    out = {}
    for k in args.kernel:
        s = summarize(rows, k)
        if k in dur and "MfmaFlopsF16" in s:
            s["MfmaF16_TFLOPs"] = round(s["MfmaFlopsF16"] / (float(dur[k]) * 1e-6) / 1e12, 1)
        out[k] = s
    print(json.dumps(out, indent=1))


if __name__ == "__main__":
    main()
