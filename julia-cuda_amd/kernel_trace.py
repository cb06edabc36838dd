"""rocprofv3 dispatch durations of bench.py's own timed kernel runs: pairs the kernel trace of a
profiled bench.py run (`rocprofv3 --kernel-trace -f csv`) with the ordered run list bench.py
writes with --trace-labels, so that each of bench.py's HIP-event figures has the profiler's
duration of exactly the same launches beside it.

    rocprofv3 --kernel-trace --stats -f csv -d OUT/bk -o bk -- \\
        python3 bench.py --section kernels,fused_gemm --path per-step --trace-labels OUT/labels.json
    python julia-cuda_amd/kernel_trace.py OUT/bk OUT/labels.json --out profiles/bench_kernels_rocprof.json

A label's run is the next stretch of consecutive dispatches of its kernel (name containing the
label's instance) at least warm-up + timed long; its timed launches are the last `timed` of the
stretch. Prints a table (label, kernel, launches, average / median / min / max us) and writes
{"runs": {label: {...}}} for bench.py.
"""

import argparse
import csv
import glob
import json
import os
import statistics


def dispatches(path):
    files = [path] if os.path.isfile(path) else sorted(
        glob.glob(os.path.join(path, "**", "*kernel_trace.csv"), recursive=True))
    if not files:
        raise SystemExit(f"no kernel_trace CSV under {path}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            rows.extend(csv.DictReader(fh))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    return [(r["Kernel_Name"], (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3) for r in rows]


def stretches(ds):
    """[(name, [durations])] of consecutive dispatches of one kernel."""
    out = []
    for name, us in ds:
        if out and out[-1][0] == name:
            out[-1][1].append(us)
        else:
            out.append((name, [us]))
    return out


def pair(ds, labels):
    runs, at = {}, 0
    st = stretches(ds)
    for lab in labels:
        need = lab["warmup"] + lab["timed"]
        while at < len(st) and not (lab["kernel"] in st[at][0] and len(st[at][1]) >= need):
            at += 1
        if at == len(st):
            raise SystemExit(f"no run of {lab['kernel']} ({need} launches) for {lab['label']}")
        us = st[at][1][-lab["timed"]:]
        runs[lab["label"]] = {"kernel": lab["kernel"], "name": st[at][0], "launches": len(us),
                              "avg_us": round(statistics.mean(us), 3),
                              "median_us": round(statistics.median(us), 3),
                              "min_us": round(min(us), 3), "max_us": round(max(us), 3)}
        at += 1
    return runs


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("trace", help="rocprofv3 output directory or kernel_trace CSV")
    ap.add_argument("labels", help="bench.py --trace-labels output")
    ap.add_argument("--out")
    args = ap.parse_args()
    with open(args.labels) as fh:
        labels = json.load(fh)
    runs = pair(dispatches(args.trace), labels)
    print("| run | kernel | launches | avg us | median us | min us | max us |")
    print("|---|---|---:|---:|---:|---:|---:|")
    for k, r in runs.items():
        print(f"| {k} | `{r['name']}` | {r['launches']} | {r['avg_us']} | {r['median_us']} | "
              f"{r['min_us']} | {r['max_us']} |")
    if args.out:
        with open(args.out, "w") as fh:
            json.dump({"runs": runs}, fh, indent=1)
            fh.write("\n")


if __name__ == "__main__":
    main()
